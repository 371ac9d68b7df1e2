"""The reference operator mirrors on the reference's own device layout, through
the C ABI: moe_router_topk -> moe_experts_masked_int4 / the grouped INT4 pair
/ the BF16 pair / moe_gemm_int4 (include/uocr/cuda_ops.h:125-239).

Routing and tables come from the GPU router mirror (bit-exact with the
oracle); expert outputs are checked against the CPU oracle within rel_l2 <=
5e-3 and max-abs <= 2e-2 (the f32 atomics of the down scatter-add leave the
order of the per-token sums open, as in the reference).
"""
import numpy as np
import pytest

from helpers import MAX_ABS_TOL, REL_L2_TOL, awq_layer, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def _route(L, x, dev):
    import torch
    import oracle as O
    from uocr_hip import ops
    seq, E, k = x.shape[0], L.n_experts, L.top_k
    logits = O.matmul_t_bf16(x, L.router_bf16)  # the reference's router GEMV (pinned)
    ids = torch.empty(seq, k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, k, dtype=torch.float32, device=dev)
    at = torch.full((E, seq), -1, dtype=torch.int32, device=dev)
    aw = torch.zeros(E, seq, dtype=torch.float32, device=dev)
    cnt = torch.empty(E, dtype=torch.int32, device=dev)
    ops.moe_router_topk(torch.from_numpy(logits).to(dev), k, False, 1.0, False, ids, w, at, aw, cnt, seq)
    torch.cuda.synchronize()
    ids_o, w_o = O.moe_gate(x, L.router_bf16, k)
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), w_o.view(np.uint32))
    return at, aw, cnt, ids_o, w_o


def _check(got, want, label):
    r, m = rel_l2(got, want), max_abs(got, want)
    print(f"[mirror] {label}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    assert np.isfinite(got).all() and r <= REL_L2_TOL and m <= MAX_ABS_TOL, label


@pytest.mark.parametrize("seq", [16, 300])
@pytest.mark.parametrize("quant", ["awq", "sym"])
def test_masked_and_grouped_int4(dev, seq, quant):
    import torch
    import oracle as O
    from uocr_hip import ops, synth
    L = awq_layer(3000 + seq, group=32, n_shared=0, quantizer=quant)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    at, aw, cnt, _, _ = _route(L, x, dev)
    _, _, want = O.moe_layer(L, x, threads=16)  # n_shared = 0: the routed sum only
    xt = torch.from_numpy(x).to(dev)
    g, u, d = (ops.RefInt4Table(q, dev) for q in (L.gate, L.up, L.down))
    act = torch.empty(L.n_experts, seq, L.inter, dtype=torch.float32, device=dev)
    out = torch.zeros(seq, L.hidden, dtype=torch.float32, device=dev)
    ops.moe_experts_masked_int4(xt, g, u, d, at, aw, cnt, seq, act, out)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), want, f"masked_int4-{quant}-t{seq}")
    act2 = torch.empty_like(act)
    out2 = torch.zeros_like(out)
    ops.moe_grouped_gate_up_int4(xt, g, u, at, cnt, seq, act2)
    ops.moe_grouped_down_int4(act2, d, at, aw, cnt, seq, out2)
    torch.cuda.synchronize()
    _check(out2.cpu().numpy(), want, f"grouped_int4-{quant}-t{seq}")
    # act rows agree bit for bit between the two entry points (same kernel)
    c = cnt.cpu().numpy()
    a1, a2 = act.cpu().numpy(), act2.cpu().numpy()
    for e in range(L.n_experts):
        assert np.array_equal(a1[e, : c[e]], a2[e, : c[e]])


def _bf16_experts(L):
    """The layer's INT4 experts dequantised and rounded to bf16 (the BF16 expert
    format, include/uocr/config.h:111)."""
    import oracle as O
    from uocr_hip import synth
    conv = lambda q: synth.f32_to_bf16_bits(O.dequantize(q))  # noqa: E731
    return [conv(q) for q in L.gate], [conv(q) for q in L.up], [conv(q) for q in L.down]


def _bf16_reference(L, x, ids, w, gb, ub, db):
    """Reference CPU path with BF16 experts: WeightMatrix::matmul on BF16 runs
    ops::matmul_t_bf16 (src/runtime/weights.cpp:47-49), then silu_mul and the
    j-ordered weighted sum (src/engine/moe_decoder.cpp:62-97)."""
    import oracle as O
    seq, H = x.shape
    y = np.zeros((seq, L.top_k, H), np.float32)
    for e in range(L.n_experts):
        tok, j = np.nonzero(ids == e)
        if len(tok) == 0:
            continue
        xe = x[tok]
        act = O.silu_mul(O.matmul_t_bf16(xe, gb[e]), O.matmul_t_bf16(xe, ub[e]))
        y[tok, j] = O.matmul_t_bf16(act, db[e])
    out = np.zeros((seq, H), np.float32)
    for j in range(L.top_k):
        out = (w[:, j:j + 1] * y[:, j] + out).astype(np.float32)
    return out


@pytest.mark.parametrize("seq", [16, 300])
def test_masked_and_grouped_bf16(dev, seq):
    import torch
    from uocr_hip import ops, synth
    L = awq_layer(3100 + seq, group=32, n_experts=8, top_k=2, n_shared=0)
    x = synth.bf16_normal(np.random.default_rng(seq + 1), (seq, L.hidden), 1.0)
    at, aw, cnt, ids_o, w_o = _route(L, x, dev)
    gb, ub, db = _bf16_experts(L)
    want = _bf16_reference(L, x, ids_o, w_o, gb, ub, db)
    xt = torch.from_numpy(x).to(dev)
    to_dev = lambda mats: [torch.from_numpy(m.view(np.int16)).to(dev) for m in mats]  # noqa: E731
    gd, ud, dd = to_dev(gb), to_dev(ub), to_dev(db)
    act = torch.empty(L.n_experts, seq, L.inter, dtype=torch.float32, device=dev)
    out = torch.zeros(seq, L.hidden, dtype=torch.float32, device=dev)
    keep = ops.moe_experts_masked(xt, gd, ud, dd, at, aw, cnt, seq, act, out)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), want, f"masked_bf16-t{seq}")
    out2 = torch.zeros_like(out)
    k1 = ops.moe_grouped_gate_up_bf16(xt, gd, ud, at, cnt, seq, act)
    k2 = ops.moe_grouped_down_bf16(act, dd, at, aw, cnt, seq, out2)
    torch.cuda.synchronize()
    _check(out2.cpu().numpy(), want, f"grouped_bf16-t{seq}")
    del keep, k1, k2


@pytest.mark.parametrize("group", [32, 128])
def test_gemm_int4_variants(dev, group):
    """y = x . dequant(W)^T for one INT4 matrix (the per-expert GEMM of the host
    grouping path) against the oracle's INT4 matmul (weights.cpp:51-72, pinned);
    f32 inputs that are not bf16-valued; every _tc* variant gives the same bits."""
    import torch
    import oracle as O
    from uocr_hip import ops
    L = awq_layer(3200 + group, group=group, n_experts=1, n_shared=0)
    q = L.gate[0]
    x = (np.random.default_rng(group).standard_normal((37, q.cols)) * 0.7).astype(np.float32)
    want = O.matmul_int4(q, x)
    xt = torch.from_numpy(x).to(dev)
    pk = torch.from_numpy(q.packed).to(dev)
    sc = torch.from_numpy(q.scales).to(dev)
    zr = torch.from_numpy(q.zeros).to(dev)
    ys = []
    for v in ["", "_tc", "_tc_n", "_tc_nk", "_tc_pipe"]:
        y = torch.full((37, q.rows), float("nan"), dtype=torch.float32, device=dev)
        ops.moe_gemm_int4(xt, pk, sc, zr, q.rows, q.cols, group, y, variant=v)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    _check(ys[0], want, f"gemm_int4-g{group}")
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


def test_grouped_int4_skewed_groups(dev):
    """Zipf-routed tokens: the most popular expert holds several 64-row m-tiles,
    which the grouped mirrors spread over workgroups."""
    import torch
    import oracle as O
    from uocr_hip import ops, synth
    L = awq_layer(3300, group=32, n_experts=64, n_shared=0, router_bias=synth.zipf_bias())
    x = synth.bf16_normal(np.random.default_rng(33), (600, L.hidden), 1.0)
    x[:, 0] = 1.0
    at, aw, cnt, ids_o, _ = _route(L, x, dev)
    assert cnt.max().item() > 200, cnt.max().item()
    top = np.argmax(np.bincount(ids_o.ravel()))
    sel = np.unique(np.concatenate([np.nonzero((ids_o == top).any(1))[0][:24], np.arange(0, 600, 37)]))
    _, _, want = O.moe_layer(L, x, sel=sel.astype(np.int32), threads=16)
    xt = torch.from_numpy(x).to(dev)
    g, u, d = (ops.RefInt4Table(q, dev) for q in (L.gate, L.up, L.down))
    act = torch.empty(L.n_experts, 600, L.inter, dtype=torch.float32, device=dev)
    out = torch.zeros(600, L.hidden, dtype=torch.float32, device=dev)
    ops.moe_grouped_gate_up_int4(xt, g, u, at, cnt, 600, act)
    ops.moe_grouped_down_int4(act, d, at, aw, cnt, 600, out)
    torch.cuda.synchronize()
    _check(out.cpu().numpy()[sel], want[sel], "grouped_int4-zipf-t600")


def test_dense_and_elementwise_mirrors(dev):
    """matmul_t_bf16 / matvec_bf16 against the reference's CPU matmul_t_bf16
    (pinned), silu_mul / add_scaled / scatter_add_scaled / gather_rows against
    their definitions (gpu_ops.cu:12-45)."""
    import torch
    import oracle as O
    from uocr_hip import ops, synth
    rng = np.random.default_rng(44)
    for m, n, k in [(5, 1792, 1280), (300, 1280, 1792), (1, 64, 1280)]:
        x = rng.standard_normal((m, k)).astype(np.float32)
        wb = synth.f32_to_bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02))
        bias = rng.standard_normal(n).astype(np.float32)
        want = O.matmul_t_bf16(x, wb, bias)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        xt, wt, bt = (torch.from_numpy(a).to(dev) for a in (x, wb.view(np.int16), bias))
        if m == 1:
            ops.matvec_bf16(xt, wt, y, bt)
        else:
            ops.matmul_t_bf16(xt, wt, y, bt)
        torch.cuda.synchronize()
        _check(y.cpu().numpy(), want, f"matmul_t_bf16-{m}x{n}x{k}")
    g = (rng.standard_normal(5000) * 4).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    o = torch.empty(5000, dtype=torch.float32, device=dev)
    ops.silu_mul(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev), o)
    torch.cuda.synchronize()
    np.testing.assert_allclose(o.cpu().numpy(), O.silu_mul(g, u), rtol=2e-6, atol=1e-30)
    d0 = rng.standard_normal(5000).astype(np.float32)
    dt = torch.from_numpy(d0).to(dev)
    ops.add_scaled(dt, torch.from_numpy(u).to(dev), 0.37)
    torch.cuda.synchronize()
    exact = (d0.astype(np.float64) + np.float32(0.37) * u.astype(np.float64)).astype(np.float32)  # one rounding
    np.testing.assert_array_equal(dt.cpu().numpy(), exact)
    src = rng.standard_normal((40, 96)).astype(np.float32)
    idx = rng.integers(0, 40, 25).astype(np.int32)
    dst = torch.empty(25, 96, dtype=torch.float32, device=dev)
    ops.gather_rows(dst, torch.from_numpy(src).to(dev), torch.from_numpy(idx).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dst.cpu().numpy(), src[idx])
    vals = rng.standard_normal((25, 96)).astype(np.float32)
    wts = rng.standard_normal(25).astype(np.float32)
    rows = rng.permutation(40)[:25].astype(np.int32)  # distinct rows: the reference's exact result
    base = rng.standard_normal((40, 96)).astype(np.float32)
    out = torch.from_numpy(base.copy()).to(dev)
    ops.scatter_add_scaled(out, torch.from_numpy(vals).to(dev), torch.from_numpy(rows).to(dev),
                           torch.from_numpy(wts).to(dev))
    torch.cuda.synchronize()
    want = base.copy()
    want[rows] = (base[rows] + (wts[:, None] * vals)).astype(np.float32)
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    dup = np.array([3, 3, 3, 7], np.int32)  # repeated rows add up (atomically)
    out = torch.zeros(40, 96, dtype=torch.float32, device=dev)
    ops.scatter_add_scaled(out, torch.from_numpy(vals[:4]).to(dev), torch.from_numpy(dup).to(dev),
                           torch.from_numpy(np.ones(4, np.float32)).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy()[3], vals[:3].sum(0), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("seq", [16, 300])
def test_host_grouping_branch_from_mirrors(dev, seq):
    """GpuDecoder::mlp_block's host-grouping branch (src/engine/gpu_decoder.cu:
    590-657) rebuilt one operator at a time from the mirrors: per expert
    gather_rows -> moe_gemm_int4 (gate, up) -> silu_mul -> moe_gemm_int4 (down)
    -> scatter_add_scaled; the bf16 shared MLP as matmul_t_bf16 x 3 + silu_mul;
    out = add_scaled(moe) + add_scaled(shared). Against the CPU layer."""
    import torch
    import oracle as O
    from uocr_hip import ops, synth
    L = synth.with_bf16_shared(awq_layer(3400 + seq, group=32, n_experts=16), 3401)
    x = synth.bf16_normal(np.random.default_rng(seq + 5), (seq, L.hidden), 1.0)
    at, aw, cnt, _, _ = _route(L, x, dev)
    _, _, want = O.moe_layer(L, x, threads=16)
    H, I, SI = L.hidden, L.inter, L.n_shared * L.inter
    xt = torch.from_numpy(x).to(dev)
    moe = torch.zeros(seq, H, dtype=torch.float32, device=dev)
    c, atn, awn = cnt.cpu().numpy(), at.cpu().numpy(), aw.cpu().numpy()
    for e in range(L.n_experts):
        r = int(c[e])
        if r == 0:
            continue
        rows = torch.from_numpy(atn[e, :r].copy()).to(dev)
        rw = torch.from_numpy(awn[e, :r].copy()).to(dev)
        xg = torch.empty(r, H, dtype=torch.float32, device=dev)
        ops.gather_rows(xg, xt, rows)
        gg = torch.empty(r, I, dtype=torch.float32, device=dev)
        uu = torch.empty_like(gg)
        for q, dst in ((L.gate[e], gg), (L.up[e], uu)):
            ops.moe_gemm_int4(xg, torch.from_numpy(q.packed).to(dev), torch.from_numpy(q.scales).to(dev),
                              torch.from_numpy(q.zeros).to(dev), q.rows, q.cols, q.group, dst)
        act = torch.empty_like(gg)
        ops.silu_mul(gg, uu, act)
        yg = torch.empty(r, H, dtype=torch.float32, device=dev)
        q = L.down[e]
        ops.moe_gemm_int4(act, torch.from_numpy(q.packed).to(dev), torch.from_numpy(q.scales).to(dev),
                          torch.from_numpy(q.zeros).to(dev), q.rows, q.cols, q.group, yg)
        ops.scatter_add_scaled(moe, yg, rows, rw)
    dw = lambda d: torch.from_numpy(d.data.view(np.int16)).to(dev)  # noqa: E731
    sg, su = torch.empty(seq, SI, dtype=torch.float32, device=dev), torch.empty(seq, SI, dtype=torch.float32, device=dev)
    ops.matmul_t_bf16(xt, dw(L.shared_gate_w), sg)
    ops.matmul_t_bf16(xt, dw(L.shared_up_w), su)
    sa = torch.empty_like(sg)
    ops.silu_mul(sg, su, sa)
    so = torch.empty(seq, H, dtype=torch.float32, device=dev)
    ops.matmul_t_bf16(sa, dw(L.shared_down_w), so)
    out = torch.zeros(seq, H, dtype=torch.float32, device=dev)
    ops.add_scaled(out, moe, 1.0)
    ops.add_scaled(out, so, 1.0)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), want, f"host-grouping-mirrors-t{seq}")
