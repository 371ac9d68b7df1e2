"""GPU parity of the fused INT4 MoE layer against the CPU oracle.

Routing ids, routing weights and the per-expert permutation must be bit-exact;
layer outputs within rel_l2 <= 5e-3 and max-abs <= 2e-2.
"""
import numpy as np
import pytest

from helpers import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2, subsample

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def run_layer(layer, x_np, dtype, dev):
    torch = _torch()
    seq, H = x_np.shape
    x = torch.from_numpy(x_np).to(dev)
    x = x.to(torch.bfloat16) if dtype == "bf16" else x.float()
    out = torch.empty(seq, H, dtype=torch.float32, device=dev)
    ids = torch.empty(seq, layer.top_k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, layer.top_k, dtype=torch.float32, device=dev)
    ws = layer.alloc_workspace(seq, dev)
    layer.forward(x, out, ws, ids, w)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()


def check_parity(L, x, dev, sample=None, dtype="bf16", label=""):
    import oracle as O
    from uocr_hip import MoELayerInt4

    print(f"[parity] {label} seq={x.shape[0]} group={L.group} dtype={dtype}", flush=True)
    layer = MoELayerInt4(L)
    ids, w, out = run_layer(layer, x, dtype, dev)
    seq = x.shape[0]
    sel = None if sample is None else subsample(ids, seq, sample)
    ids_o, w_o, out_o = O.moe_layer(L, x, sel=sel, threads=16)
    assert np.array_equal(ids, ids_o), f"routing ids differ at {np.argwhere(ids != ids_o)[:5]}"
    assert np.array_equal(w.view(np.uint32), w_o.view(np.uint32)), "routing weights not bit-exact"
    rows = np.arange(seq) if sel is None else sel
    r, m = rel_l2(out[rows], out_o[rows]), max_abs(out[rows], out_o[rows])
    print(f"[parity] {label}: rel_l2={r:.3e} max_abs={m:.3e} rows={len(rows)}", flush=True)
    assert r <= REL_L2_TOL and m <= MAX_ABS_TOL
    layer.close()
    return ids, w, out


def test_config0_decode_t1(dev):
    from uocr_hip import synth
    w = synth.make_config(0)
    check_parity(w.layers[0], w.x, dev, label="cfg0")


def test_config1_decode_t16(dev):
    from uocr_hip import synth
    w = synth.make_config(1)
    check_parity(w.layers[0], w.x, dev, label="cfg1")


def test_config1_group128_f32_input(dev):
    from uocr_hip import synth
    w = synth.make_config(1, group=128)
    check_parity(w.layers[0], w.x, dev, dtype="f32", label="cfg1-g128-f32")


def test_config2_prefill_t1024(dev):
    from uocr_hip import synth
    w = synth.make_config(2)
    check_parity(w.layers[0], w.x, dev, sample=48, label="cfg2")


def test_config3_prefill_t4096_zipf(dev):
    from uocr_hip import synth
    w = synth.make_config(3)
    ids, _, _ = check_parity(w.layers[0], w.x, dev, sample=48, label="cfg3")
    counts = np.bincount(ids.ravel(), minlength=64)
    assert counts.max() > 1000, counts  # the skew the config asks for


@pytest.mark.parametrize("group", [32, 64, 128])
def test_prefill_full_and_half_mode_tiles(dev, group):
    """600 Zipf-routed tokens, every row checked: groups of several 256-row
    tiles, last tiles of 129..255 rows (full mode) and of 1..128 rows (half
    mode, listed after all full-mode tiles), including the shared groups'
    88-row last tiles; each quantisation group size has its own scale loads
    in the large-tile kernel."""
    from uocr_hip import synth
    import oracle as O
    L = synth.random_layer(4242, group=group, router_bias=synth.zipf_bias())
    x = synth.bf16_normal(np.random.default_rng(5), (600, L.hidden), 1.0)
    x[:, 0] = 1.0
    ids, _ = O.moe_gate(x, L.router_bf16, L.top_k)
    rem = np.bincount(ids.ravel(), minlength=L.n_experts) % 256
    counts = np.bincount(ids.ravel(), minlength=L.n_experts)
    assert (counts > 256).sum() >= 4 and (rem > 128).sum() >= 2 and ((rem > 0) & (rem <= 128)).sum() >= 8
    check_parity(L, x, dev, label=f"prefill-600-zipf-g{group}")


def test_config4_rmsnorm_residual_t64(dev):
    """Config 4's layer form: out = h + moe(rmsnorm(h)) with f32 h, 64 tokens;
    the second layer takes the oracle's f32 output of the first (not bf16-valued)."""
    import oracle as O
    from uocr_hip import synth
    w = synth.make_config(4, n_layers=2)
    check_parity(w.layers[0], w.x, dev, dtype="f32", label="cfg4-l0")
    _, _, h1 = O.moe_layer(w.layers[0], w.x, threads=16)
    check_parity(w.layers[1], h1, dev, dtype="f32", label="cfg4-l1")


@pytest.mark.parametrize("seq", [2, 63, 64, 65, 100, 255])
def test_decode_batch_sizes(dev, seq):
    """Both decode routers (one workgroup per token up to 64 tokens, LDS-shared
    router weights above) and the multi-m-tile expert loop (up to 16 tiles)."""
    from uocr_hip import synth
    L = synth.random_layer(500 + seq, group=32)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=24, label=f"decode-t{seq}")


def test_decode_group64_and_one_hot_expert(dev):
    """group 64, and a router that sends every token to the same experts
    (one expert with the whole batch: 48 tokens = 3 m-tiles)."""
    from uocr_hip import synth
    L = synth.random_layer(77, group=64)
    rb = L.router_bf16.copy()
    rb[:, 0] = synth.f32_to_bf16_bits(np.linspace(-8.0, 8.0, 64, dtype=np.float32))
    L.router_bf16 = rb
    x = synth.bf16_normal(np.random.default_rng(1), (48, L.hidden), 1.0)
    x[:, 0] = 64.0
    ids, _, _ = check_parity(L, x, dev, label="decode-onehot")
    assert (ids[:, 0] == 63).all()


@pytest.mark.parametrize("seq", [10, 300])
def test_other_shapes_prefill_kernels(dev, seq):
    """Shapes outside the decode instantiations (inter 384 = 3 k-tiles) run on
    the grouped prefill kernels at any batch; 16 experts, top-4, one shared."""
    from uocr_hip import synth
    L = synth.random_layer(900 + seq, hidden=512, inter=384, n_experts=16, top_k=4, n_shared=1, group=128)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, 512), 1.0)
    check_parity(L, x, dev, sample=32, label=f"shape512x384-t{seq}")


def test_permutation_bit_exact(dev):
    """Grouped slot order equals the reference host grouping
    (gpu_decoder.cu:602-609): checked through the mirror router's
    [n_experts, cap] tables on the same routing."""
    torch = _torch()
    import oracle as O
    from uocr_hip import ops, synth

    rng = np.random.default_rng(3)
    ops.moe_router_overflow(clear=True)
    for seq, E, k in [(1, 64, 6), (16, 64, 6), (517, 64, 6), (2048, 8, 2), (300, 128, 8), (1111, 64, 6)]:
        logits = rng.standard_normal((seq, E)).astype(np.float32)
        lg = torch.from_numpy(logits).to(dev)
        cap = seq
        ids = torch.empty(seq, k, dtype=torch.int32, device=dev)
        w = torch.empty(seq, k, dtype=torch.float32, device=dev)
        at = torch.full((E, cap), -1, dtype=torch.int32, device=dev)
        aw = torch.zeros(E, cap, dtype=torch.float32, device=dev)
        cnt = torch.empty(E, dtype=torch.int32, device=dev)
        ops.moe_router_topk(lg, k, False, 1.0, False, ids, w, at, aw, cnt, cap)
        torch.cuda.synchronize()
        # oracle: identity router on one-hot inputs reproduces logits exactly
        ids_o, w_o = O.moe_gate_f32router(logits, np.eye(E, dtype=np.float32), k)
        assert np.array_equal(ids.cpu().numpy(), ids_o)
        assert np.array_equal(w.cpu().numpy().view(np.uint32), w_o.view(np.uint32))
        counts, offs, perm = O.stable_group(ids_o, E)
        c = cnt.cpu().numpy()
        a = at.cpu().numpy()
        assert np.array_equal(c, np.minimum(counts, cap))
        aw_h = aw.cpu().numpy()
        for e in range(E):
            assert np.array_equal(a[e, : c[e]], perm[offs[e]: offs[e] + c[e]])
            # nothing written past an expert's entries (the multi-round grouping
            # once placed stale entries there)
            assert (a[e, c[e]:] == -1).all() and (aw_h[e, c[e]:] == 0).all(), e
        assert ops.moe_router_overflow() == 0
        # brute force: the stable sort of (expert, token) pairs
        flat_tok = np.repeat(np.arange(seq), k)
        assert np.array_equal(perm, flat_tok[np.argsort(ids_o.ravel(), kind="stable")])


def test_router_overflow_reported(dev):
    """cap below an expert's count: the tables keep the first `cap` entries in
    (token, j) order, count reads min(count, cap), and the overflow flag is
    raised (the reference drops the rest silently, moe_device.cu:90-95)."""
    torch = _torch()
    import oracle as O
    from uocr_hip import ops

    rng = np.random.default_rng(8)
    seq, E, k, cap = 64, 8, 2, 8
    logits = rng.standard_normal((seq, E)).astype(np.float32)
    lg = torch.from_numpy(logits).to(dev)
    ids = torch.empty(seq, k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, k, dtype=torch.float32, device=dev)
    at = torch.full((E, cap), -1, dtype=torch.int32, device=dev)
    aw = torch.zeros(E, cap, dtype=torch.float32, device=dev)
    cnt = torch.empty(E, dtype=torch.int32, device=dev)
    ops.moe_router_overflow(clear=True)
    ops.moe_router_topk(lg, k, False, 1.0, False, ids, w, at, aw, cnt, cap)
    torch.cuda.synchronize()
    ids_o, _ = O.moe_gate_f32router(logits, np.eye(E, dtype=np.float32), k)
    counts, offs, perm = O.stable_group(ids_o, E)
    assert counts.max() > cap
    assert np.array_equal(cnt.cpu().numpy(), np.minimum(counts, cap))
    a = at.cpu().numpy()
    for e in range(E):
        n = min(counts[e], cap)
        assert np.array_equal(a[e, :n], perm[offs[e]: offs[e] + n])
    assert ops.moe_router_overflow(clear=True) == 1
    assert ops.moe_router_overflow(clear=True) == 0


@pytest.mark.parametrize("seq", [5, 16, 300])
def test_routing_options(dev, seq):
    """norm_topk_prob = 1, sigmoid scoring and routed_scaling_factor = 2.5 on
    the decode (5), single-kernel (16, bf16) and prefill (300) paths."""
    from uocr_hip import synth
    for norm, sig, scale in [(1, 0, 1.0), (0, 1, 2.5), (1, 1, 2.5)]:
        L = synth.random_layer(700 + seq + 10 * sig + norm, group=32)
        L.norm_topk_prob, L.scoring_sigmoid, L.routed_scaling_factor = norm, sig, scale
        x = synth.bf16_normal(np.random.default_rng(seq + norm), (seq, L.hidden), 1.0)
        check_parity(L, x, dev, sample=24 if seq > 64 else None, label=f"route-n{norm}-s{sig}-x{scale}-t{seq}")


@pytest.mark.parametrize("seq", [5, 16, 300])
def test_no_shared_experts(dev, seq):
    """n_shared = 0 with 8 experts, top-2: no shared rows in y, on the decode,
    single-kernel and prefill paths."""
    from uocr_hip import synth
    L = synth.random_layer(800 + seq, n_experts=8, top_k=2, n_shared=0, group=32)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=24 if seq > 64 else None, label=f"noshared-t{seq}")


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("seq,dtype", [(5, "bf16"), (16, "bf16"), (16, "f32"), (300, "bf16")])
def test_awq_asymmetric_weights(dev, group, seq, dtype):
    """Weights from the reference's quantize_int4_awq (zeros 0..15, arbitrary f32
    scales) on every path: decode (5; 16 f32), single-kernel (16 bf16) and
    prefill (300). Scales are rounded to f16 on upload (relative error
    <= 2^-11 per scale)."""
    from helpers import awq_layer
    from uocr_hip import synth
    L = awq_layer(1000 + group + seq, group=group)
    zs = np.concatenate([q.zeros.ravel() for q in L.gate[:2]])
    assert zs.min() == 0 and zs.max() == 15 and (zs != 8).mean() > 0.5
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, dtype=dtype, label=f"awq-g{group}-t{seq}-{dtype}")


def test_awq_config4_form(dev):
    """AWQ weights in config 4's layer form (RMSNorm prologue + residual, f32 h)."""
    from helpers import awq_layer
    from uocr_hip import synth
    L = awq_layer(1999, group=32)
    L.rms_weight = np.random.default_rng(3).uniform(0.5, 2.0, L.hidden).astype(np.float32)
    x = synth.bf16_normal(np.random.default_rng(4), (64, L.hidden), 1.0)
    check_parity(L, x, dev, dtype="f32", label="awq-rms-t64")


@pytest.mark.parametrize("seq", [16, 300])
def test_symmetric_quantizer_f32_scales(dev, seq):
    """quantize_int4_symmetric output (zero 8, arbitrary f32 scales amax / 7):
    the implicit-zero layout with scales that are not bf16-valued."""
    from helpers import awq_layer
    from uocr_hip import synth
    L = awq_layer(2100 + seq, group=32, quantizer="sym")
    assert all((q.zeros == 8).all() for q in L.down[:3])
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, label=f"sym-f32scale-t{seq}")


@pytest.mark.parametrize("seq,dtype", [(300, "bf16"), (16, "f32")])
def test_f16_staging_overflow_flagged(dev, seq, dtype):
    """Activations staged as f16 that leave f16's range set status bit 2 (and
    reach the output as non-finite values); ordinary inputs leave it clear."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(900 + seq, group=32)
    layer = MoELayerInt4(L)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    run_layer(layer, x, dtype, dev)
    assert layer.status() == 0
    _, _, out = run_layer(layer, x * np.float32(2000.0), dtype, dev)  # |silu(g) * u| >> 65504
    assert layer.status() & 4 and not np.isfinite(out).all()
    assert layer.status() == 0  # cleared by the read
    layer.close()
