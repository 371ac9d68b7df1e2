"""GPU parity of the single-kernel decode paths (router + experts + combine in
one persistent launch; seq <= 16, bf16 input, hidden 1280 / inter 896): the
streamed kernel (every expert group once, gate/up and down together as split-K
partials) and the fused kernel (gate/up -> down hand-over between
workgroups), each forced with set_decode_kernel and run on the same cases.

The kernel's workgroups publish per-call progress words that must advance in
step across calls, so the tests reuse one layer object across batch sizes and
repeat calls, and replay it from a captured HIP graph. Routing ids / weights
bit-exact, outputs within rel_l2 <= 5e-3 and max-abs <= 2e-2.
"""
import numpy as np
import pytest

from helpers import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2

pytestmark = pytest.mark.gpu

KINDS = ["stream", "fused"]


def _layer(L, kind):
    from uocr_hip import MoELayerInt4
    layer = MoELayerInt4(L)
    layer.set_decode_kernel(kind)
    return layer


def _forward(layer, x_np, dev, ws=None):
    import torch
    seq, H = x_np.shape
    x = torch.from_numpy(x_np).to(dev).to(torch.bfloat16)
    out = torch.empty(seq, H, dtype=torch.float32, device=dev)
    ids = torch.empty(seq, layer.top_k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, layer.top_k, dtype=torch.float32, device=dev)
    ws = layer.alloc_workspace(seq, dev) if ws is None else ws
    layer.forward(x, out, ws, ids, w)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()


def _check(L, x, got, label):
    import oracle as O
    ids, w, out = got
    ids_o, w_o, out_o = O.moe_layer(L, x, threads=16)
    assert np.array_equal(ids, ids_o), f"{label}: routing ids differ at {np.argwhere(ids != ids_o)[:5]}"
    assert np.array_equal(w.view(np.uint32), w_o.view(np.uint32)), f"{label}: routing weights not bit-exact"
    r, m = rel_l2(out, out_o), max_abs(out, out_o)
    print(f"[decode1] {label}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    assert r <= REL_L2_TOL and m <= MAX_ABS_TOL, label


def _status_clear(layer, label):
    flags = layer.status()
    assert flags == 0, f"{label}: fused status flags {flags:#x}"


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("group", [32, 64, 128])
def test_fused_batch_sizes_one_layer(dev, group, kind):
    """One layer object, the batch size changing between calls: 12..16 tokens
    run the single kernel with dense gate/up, 1..11 tokens the same kernel with
    gate/up over the candidate groups only, so the progress words and the
    schedule must stay consistent across calls that switch modes."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(4100 + group, group=group)
    layer = _layer(L, kind)
    for seq in (16, 1, 3, 11, 12, 16, 7):
        x = synth.bf16_normal(np.random.default_rng(seq * 7 + group), (seq, L.hidden), 1.0)
        print(f"[decode1] {kind} group={group} seq={seq}", flush=True)
        assert layer.decode_kernel(seq) == kind
        _check(L, x, _forward(layer, x, dev), f"{kind}-g{group}-t{seq}")
    _status_clear(layer, f"g{group}")
    layer.close()


@pytest.mark.parametrize("kind", KINDS)
def test_fused_repeat_deterministic(dev, kind):
    """Ten calls in a row give bit-identical results (fixed reduction order,
    progress words advancing every call)."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(4200)
    layer = _layer(L, kind)
    x = synth.bf16_normal(np.random.default_rng(5), (16, L.hidden), 1.0)
    first = _forward(layer, x, dev)
    _check(L, x, first, "repeat-0")
    for i in range(9):
        ids, w, out = _forward(layer, x, dev)
        assert np.array_equal(ids, first[0]) and np.array_equal(w, first[1])
        assert np.array_equal(out.view(np.uint32), first[2].view(np.uint32)), f"call {i + 1} differs"
    layer.close()


@pytest.mark.parametrize("kind", KINDS)
def test_fused_two_layers_interleaved(dev, kind):
    """Two layers (separate progress words) called alternately on one workspace."""
    from uocr_hip import MoELayerInt4, synth
    La, Lb = synth.random_layer(4300), synth.random_layer(4301)
    la, lb = _layer(La, kind), _layer(Lb, kind)
    x = synth.bf16_normal(np.random.default_rng(9), (14, La.hidden), 1.0)
    ws = la.alloc_workspace(14, dev)
    for rep in range(3):
        _check(La, x, _forward(la, x, dev, ws), f"A{rep}")
        _check(Lb, x, _forward(lb, x, dev, ws), f"B{rep}")
    la.close()
    lb.close()


@pytest.mark.parametrize("kind", KINDS)
def test_fused_graph_replay(dev, kind):
    """Captured in a HIP graph and replayed: every replay equals the eager
    result, with eager work and synchronisations between the replays."""
    import torch
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(4400)
    layer = _layer(L, kind)
    seq = 16
    x_np = synth.bf16_normal(np.random.default_rng(11), (seq, L.hidden), 1.0)
    eager = _forward(layer, x_np, dev)
    _check(L, x_np, eager, "graph-eager")
    x = torch.from_numpy(x_np).to(dev).to(torch.bfloat16)
    out = torch.empty(seq, L.hidden, dtype=torch.float32, device=dev)
    ids = torch.empty(seq, layer.top_k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, layer.top_k, dtype=torch.float32, device=dev)
    ws = layer.alloc_workspace(seq, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.forward(x, out, ws, ids, w)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.forward(x, out, ws, ids, w)
    for rep in range(4):
        out.fill_(float("nan"))
        ids.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), eager[0]), f"replay {rep}: ids"
        assert np.array_equal(out.cpu().numpy().view(np.uint32), eager[2].view(np.uint32)), f"replay {rep}: out"
        _forward(layer, x_np, dev)  # eager call between replays
    layer.close()


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("ulps", [0, 1])
def test_fused_tied_router_rows(dev, ulps, kind):
    """Ties at the top-k boundary: five experts lead by a router bias, then a
    pair whose router rows are identical (ulps=0: equal scores, the lower index
    wins) or one bf16 ulp apart in one column. The candidate experts must hold
    every exact pick (status flag bit 1 stays clear) and the output match."""
    from uocr_hip import MoELayerInt4, synth
    bias = np.full(64, -1.0, np.float32)
    bias[[2, 11, 30, 41, 55]] = 2.0
    bias[[9, 20]] = 1.0
    L = synth.random_layer(4500 + ulps, router_bias=bias)
    L.router_bf16[20] = L.router_bf16[9]
    if ulps:
        L.router_bf16[20, 100] = L.router_bf16[9, 100] + np.uint16(ulps)
    layer = _layer(L, kind)
    # every candidate source: 16 tokens (dense, the routers' candidates), 7
    # (sparse, the routers' candidates), 3 and 1 (sparse, the per-expert
    # estimate workgroups)
    for seq in (16, 7, 3, 1):
        print(f"[decode1] {kind} tied ulps={ulps} seq={seq}", flush=True)
        # small channels 1.. keep the bias order: five leaders, then the pair
        x = synth.bf16_normal(np.random.default_rng(13), (seq, L.hidden), 0.01)
        x[:, 0] = 1.0
        got = _forward(layer, x, dev)
        _check(L, x, got, f"tied-{ulps}-t{seq}")
        if ulps == 0:
            assert (got[0] == 9).any(axis=1).all() and not (got[0] == 20).any(), "equal scores: lower index"
        _status_clear(layer, f"tied-{ulps}-t{seq}")
    layer.close()


@pytest.mark.parametrize("kind", KINDS)
def test_fused_status_async_and_path(dev, kind):
    """The stream-ordered status copy reads the same (clear) flags as the
    synchronising query, and 16-token bf16 calls take the decode path."""
    import torch
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(4600)
    layer = _layer(L, kind)
    x = synth.bf16_normal(np.random.default_rng(21), (16, L.hidden), 1.0)
    _check(L, x, _forward(layer, x, dev), "status-async")
    flags = torch.full((1,), -1, dtype=torch.int32, device=dev)
    layer.status_async(flags)
    torch.cuda.synchronize()
    assert int(flags.item()) == 0
    assert layer.path(16) == "decode"
    _status_clear(layer, "status-async")
    layer.close()


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("quantizer", ["awq", "symmetric"])
def test_stream_reference_quantizers(dev, group, quantizer):
    """The streamed kernel on layers from the reference's own quantizers
    (asymmetric zeros in [0, 15] and arbitrary f32 scales for AWQ): its down
    scales and zero offsets come from the k-tile-ordered copy made at create."""
    from helpers import awq_layer
    L = awq_layer(4700 + group, group=group, quantizer=quantizer)
    layer = _layer(L, "stream")
    for seq in (16, 5):
        x = synth_x(seq, L.hidden, 4700 + seq)
        print(f"[decode1] stream {quantizer} g{group} seq={seq}", flush=True)
        _check(L, x, _forward(layer, x, dev), f"stream-{quantizer}-g{group}-t{seq}")
    _status_clear(layer, f"stream-{quantizer}")
    layer.close()


def test_stream_bf16_shared(dev):
    """INT4 routed experts beside the reference's unquantised (bf16) shared
    MLP: the shared MLP's launches write y_shared, which the streamed kernel's
    combine adds."""
    from uocr_hip import synth
    L = synth.random_layer(4800)
    synth.with_bf16_shared(L, 4801)
    layer = _layer(L, "stream")
    for seq in (16, 3):
        x = synth_x(seq, L.hidden, 4800 + seq)
        print(f"[decode1] stream bf16-shared seq={seq}", flush=True)
        _check(L, x, _forward(layer, x, dev), f"stream-bf16shared-t{seq}")
    _status_clear(layer, "stream-bf16shared")
    layer.close()


def synth_x(seq, hidden, seed):
    from uocr_hip import synth
    return synth.bf16_normal(np.random.default_rng(seed), (seq, hidden), 1.0)
