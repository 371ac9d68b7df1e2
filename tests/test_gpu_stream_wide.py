"""GPU parity of the streamed decode kernel's wide mode: up to 64 tokens, bf16
or f32 input, optionally the RMSNorm prologue with the residual added (the
engine's decode-layer form, src/engine/moe_decoder.cpp:166-179). The routers
finish the exact routing first; every item then takes one 16-token block of
its group's tokens, and groups with more than 16 tokens (the shared groups
from 17 tokens, popular experts under skewed routing) get extra blocks.

Routing ids / weights bit-exact, outputs within rel_l2 <= 5e-3 and
max-abs <= 2e-2 of the oracle. One layer object serves several batch sizes in
a row, as the kernel's progress words must advance in step across calls.
"""
import numpy as np
import pytest

from helpers import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def _forward(layer, x_np, dev, dtype):
    import torch
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


def _check(layer, L, x, dev, dtype, label):
    import oracle as O
    seq = x.shape[0]
    kind = layer.decode_kernel(seq, dtype)
    print(f"[wide] {label} seq={seq} dtype={dtype} kernel={kind}", flush=True)
    assert kind == "stream", f"{label}: decode kernel {kind}"
    ids, w, out = _forward(layer, x, dev, dtype)
    ids_o, w_o, out_o = O.moe_layer(L, x, threads=16)
    assert np.array_equal(ids, ids_o), f"{label}: routing ids differ at {np.argwhere(ids != ids_o)[:5]}"
    assert np.array_equal(w.view(np.uint32), w_o.view(np.uint32)), f"{label}: routing weights not bit-exact"
    r, m = rel_l2(out, out_o), max_abs(out, out_o)
    print(f"[wide] {label}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    assert r <= REL_L2_TOL and m <= MAX_ABS_TOL, label
    flags = layer.status()
    assert flags == 0, f"{label}: status flags {flags:#x}"
    return ids, w, out


def _x(seq, hidden, seed, scale=1.0):
    from uocr_hip import synth
    return synth.bf16_normal(np.random.default_rng(seed), (seq, hidden), scale)


@pytest.mark.parametrize("group", [32, 128])
def test_wide_batch_sizes_bf16(dev, group):
    """bf16 input beyond 16 tokens, with calls of the 16-token mode between."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6100 + group, group=group)
    layer = MoELayerInt4(L)
    layer.set_decode_kernel("stream")
    for seq in (17, 64, 3, 40, 64):
        _check(layer, L, _x(seq, L.hidden, 6100 + seq), dev, "bf16", f"wide-g{group}-t{seq}")
    layer.close()


@pytest.mark.parametrize("group", [32, 128])
def test_wide_rmsnorm_f32(dev, group):
    """Config 4's layer form (f32 h, RMSNorm weights in [0.5, 2), residual)
    through the default kernel choice, 1 to 64 tokens."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6200 + group, group=group, rms=True)
    layer = MoELayerInt4(L)
    for seq in (64, 1, 8, 33):
        _check(layer, L, _x(seq, L.hidden, 6200 + seq), dev, "f32", f"wide-rms-g{group}-t{seq}")
    layer.close()


@pytest.mark.parametrize("kind", ["fused", "stream"])
def test_single_kernel_f32_input(dev, kind):
    """f32 hidden states without RMSNorm (the engine's normed2) up to 16
    tokens on both single-kernel decode paths: the routers read the f32 rows
    and the workers convert them to f16 themselves (the default choice takes
    the fused kernel below 6 tokens, the streamed one from 6)."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6350, group=32)
    layer = MoELayerInt4(L)
    layer.set_decode_kernel(kind)
    for seq in (1, 5, 16, 3):
        x = _x(seq, L.hidden, 6350 + seq)
        got = layer.decode_kernel(seq, "f32")
        assert got == kind, f"f32 t{seq}: decode kernel {got}"
        import oracle as O
        print(f"[wide] {kind}-f32-t{seq}", flush=True)
        ids, w, out = _forward(layer, x, dev, "f32")
        ids_o, w_o, out_o = O.moe_layer(L, x, threads=16)
        assert np.array_equal(ids, ids_o), f"{kind}-f32-t{seq}: routing ids"
        assert np.array_equal(w.view(np.uint32), w_o.view(np.uint32)), f"{kind}-f32-t{seq}: routing weights"
        r, m = rel_l2(out, out_o), max_abs(out, out_o)
        print(f"[wide] {kind}-f32-t{seq}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
        assert r <= REL_L2_TOL and m <= MAX_ABS_TOL
    assert layer.status() == 0
    layer.close()
    auto = MoELayerInt4(L)
    assert auto.decode_kernel(3, "f32") == "fused" and auto.decode_kernel(8, "f32") == "stream"
    auto.close()


def test_wide_f32_input_no_rms(dev):
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6300, group=64)
    layer = MoELayerInt4(L)
    for seq in (16, 50):
        _check(layer, L, _x(seq, L.hidden, 6300 + seq), dev, "f32", f"wide-f32-t{seq}")
    layer.close()


def test_wide_skewed_extra_blocks(dev):
    """Zipf-biased routing at 64 tokens: the most popular experts take more
    than 16 and more than 32 tokens (2 to 4 blocks each)."""
    import oracle as O
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6400, router_bias=synth.zipf_bias(beta=2.0))
    x = _x(64, L.hidden, 6400)
    x[:, 0] = 1.0
    ids, _ = O.moe_gate(x, L.router_bf16, L.top_k)
    counts = np.bincount(ids.ravel(), minlength=L.n_experts)
    print(f"[wide] skewed counts: max {counts.max()}, >16: {(counts > 16).sum()}, >32: {(counts > 32).sum()}",
          flush=True)
    assert (counts > 32).sum() >= 1 and (counts > 16).sum() >= 2
    layer = MoELayerInt4(L)
    _check(layer, L, x, dev, "bf16", "wide-skewed-t64")
    layer.close()


def test_wide_few_experts_no_shared(dev):
    """8 experts, top-2, no shared MLP: fewer block-0 items than workers, so
    workers start on extra blocks known only after the routing."""
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6500, n_experts=8, top_k=2, n_shared=0)
    layer = MoELayerInt4(L)
    layer.set_decode_kernel("stream")
    for seq in (64, 20):
        _check(layer, L, _x(seq, L.hidden, 6500 + seq), dev, "bf16", f"wide-e8-t{seq}")
    layer.close()


def test_wide_graph_replay(dev):
    """The 64-token RMSNorm layer captured in a HIP graph: every replay equals
    the eager result bit for bit, with eager calls between the replays."""
    import torch
    from uocr_hip import MoELayerInt4, synth
    L = synth.random_layer(6600, rms=True)
    layer = MoELayerInt4(L)
    seq = 64
    x_np = _x(seq, L.hidden, 6600)
    eager = _check(layer, L, x_np, dev, "f32", "wide-graph-eager")
    x = torch.from_numpy(x_np).to(dev).float()
    out = torch.empty(seq, L.hidden, dtype=torch.float32, device=dev)
    ids = torch.empty(seq, layer.top_k, dtype=torch.int32, device=dev)
    w = torch.empty(seq, layer.top_k, dtype=torch.float32, device=dev)
    ws = layer.alloc_workspace(seq, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.forward(x, out, ws, ids, w)
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
        _forward(layer, x_np, dev, "f32")
    assert layer.status() == 0
    layer.close()


@pytest.mark.parametrize("group", [32, 128])
def test_wide_reference_quantizers_rmsnorm(dev, group):
    """Wide mode on a layer from the reference's AWQ quantizer (zeros in
    [0, 15], arbitrary f32 scales): the zero offsets of the down projection
    come from the k-tile-ordered copy; with the RMSNorm prologue and f32 input."""
    from helpers import awq_layer
    from uocr_hip import MoELayerInt4
    L = awq_layer(6700 + group, group=group)
    L.rms_weight = np.random.default_rng(6701).uniform(0.5, 2.0, L.hidden).astype(np.float32)
    layer = MoELayerInt4(L)
    for seq in (40, 64, 7):
        _check(layer, L, _x(seq, L.hidden, 6700 + seq), dev, "f32", f"wide-awq-rms-g{group}-t{seq}")
    layer.close()


def _f32_router(L, seed):
    L.router_f32 = (np.random.default_rng(seed).standard_normal((L.n_experts, L.hidden)) * 0.03).astype(np.float32)
    return L


@pytest.mark.parametrize("group", [32, 128])
def test_wide_f32_router_rmsnorm(dev, group):
    """The engine's AWQ-folded layer form: an f32 router (the reference's
    uncontracted f32 chain), the RMSNorm prologue on f32 hidden states, through
    the streamed kernel's f32-router instantiation at 17 to 64 tokens and below."""
    from helpers import awq_layer
    from uocr_hip import MoELayerInt4
    L = _f32_router(awq_layer(6800 + group, group=group), 6801)
    L.rms_weight = np.random.default_rng(6802).uniform(0.5, 2.0, L.hidden).astype(np.float32)
    layer = MoELayerInt4(L)
    for seq in (17, 32, 64, 1, 8):
        _check(layer, L, _x(seq, L.hidden, 6800 + seq), dev, "f32", f"wide-f32router-g{group}-t{seq}")
    layer.close()


@pytest.mark.parametrize("group", [32, 64])
def test_f32_router_16_token_mode(dev, group):
    """An f32 router without RMSNorm, bf16 and f32 input, 1 to 16 tokens: the
    16-token mode's f32-router instantiation (every batch size, as the fused
    kernel needs the bf16 router)."""
    from helpers import awq_layer
    from uocr_hip import MoELayerInt4
    L = _f32_router(awq_layer(6900 + group, group=group), 6901)
    layer = MoELayerInt4(L)
    for seq, dt in ((16, "bf16"), (3, "bf16"), (9, "f32"), (1, "f32")):
        _check(layer, L, _x(seq, L.hidden, 6900 + seq), dev, dt, f"f32router-g{group}-t{seq}-{dt}")
    layer.close()
