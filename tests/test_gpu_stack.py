"""Config 4 end to end: the 12-layer INT4 stack at 64 tokens, each layer
h <- h + moe(rmsnorm(h)) (src/engine/moe_decoder.cpp:166-179), captured in
one HIP graph and replayed, at group 32 and group 128.

Each layer is checked on the input the GPU itself gave it (its previous
layer's GPU output): routing ids / weights bit-exact, the layer output within
rel_l2 <= 5e-3 and max-abs <= 2e-2 of the oracle. The final hidden state is
also compared with the oracle chained from the step input alone, on the
tokens whose routing agrees in every layer.
"""
import numpy as np
import pytest

from helpers import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("group", [32, 128])
def test_config4_stack12_hipgraph(dev, group):
    import torch
    import oracle as O
    from uocr_hip import MoELayerInt4, synth

    wl = synth.make_config(4, group=group)
    seq, H = wl.seq, wl.layers[0].hidden
    print(f"[stack] group={group} layers={len(wl.layers)} seq={seq}", flush=True)
    layers = [MoELayerInt4(L) for L in wl.layers]
    x = torch.from_numpy(wl.x).to(dev).float()
    outs = [torch.empty(seq, H, dtype=torch.float32, device=dev) for _ in layers]
    ids = [torch.empty(seq, 6, dtype=torch.int32, device=dev) for _ in layers]
    wts = [torch.empty(seq, 6, dtype=torch.float32, device=dev) for _ in layers]
    ws = layers[0].alloc_workspace(seq, dev)

    def step():
        h = x
        for li, lay in enumerate(layers):
            lay.forward(h, outs[li], ws, ids[li], wts[li])
            h = outs[li]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = [o.cpu().numpy().copy() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for li, o in enumerate(outs):
            assert np.array_equal(o.cpu().numpy().view(np.uint32), eager[li].view(np.uint32)), (rep, li)
        step()  # eager work between replays
        torch.cuda.synchronize()

    h_in = wl.x.astype(np.float32)
    for li, L in enumerate(wl.layers):
        ids_o, w_o, out_o = O.moe_layer(L, h_in, threads=16)
        got_ids, got_w = ids[li].cpu().numpy(), wts[li].cpu().numpy()
        assert np.array_equal(got_ids, ids_o), f"layer {li}: ids differ at {np.argwhere(got_ids != ids_o)[:5]}"
        assert np.array_equal(got_w.view(np.uint32), w_o.view(np.uint32)), f"layer {li}: weights not bit-exact"
        r, m = rel_l2(eager[li], out_o), max_abs(eager[li], out_o)
        print(f"[stack] g{group} layer {li}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
        assert r <= REL_L2_TOL and m <= MAX_ABS_TOL, li
        h_in = eager[li]  # the GPU's own output feeds the next layer

    # Chained from the step input alone, the oracle's h drifts from the GPU's
    # by the per-layer rounding differences; a token whose top-k choice is a
    # near tie can then pick another expert in a later layer, which changes
    # its row by far more than the tolerance. Tokens routed identically in
    # every layer must match within tolerance; the flips are counted.
    h = wl.x.astype(np.float32)
    same = np.ones(seq, bool)
    for li, L in enumerate(wl.layers):
        ids_c, _, h = O.moe_layer(L, h, threads=16)
        same &= (ids_c == ids[li].cpu().numpy()).all(axis=1)
    r, m = rel_l2(eager[-1][same], h[same]), max_abs(eager[-1][same], h[same])
    print(f"[stack] g{group} chained from the step input: {int((~same).sum())} of {seq} tokens routed "
          f"differently in some layer; the rest rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    # (per-layer parity above is the bar; over 12 chained layers the residual
    # stream grows and the absolute differences with it, so only rel_l2 holds)
    assert same.sum() >= seq - seq // 8
    assert r <= REL_L2_TOL
    for lay in layers:
        lay.close()
