"""uocr_hip_moe_layer_forward_noalloc (library-owned device scratch, no
workspace argument, no allocation) against uocr_hip_moe_layer_forward on the
same inputs, through the C ABI: two calls in a row, the second with a smaller
batch, bit-identical outputs and routing (the same kernels run on both)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(layer, x, dev, noalloc):
    import torch
    seq = x.shape[0]
    out = torch.full((seq, layer.hidden), float("nan"), dtype=torch.float32, device=dev)
    ids = torch.full((seq, layer.top_k), -1, dtype=torch.int32, device=dev)
    w = torch.zeros(seq, layer.top_k, dtype=torch.float32, device=dev)
    if noalloc:
        layer.forward_noalloc(x, out, ids, w)
    else:
        ws = layer.alloc_workspace(seq, dev)
        layer.forward(x, out, ws, ids, w)
    torch.cuda.synchronize()
    return out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("sizes,dtype", [((200, 16), "bf16"), ((64, 5), "f32"), ((16, 12), "bf16")])
def test_noalloc_matches_forward(dev, sizes, dtype):
    import torch
    from uocr_hip import MoELayerInt4, synth

    L = synth.random_layer(6100 + sizes[0], group=32)
    layer = MoELayerInt4(L)
    for seq in sizes:  # second call smaller than the first
        print(f"[noalloc] seq={seq} dtype={dtype}", flush=True)
        assert layer.workspace_size(seq) <= 64 << 20
        xn = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
        x = torch.from_numpy(xn).to(dev)
        x = x.to(torch.bfloat16) if dtype == "bf16" else x.float()
        a = _run(layer, x, dev, noalloc=True)
        b = _run(layer, x, dev, noalloc=False)
        assert np.array_equal(a[1], b[1]) and np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)), seq
    layer.close()


def test_noalloc_rejects_oversized_batch(dev):
    from uocr_hip import MoELayerInt4, synth
    from uocr_hip._lib import EINVAL, HipError
    import torch

    L = synth.random_layer(6200, group=32)
    layer = MoELayerInt4(L)
    seq = 4096
    assert layer.workspace_size(seq) > 64 << 20
    x = torch.zeros(seq, L.hidden, dtype=torch.bfloat16, device=dev)
    out = torch.empty(seq, L.hidden, dtype=torch.float32, device=dev)
    with pytest.raises(HipError) as ei:
        layer.forward_noalloc(x, out)
    assert ei.value.code == EINVAL and "no-alloc scratch" in str(ei.value)
    layer.close()
