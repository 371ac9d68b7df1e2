"""GPU parity of unquantised matrices: the shared MLP in the reference's own
form (bf16 checkpoint views, F32 gate/up after the AWQ fold;
src/runtime/weights.cpp:185-207,289-292, run as bf16 linear_forward calls in
src/engine/gpu_decoder.cu:647-652) and bf16 routed experts (the reference's
default expert format, include/uocr/config.h:111; moe_grouped_*_bf16,
src/kernels/cuda/moe_gemm_bf16.cu:122-353).

The oracle runs those matrices through the reference's CPU chains
(WeightMatrix::matmul -> matmul_t_bf16 / matmul_t, weights.cpp:51-60), pinned
to the reference's own cpu_ops.cpp in tests/test_oracle.py. Routing ids and
weights bit-exact; outputs within rel_l2 <= 5e-3 and max-abs <= 2e-2.
"""
import numpy as np
import pytest

from test_gpu_layer import check_parity, run_layer

pytestmark = pytest.mark.gpu


def _stages(L, x, dtype, dev):
    from uocr_hip import MoELayer
    layer = MoELayer(L)
    layer.set_timing(True)
    run_layer(layer, x, dtype, dev)
    t, n = layer.read_timing()
    layer.close()
    assert n == 1
    return t


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_bf16_shared_mlp_configs(dev, cfg):
    """BASELINE configs with the shared MLP as bf16 matrices; INT4 routed experts."""
    from uocr_hip import synth
    w = synth.make_config(cfg)
    L = synth.with_bf16_shared(w.layers[0], 500 + cfg)
    check_parity(L, w.x, dev, sample=48 if w.seq > 64 else None, label=f"cfg{cfg}-bf16-shared")


def test_bf16_shared_paths(dev):
    """16 tokens: bf16 and f32 input both take the single-kernel decode with
    the shared MLP launched before it (f32 input: on f16 rows of the input)."""
    from uocr_hip import synth
    w = synth.make_config(1)
    L = synth.with_bf16_shared(w.layers[0], 511)
    for dt in ("bf16", "f32"):
        t = _stages(L, w.x, dt, dev)
        assert t["fused"] > 0 and t["shared"] > 0 and t["gate_up"] == 0, (dt, t)
    check_parity(L, w.x, dev, dtype="f32", label="cfg1-bf16-shared-f32")


@pytest.mark.parametrize("seq", [1, 16, 40])
def test_bf16_shared_rmsnorm_single_kernel(dev, seq):
    """The engine's layer form (f32 hidden states, RMSNorm prologue, residual,
    bf16 shared MLP) up to 64 tokens: the shared MLP runs on f16 rows of the
    normalised input, then the streamed kernel's wide mode adds its rows."""
    from uocr_hip import synth
    L = synth.with_bf16_shared(synth.random_layer(540 + seq, group=32, rms=True), 541 + seq)
    x = synth.bf16_normal(np.random.default_rng(seq + 7), (seq, L.hidden), 1.0)
    t = _stages(L, x, "f32", dev)
    assert t["fused"] > 0 and t["shared"] > 0 and t["gate_up"] == 0, t
    check_parity(L, x, dev, dtype="f32", label=f"rms-bf16-shared-single-t{seq}")


@pytest.mark.parametrize("seq", [64, 200])
def test_bf16_shared_rmsnorm_residual(dev, seq):
    """The engine's own form: f32 hidden states, RMSNorm prologue, residual,
    bf16 shared MLP (64 tokens: decode tiles; 200: the 128-slot tiles)."""
    from uocr_hip import synth
    L = synth.with_bf16_shared(synth.random_layer(520 + seq, group=32, rms=True), 521 + seq)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, dtype="f32", label=f"rms-bf16-shared-t{seq}")


@pytest.mark.parametrize("seq", [16, 300])
def test_f32_shared_gate_up(dev, seq):
    """Shared gate/up as F32 matrices (what scale_columns materialises after the
    AWQ fold, weights.cpp:185-207), down bf16; the oracle takes matmul_t for
    the F32 ones."""
    from uocr_hip import synth
    L = synth.with_bf16_shared(synth.random_layer(530 + seq, group=32), 531)
    rng = np.random.default_rng(seq)
    s = rng.uniform(0.25, 4.0, L.hidden).astype(np.float32)
    L.shared_gate_w = synth.Dense(L.shared_gate_w.to_f32() * s[None, :])
    L.shared_up_w = synth.Dense(L.shared_up_w.to_f32() * s[None, :])
    x = synth.bf16_normal(rng, (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, label=f"f32-shared-t{seq}")


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_bf16_experts_configs(dev, cfg):
    """bf16 routed experts and bf16 shared MLP, 64 experts top-6, at the
    BASELINE configs' token counts and inputs (config 3 with the Zipf router)."""
    from uocr_hip import synth
    w = synth.make_config(cfg)
    L = synth.random_layer_bf16(600 + cfg, router_bias=synth.zipf_bias() if cfg == 3 else None)
    check_parity(L, w.x, dev, sample=48 if w.seq > 64 else None, label=f"cfg{cfg}-bf16-experts")


@pytest.mark.parametrize("seq", [5, 37, 255])
def test_bf16_experts_decode_sizes(dev, seq):
    from uocr_hip import synth
    L = synth.random_layer_bf16(610 + seq)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, dtype="f32" if seq == 37 else "bf16",
                 label=f"bf16-experts-t{seq}")


def test_bf16_experts_rmsnorm_residual_no_shared(dev):
    from uocr_hip import synth
    L = synth.random_layer_bf16(620, rms=True)
    x = synth.bf16_normal(np.random.default_rng(1), (64, L.hidden), 1.0)
    check_parity(L, x, dev, dtype="f32", label="bf16-experts-rms-t64")
    L = synth.random_layer_bf16(621, n_experts=8, top_k=2, n_shared=0)
    x = synth.bf16_normal(np.random.default_rng(2), (300, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32, label="bf16-experts-noshared-t300")


def test_dense_refusals(dev):
    """Values beyond f16's range are refused, and so are unquantised routed
    experts beside an INT4 shared MLP (the reference's shared MLP is never
    quantised); INT4 routed experts beside an unquantised shared MLP are fine."""
    from uocr_hip import HipError, MoELayer, synth
    L = synth.random_layer_bf16(630, hidden=256, inter=128, n_experts=4, top_k=2, n_shared=1)
    big = L.shared_up_w.to_f32().copy()
    big[3, 5] = 1e5
    L.shared_up_w = synth.Dense(big)
    with pytest.raises(HipError, match="f16 range"):
        MoELayer(L)
    L = synth.random_layer(631, hidden=256, inter=128, n_experts=4, top_k=2, n_shared=1, group=32)
    D = synth.random_layer_bf16(632, hidden=256, inter=128, n_experts=4, top_k=2, n_shared=1)
    L.gate_w, L.up_w, L.down_w = D.gate_w, D.up_w, D.down_w
    with pytest.raises(HipError, match="unquantised shared MLP"):
        MoELayer(L)
    L.gate_w = L.up_w = L.down_w = None
    L.shared_gate_w, L.shared_up_w, L.shared_down_w = D.shared_gate_w, D.shared_up_w, D.shared_down_w
    MoELayer(L).close()
