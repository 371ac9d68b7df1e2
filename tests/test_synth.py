"""Seeded synthetic workloads match the BASELINE config shapes and statistics."""
import numpy as np

import oracle as O
from uocr_hip import synth


def test_config_shapes():
    for cfg, seq in [(0, 1), (1, 16), (2, 1024)]:
        w = synth.make_config(cfg)
        assert w.x.shape == (seq, 1280) and w.seq == seq
        L = w.layers[0]
        assert (L.n_experts, L.top_k, L.n_shared, L.group) == (64, 6, 2, 32)
        assert L.gate[0].packed.shape == (896, 640) and L.down[0].packed.shape == (1280, 448)
        assert L.shared_gate.rows == 1792 and L.shared_down.cols == 1792
        assert np.all(L.gate[0].zeros == 8.0)
        # bf16-valued inputs and scales (exact upcast into the f32 oracle)
        assert np.array_equal(synth.bf16_round(w.x), w.x)
        assert np.array_equal(synth.bf16_round(L.gate[3].scales), L.gate[3].scales)
    w2 = synth.make_config(2)
    assert abs(w2.x[:900].std() - 0.5) < 0.01 and abs(w2.x[900:].std() - 1.0) < 0.02


def test_config4_stack():
    w = synth.make_config(4, group=128, n_layers=2)
    assert w.seq == 64 and len(w.layers) == 2 and w.layers[0].group == 128
    rw = w.layers[0].rms_weight
    assert rw.min() >= 0.5 and rw.max() <= 2.0


def test_config3_zipf_skew():
    """Zipf(1.1) popularity: the top expert gets > 1000 of 4096 tokens, the
    tail almost nothing, and popularity falls with expert rank."""
    w = synth.make_config(3)
    L = w.layers[0]
    ids, _ = O.moe_gate(w.x, L.router_bf16, L.top_k)
    counts = np.bincount(ids.ravel(), minlength=64)
    assert counts.max() > 1000
    assert counts[:8].sum() > counts[32:].sum() * 4
    assert np.corrcoef(np.arange(64), counts)[0, 1] < -0.5


def test_config1_ragged_groups():
    w = synth.make_config(1)
    L = w.layers[0]
    ids, _ = O.moe_gate(w.x, L.router_bf16, L.top_k)
    counts = np.bincount(ids.ravel(), minlength=64)
    assert counts.sum() == 96 and counts.max() <= 16
    assert 30 <= (counts > 0).sum() <= 64  # ragged groups of 0..16 tokens
