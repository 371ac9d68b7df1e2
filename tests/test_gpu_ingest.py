"""GPU parity of layers built through the weight-ingest entry points.

A layer's routed experts go through a GPTQ-format safetensors file
(<weight>.packed / .scales / .zeros with the "uocr_int4" group metadata,
tools/reference/quantize_gptq.py:380-412) and back through
uocr_hip_gptq_qmatrix; the file's expert_in_scale is folded into the norm and
the router (weights.cpp:199-207), which makes the router f32. The f32 router
routes with the reference's uncontracted matmul_t chain (cpu_ops.cpp:11-24),
so routing ids and weights must stay bit-exact against the oracle; outputs
within the north_star tolerance.
"""
import json

import numpy as np
import pytest

from helpers import awq_layer
from test_gpu_layer import check_parity
from test_ingest import gptq_file

pytestmark = pytest.mark.gpu


def gptq_round_trip(tmp_path, L, layer_index, s=None):
    from uocr_hip import ingest
    mats = {}
    for e in range(L.n_experts):
        ep = f"model.layers.{layer_index}.mlp.experts.{e}."
        mats[ep + "gate_proj.weight"] = L.gate[e]
        mats[ep + "up_proj.weight"] = L.up[e]
        mats[ep + "down_proj.weight"] = L.down[e]
    extra = {}
    if s is not None:
        extra[f"model.layers.{layer_index}.expert_in_scale"] = ("F32", s.shape, s.astype(np.float32).tobytes())
    p = tmp_path / "experts_int4.safetensors"
    gptq_file(p, mats, L.group, extra)
    with ingest.SafetensorsFile(p) as f:
        assert json.loads(f.metadata("uocr_int4"))["group"] == L.group
        return ingest.load_moe_layer(f, layer_index, L, fallback_group=999)


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("seq", [1, 16, 100, 600])
def test_gptq_file_with_awq_fold(dev, tmp_path, group, seq):
    from uocr_hip import synth
    base = awq_layer(4000 + group, group=group, n_experts=64)
    rng = np.random.default_rng(group)
    base.rms_weight = rng.uniform(0.5, 2.0, base.hidden).astype(np.float32)
    s = rng.uniform(1 / 16, 16, base.hidden).astype(np.float32)
    L = gptq_round_trip(tmp_path, base, 7, s)
    assert L.router_f32 is not None and L.group == group
    np.testing.assert_array_equal(L.gate[3].packed, base.gate[3].packed)
    x = synth.bf16_normal(np.random.default_rng(seq), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, dtype="f32", label=f"gptq-awq-g{group}-t{seq}")


@pytest.mark.parametrize("seq", [16, 600])
def test_gptq_file_fold_into_bf16_shared_mlp(dev, tmp_path, seq):
    """The reference's real layer form: GPTQ INT4 routed experts from the file,
    a bf16 shared MLP from the checkpoint; the file's expert_in_scale turns the
    shared gate/up into F32 matrices (scale_columns, weights.cpp:185-207) and
    the router into f32, and the layer takes them as they are."""
    from uocr_hip import synth
    base = synth.with_bf16_shared(awq_layer(4500, group=32, n_experts=64), 4501)
    rng = np.random.default_rng(seq)
    base.rms_weight = rng.uniform(0.5, 2.0, base.hidden).astype(np.float32)
    s = rng.uniform(1 / 16, 16, base.hidden).astype(np.float32)
    L = gptq_round_trip(tmp_path, base, 3, s)
    assert L.shared_gate_w.data.dtype == np.float32 and L.shared_down_w.data.dtype == np.uint16
    np.testing.assert_array_equal(L.shared_gate_w.data, base.shared_gate_w.to_f32() * s[None, :])
    x = synth.bf16_normal(np.random.default_rng(seq + 3), (seq, L.hidden), 1.0)
    check_parity(L, x, dev, sample=32 if seq > 64 else None, dtype="f32", label=f"gptq-awq-bf16shared-t{seq}")


@pytest.mark.parametrize("seq", [16, 300])
def test_f32_router_bf16_input(dev, seq):
    """An f32 router with bf16 input and no norm: 16 tokens run the streamed
    kernel's f32-router instantiation (the fused kernel takes only a bf16
    router), 300 the grouped prefill path with the f32 chain."""
    from test_gpu_layer import run_layer
    from uocr_hip import MoELayerInt4, synth
    L = awq_layer(4300 + seq, group=32, n_experts=64)
    L.router_f32 = np.random.default_rng(seq).standard_normal((64, L.hidden)).astype(np.float32) * np.float32(0.03)
    x = synth.bf16_normal(np.random.default_rng(seq + 1), (seq, L.hidden), 1.0)
    layer = MoELayerInt4(L)
    if seq <= 16:
        assert layer.decode_kernel(seq, "bf16") == "stream"
    else:
        layer.set_timing(True)
        run_layer(layer, x, "bf16", dev)
        t, n = layer.read_timing()
        assert n == 1 and t["fused"] == 0.0 and t["router"] > 0.0, t
    layer.close()
    check_parity(L, x, dev, sample=32 if seq > 64 else None, label=f"f32router-bf16-t{seq}")
