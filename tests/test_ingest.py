"""CPU tests of the weight-ingest entry points (no device work).

The safetensors reader is checked against files written two ways: by the
`safetensors` package (the format's own writer) and by a byte-level writer
below that can produce what the package cannot (BF16 tensors, odd offsets,
malformed metadata). Conversions are checked against numpy (F16 -> f32 is
numpy's float16 widening; BF16 is the upper half of the f32 bits). The GPTQ
matrix entry follows make_quantized's pre-quantized branch
(src/runtime/weights.cpp:138-165): the group from the "uocr_int4" metadata,
element-count checks, and ENOTFOUND when <name>.packed is absent. The AWQ fold
(weights.cpp:185-207) is pinned to its closed form in numpy float32 (IEEE
division and multiplication, one rounding each) and to the oracle.
"""
import json
import struct

import numpy as np
import pytest

import oracle as O
from uocr_hip import ingest, synth
from uocr_hip._lib import HipError


def write_st(path, tensors, metadata=None, pad=0):
    """tensors: name -> (dtype string, shape, raw bytes). `pad` extra bytes
    before each tensor (misaligns the data on purpose)."""
    header, blob = {}, b""
    for name, (dt, shape, raw) in tensors.items():
        blob += b"\0" * pad
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(blob), len(blob) + len(raw)]}
        blob += raw
    if metadata is not None:
        header["__metadata__"] = metadata
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + blob)


def test_reader_against_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    t = {"a": rng.standard_normal((3, 5)).astype(np.float32),
         "b": rng.standard_normal(7).astype(np.float16),
         "c": rng.integers(-100, 100, (4, 2)).astype(np.int32),
         "d": rng.integers(0, 255, 9).astype(np.uint8),
         "e": rng.integers(-128, 127, 3).astype(np.int8)}
    p = tmp_path / "x.safetensors"
    save_file(t, str(p), metadata={"uocr_int4": json.dumps({"group": 64}), "format": "np"})
    with ingest.SafetensorsFile(p) as f:
        assert f.contains("a") and not f.contains("zz")
        np.testing.assert_array_equal(f.read_f32("a"), t["a"].ravel())
        np.testing.assert_array_equal(f.read_f32("b"), t["b"].astype(np.float32).ravel())
        np.testing.assert_array_equal(f.read_f32("c"), t["c"].astype(np.float32).ravel())
        np.testing.assert_array_equal(f.read_f32("e"), t["e"].astype(np.float32))
        np.testing.assert_array_equal(f.read_u8("d"), t["d"])
        np.testing.assert_array_equal(f.read_u8("e"), t["e"].view(np.uint8))
        assert f.metadata("format") == "np" and f.metadata("nope") is None
        assert f.gptq_group(32) == 64
        with pytest.raises(HipError):
            f.read_u8("a")  # read_u8 takes U8/I8 only (safetensors.cpp:131)


def test_reader_bf16_f16_special_values_and_misaligned_data(tmp_path):
    f16 = np.array([0.0, -0.0, 1.0, 65504.0, 6.1e-5, 5.96e-8, np.inf, -np.inf, np.nan], np.float16)
    bits = np.arange(0, 65536, 257, dtype=np.uint32).astype(np.uint16)  # bf16 patterns incl. subnormals, inf, nan
    f32 = np.array([1.5, -2.25, 3e-39], np.float32)
    p = tmp_path / "y.safetensors"
    write_st(p, {"h": ("F16", f16.shape, f16.tobytes()), "g": ("BF16", bits.shape, bits.tobytes()),
                 "f": ("F32", f32.shape, f32.tobytes())}, pad=3)
    with ingest.SafetensorsFile(p) as f:
        np.testing.assert_array_equal(f.read_f32("h").view(np.uint32), f16.astype(np.float32).view(np.uint32))
        want = (bits.astype(np.uint32) << 16)
        np.testing.assert_array_equal(f.read_f32("g").view(np.uint32), want)
        np.testing.assert_array_equal(f.read_f32("f"), f32)


@pytest.mark.parametrize("meta,expect", [
    (None, 32),                                    # no metadata: the caller's group
    ({"uocr_int4": json.dumps({"group": 128})}, 128),
    ({"uocr_int4": "not json"}, 32),               # unparsable: fallback (weights.cpp:149-151)
    ({"uocr_int4": json.dumps({"scheme": "x"})}, 32),
    ({"uocr_int4": json.dumps({"group": "64"})}, 32),  # a string: get<int>() throws, fallback
    ({"uocr_int4": json.dumps({"group": 128.0})}, 128),  # a float: get<int>() converts it
    ({"uocr_int4": json.dumps({"group": 64.9})}, 64),    # ... truncating toward zero
    ({"uocr_int4": json.dumps({"group": [64]})}, 32),    # an array: throws, fallback
])
def test_gptq_group_metadata(tmp_path, meta, expect):
    p = tmp_path / "m.safetensors"
    write_st(p, {"w.packed": ("U8", (1, 1), b"\x00")}, metadata=meta)
    with ingest.SafetensorsFile(p) as f:
        assert f.gptq_group(32) == expect


def test_shape_overflow_rejected_at_open(tmp_path):
    """A header shape whose element count wraps size_t is refused at open
    (EINVAL), not turned into a huge allocation at read time."""
    p = tmp_path / "bad.safetensors"
    write_st(p, {"w": ("F32", (1 << 40, 1 << 40), b"\0" * 16)})
    with pytest.raises(HipError, match="shape too large"):
        ingest.SafetensorsFile(p)
    write_st(p, {"w": ("F32", (1 << 31, 1 << 31, 1 << 3), b"\0" * 16)})
    with pytest.raises(HipError, match="shape too large"):
        ingest.SafetensorsFile(p)


def gptq_file(path, mats, group, extra=None):
    t = {}
    for name, q in mats.items():
        t[name + ".packed"] = ("U8", q.packed.shape, np.ascontiguousarray(q.packed).tobytes())
        t[name + ".scales"] = ("F32", q.scales.shape, np.ascontiguousarray(q.scales, np.float32).tobytes())
        t[name + ".zeros"] = ("F32", q.zeros.shape, np.ascontiguousarray(q.zeros, np.float32).tobytes())
    t.update(extra or {})
    write_st(path, t, metadata={"format": "pt", "uocr_int4": json.dumps({"group": group, "scheme": "gptq-asym"})})


def test_gptq_qmatrix_round_trip_and_checks(tmp_path):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((48, 200), dtype=np.float32) * np.float32(0.02)  # ragged: 200 % 64 != 0
    packed, scales, zeros = O.quantize_int4_awq(w, 64)
    q = synth.QMat(packed, scales, zeros, 48, 200, 64)
    p = tmp_path / "g.safetensors"
    gptq_file(p, {"m.weight": q}, 64)
    with ingest.SafetensorsFile(p) as f:
        r = f.gptq_qmatrix("m.weight", 48, 200, 32)  # the file's group wins over the fallback
        assert r.group == 64 and r.rows == 48 and r.cols == 200
        np.testing.assert_array_equal(r.packed, packed)
        np.testing.assert_array_equal(r.scales.view(np.uint32), scales.view(np.uint32))
        np.testing.assert_array_equal(r.zeros.view(np.uint32), zeros.view(np.uint32))
        assert f.gptq_qmatrix("absent.weight", 48, 200, 32) is None  # ENOTFOUND: caller quantizes
        with pytest.raises(HipError, match="packed shape mismatch"):
            f.gptq_qmatrix("m.weight", 48, 202, 32)
        with pytest.raises(HipError, match="packed shape mismatch"):
            f.gptq_qmatrix("m.weight", 47, 200, 32)


def test_gptq_scales_shape_mismatch(tmp_path):
    q = synth.QMat(np.zeros((4, 64), np.uint8), np.ones((4, 3), np.float32), np.zeros((4, 3), np.float32), 4, 128, 64)
    p = tmp_path / "s.safetensors"
    gptq_file(p, {"m.weight": q}, 64)  # 128 columns at group 64 need 2 groups, the file has 3
    with ingest.SafetensorsFile(p) as f:
        with pytest.raises(HipError, match="scales/zeros shape mismatch"):
            f.gptq_qmatrix("m.weight", 4, 128, 64)


def test_malformed_files_are_rejected(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(HipError, match="header out of range"):
        ingest.SafetensorsFile(p)
    write_st(p, {"x": ("F64", (1,), b"\0" * 8)})
    with pytest.raises(HipError, match="dtype"):
        ingest.SafetensorsFile(p)
    h = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    p.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 16)
    with pytest.raises(HipError, match="beyond file end"):
        ingest.SafetensorsFile(p)
    h = b'{"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]'
    p.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 4)
    with pytest.raises(HipError, match="header"):
        ingest.SafetensorsFile(p)
    with pytest.raises(HipError, match="cannot open"):
        ingest.SafetensorsFile(tmp_path / "missing.safetensors")


def test_fold_closed_form_and_oracle():
    rng = np.random.default_rng(11)
    H, E = 1280, 64
    s = rng.uniform(1 / 16, 16, H).astype(np.float32)  # the quantizer's clamp range (quantize_gptq.py:240)
    g = (1 + 0.01 * rng.standard_normal(H)).astype(np.float32)
    rb = synth.f32_to_bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02))
    rms, rf = ingest.fold_expert_input_scale(s, g, rb)
    # closed form: one IEEE float32 division / multiplication per element
    np.testing.assert_array_equal(rms.view(np.uint32), (g / s).view(np.uint32))
    want = (rb.astype(np.uint32) << 16).view(np.float32) * s[None, :]
    np.testing.assert_array_equal(rf.view(np.uint32), want.view(np.uint32))
    # the oracle's restatement gives the same bits
    rms_o, rf_o = O.fold_expert_input_scale(s, g, rb)
    np.testing.assert_array_equal(rms.view(np.uint32), rms_o.view(np.uint32))
    np.testing.assert_array_equal(rf.view(np.uint32), rf_o.view(np.uint32))
    w = rng.standard_normal((96, H), dtype=np.float32)
    np.testing.assert_array_equal(ingest.scale_columns_f32(w, s), w * s[None, :])
    np.testing.assert_array_equal(O.scale_columns(w, s), w * s[None, :])


def test_oracle_layer_routes_with_its_f32_router():
    """orc_moe_layer with router_f32 routes by matmul_t (the reference's
    uncontracted f32 chain, pinned against oracle/_ref) on the normed input."""
    from helpers import awq_layer
    L = awq_layer(5, group=64, n_experts=8, top_k=2, n_shared=1, hidden=256, inter=128)
    rng = np.random.default_rng(1)
    h = rng.standard_normal((6, 256)).astype(np.float32)
    L.rms_weight = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    L.router_f32 = rng.standard_normal((8, 256)).astype(np.float32) * np.float32(0.05)
    ids, w, _ = O.moe_layer(L, h)
    ids_g, w_g = O.moe_gate_f32router(O.rmsnorm(h, L.rms_weight, L.rms_eps), L.router_f32, 2)
    np.testing.assert_array_equal(ids, ids_g)
    np.testing.assert_array_equal(w.view(np.uint32), w_g.view(np.uint32))
