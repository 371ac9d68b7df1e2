"""Weight ingest through the C-ABI (host only): safetensors files, pre-quantized
(GPTQ) INT4 expert matrices and the AWQ expert input-scale fold.

Mirrors DecoderWeights::load's MoE branch (src/runtime/weights.cpp:232-298):
`load_moe_layer` reads a layer's routed experts from the pre-quantized file
(make_quantized, weights.cpp:129-166) and, when the file holds
`model.layers.<i>.expert_in_scale`, folds it into the post-attention norm and
the router (apply_expert_input_scale, weights.cpp:199-207).
"""
import ctypes as C

import numpy as np

from ._lib import QMatrixC, check, load
from . import synth


class SafetensorsFile:
    """uocr::SafetensorsFile (src/runtime/safetensors.cpp) over uocr_hip_st_*."""

    def __init__(self, path):
        self.lib = load()
        h = C.c_void_p()
        check(self.lib.uocr_hip_st_open(str(path).encode(), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.uocr_hip_st_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def contains(self, name):
        return bool(self.lib.uocr_hip_st_contains(self.h, name.encode()))

    def numel(self, name):
        n = C.c_size_t()
        check(self.lib.uocr_hip_st_numel(self.h, name.encode(), C.byref(n)))
        return n.value

    def read_f32(self, name):
        out = np.empty(self.numel(name), np.float32)
        check(self.lib.uocr_hip_st_read_f32(self.h, name.encode(), out.ctypes.data, out.size))
        return out

    def read_u8(self, name):
        out = np.empty(self.numel(name), np.uint8)
        check(self.lib.uocr_hip_st_read_u8(self.h, name.encode(), out.ctypes.data, out.size))
        return out

    def metadata(self, key):
        v = C.c_char_p()
        check(self.lib.uocr_hip_st_metadata(self.h, key.encode(), C.byref(v)))
        return None if v.value is None else v.value.decode()

    def gptq_group(self, fallback):
        return self.lib.uocr_hip_gptq_group(self.h, fallback)

    def gptq_qmatrix(self, weight_name, rows, cols, fallback_group):
        """The pre-quantized matrix as a synth.QMat (copies of the file's arrays),
        or None when <weight_name>.packed is absent."""
        q = QMatrixC()
        rc = self.lib.uocr_hip_gptq_qmatrix(self.h, weight_name.encode(), rows, cols, fallback_group, C.byref(q))
        if rc == -6:  # UOCR_HIP_ENOTFOUND
            return None
        check(rc)
        g = q.group_size
        ng = (cols + g - 1) // g
        pk = np.ctypeslib.as_array(C.cast(q.packed, C.POINTER(C.c_uint8)), (rows * ((cols + 1) // 2),)).copy()
        sc = np.ctypeslib.as_array(C.cast(q.scales, C.POINTER(C.c_float)), (rows * ng,)).copy()
        zr = np.ctypeslib.as_array(C.cast(q.zeros, C.POINTER(C.c_float)), (rows * ng,)).copy()
        return synth.QMat(pk.reshape(rows, -1), sc.reshape(rows, ng), zr.reshape(rows, ng), rows, cols, g)


def fold_expert_input_scale(s, rms_weight, router_bf16):
    """apply_expert_input_scale (weights.cpp:199-207) for the norm and the router:
    returns (rms_weight / s, the f32 router with column c times s[c])."""
    lib = load()
    s = np.ascontiguousarray(s, np.float32)
    rms = np.array(rms_weight, np.float32, copy=True)
    rb = np.ascontiguousarray(router_bf16, np.uint16)
    rf = np.empty(rb.shape, np.float32)
    check(lib.uocr_hip_fold_expert_input_scale(s.ctypes.data, s.size, rms.ctypes.data, rb.ctypes.data,
                                               rb.shape[0], rf.ctypes.data))
    return rms, rf


def scale_columns_f32(w, s):
    """scale_columns (weights.cpp:185-197) on f32 values."""
    lib = load()
    w = np.ascontiguousarray(w, np.float32)
    s = np.ascontiguousarray(s, np.float32)
    out = np.empty_like(w)
    check(lib.uocr_hip_scale_columns_f32(w.ctypes.data, w.shape[0], w.shape[1], s.ctypes.data, out.ctypes.data))
    return out


def load_moe_layer(qfile, layer_index, base, fallback_group):
    """A synth.Layer for MoE layer `layer_index`: the non-expert tensors from
    `base` (a synth.Layer with router_bf16, shared experts, rms_weight, routing
    options), the routed experts' gate/up/down from the pre-quantized file
    `qfile` (SafetensorsFile), and the file's expert_in_scale folded in when
    present. Raises if a routed expert is missing from the file (this build
    does not quantize dense expert weights at load).

    The fold also scales the shared gate/up columns (weights.cpp:205-206). An
    unquantised shared MLP (`base.shared_gate_w` etc., the reference's form)
    takes it as the reference does: gate/up become F32 matrices with column c
    times s[c] (scale_columns, weights.cpp:185-197), down stays as it is. An
    INT4 shared MLP cannot absorb a column scale exactly, so for such a base
    `shared_gate` / `shared_up` must already be the folded ones: quantized from
    scale_columns_f32(dense shared weight, s)."""
    p = f"model.layers.{layer_index}."
    H, I, E = base.hidden, base.inter, base.n_experts
    gate, up, down = [], [], []
    for e in range(E):
        ep = f"{p}mlp.experts.{e}."
        mats = [qfile.gptq_qmatrix(ep + "gate_proj.weight", I, H, fallback_group),
                qfile.gptq_qmatrix(ep + "up_proj.weight", I, H, fallback_group),
                qfile.gptq_qmatrix(ep + "down_proj.weight", H, I, fallback_group)]
        if any(m is None for m in mats):
            raise KeyError(f"expert {e} of layer {layer_index} is not pre-quantized in the file")
        gate.append(mats[0])
        up.append(mats[1])
        down.append(mats[2])
    groups = {m.group for m in gate + up + down}
    L = synth.Layer(H, I, E, base.top_k, base.n_shared, groups.pop() if len(groups) == 1 else -1,
                    base.router_bf16, gate, up, down, base.shared_gate, base.shared_up, base.shared_down,
                    base.rms_weight, base.rms_eps, base.norm_topk_prob, base.routed_scaling_factor,
                    base.scoring_sigmoid)
    L.shared_gate_w, L.shared_up_w, L.shared_down_w = base.shared_gate_w, base.shared_up_w, base.shared_down_w
    skey = p + "expert_in_scale"
    if qfile.contains(skey):
        s = qfile.read_f32(skey)
        if s.size != H:
            raise ValueError("expert_in_scale size does not match hidden size")
        if base.rms_weight is None:
            raise ValueError("an expert input scale folds into the post-attention norm: rms_weight is required")
        L.rms_weight, L.router_f32 = fold_expert_input_scale(s, base.rms_weight, base.router_bf16)
        if L.shared_gate_w is not None:
            L.shared_gate_w = synth.Dense(scale_columns_f32(L.shared_gate_w.to_f32(), s))
            L.shared_up_w = synth.Dense(scale_columns_f32(L.shared_up_w.to_f32(), s))
    return L
