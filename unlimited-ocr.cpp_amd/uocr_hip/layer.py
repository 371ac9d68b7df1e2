"""MoELayerInt4: a device-resident INT4 MoE layer behind the C ABI."""
import ctypes as C

import numpy as np

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F32, DenseMatrixC, LayerDescC, QMatrixC, check, load

STAGES = ("router", "group", "gate_up", "down", "combine", "fused", "shared")


class QMatrix:
    """Keeps a reference-layout INT4 matrix alive and exposes its C view."""

    def __init__(self, qm):
        self.packed = np.ascontiguousarray(qm.packed, np.uint8)
        self.scales = np.ascontiguousarray(qm.scales, np.float32)
        self.zeros = np.ascontiguousarray(qm.zeros, np.float32)
        self.c = QMatrixC(self.packed.ctypes.data, self.scales.ctypes.data, self.zeros.ctypes.data,
                          qm.rows, qm.cols, qm.group)


def _qarray(qms):
    keep = [QMatrix(q) for q in qms]
    arr = (QMatrixC * len(keep))(*[k.c for k in keep])
    return arr, keep


def _darray(ds):
    """uocr_hip_dense_matrix array over synth.Dense-like objects (`data`:
    uint16 bf16 bits or float32, [rows, cols])."""
    keep = [np.ascontiguousarray(d.data) for d in ds]
    for a in keep:
        if a.dtype not in (np.uint16, np.float32):
            raise TypeError("dense matrices must be bf16 bits (uint16) or float32")
    arr = (DenseMatrixC * len(keep))(*[DenseMatrixC(a.ctypes.data, DTYPE_BF16 if a.dtype == np.uint16 else DTYPE_F32,
                                                    a.shape[0], a.shape[1]) for a in keep])
    return arr, keep


class MoELayerInt4:
    """Uploads a `synth.Layer`-like object (reference host layout: INT4
    QuantizedMatrix experts, or unquantised bf16/f32 experts and shared MLP)
    once, then runs `forward` on torch device tensors through
    uocr_hip_moe_layer_forward."""

    def __init__(self, L):
        lib = load()
        self.lib = lib
        keep = []
        gate = up = down = gw = uw = dw = None
        if getattr(L, "gate_w", None) is not None:  # unquantised routed experts
            gw, k1 = _darray(L.gate_w)
            uw, k2 = _darray(L.up_w)
            dw, k3 = _darray(L.down_w)
            keep += [gw, uw, dw, k1, k2, k3]
        else:
            gate, k1 = _qarray(L.gate)
            up, k2 = _qarray(L.up)
            down, k3 = _qarray(L.down)
            keep += [gate, up, down, k1, k2, k3]
        sg = su = sd = sgw = suw = sdw = None
        if L.n_shared and getattr(L, "shared_gate_w", None) is not None:  # unquantised shared MLP
            sgw, k4 = _darray([L.shared_gate_w])
            suw, k5 = _darray([L.shared_up_w])
            sdw, k6 = _darray([L.shared_down_w])
            keep += [sgw, suw, sdw, k4, k5, k6]
        elif L.n_shared:
            sg, k4 = _qarray([L.shared_gate])
            su, k5 = _qarray([L.shared_up])
            sd, k6 = _qarray([L.shared_down])
            keep += [sg, su, sd, k4, k5, k6]
        router = np.ascontiguousarray(L.router_bf16, np.uint16)
        keep.append(router)
        rms = None
        if L.rms_weight is not None:
            rms = np.ascontiguousarray(L.rms_weight, np.float32)
            keep.append(rms)
        rf = getattr(L, "router_f32", None)
        if rf is not None:
            rf = np.ascontiguousarray(rf, np.float32)
            keep.append(rf)
        d = LayerDescC(L.hidden, L.inter, L.n_experts, L.top_k, L.n_shared, L.norm_topk_prob,
                       L.routed_scaling_factor, L.scoring_sigmoid, router.ctypes.data,
                       gate, up, down, sg, su, sd, rms.ctypes.data if rms is not None else None,
                       L.rms_eps, rf.ctypes.data if rf is not None else None, sgw, suw, sdw, gw, uw, dw)
        h = C.c_void_p()
        check(lib.uocr_hip_moe_layer_create(C.byref(d), C.byref(h)))
        self.handle = h
        self.hidden, self.top_k, self.has_rms = L.hidden, L.top_k, L.rms_weight is not None
        del keep  # host copies are no longer needed once uploaded

    def close(self):
        if self.handle:
            self.lib.uocr_hip_moe_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_bytes(self):
        return self.lib.uocr_hip_moe_layer_device_bytes(self.handle)

    def workspace_size(self, seq):
        return self.lib.uocr_hip_moe_layer_workspace_size(self.handle, seq)

    def path(self, seq):
        return "prefill" if self.lib.uocr_hip_moe_layer_path(self.handle, seq) else "decode"

    DECODE_KERNELS = {"auto": 0, "stream": 1, "fused": 2, "four_launch": 3}

    def set_decode_kernel(self, kind):
        """Force the decode-path implementation ("auto", "stream", "fused",
        "four_launch"); a forced kernel that does not apply falls back to the
        four-launch path."""
        check(self.lib.uocr_hip_moe_layer_set_decode_kernel(self.handle, self.DECODE_KERNELS[kind]))

    def decode_kernel(self, seq, x_dtype="bf16"):
        """The decode kernel forward uses for `seq` tokens (None: prefill path)."""
        v = self.lib.uocr_hip_moe_layer_decode_kernel(self.handle, seq, DTYPE_BF16 if x_dtype == "bf16" else DTYPE_F32)
        return {1: "stream", 2: "fused", 3: "four_launch"}.get(v)

    def status(self, clear=True):
        """Sticky fault flags of the single-kernel decode path (bit 0: a wait
        between workgroups timed out; bit 1: an exact pick outside the
        candidate experts). Synchronises the device."""
        flags = C.c_int(0)
        check(self.lib.uocr_hip_moe_layer_status(self.handle, 1 if clear else 0, C.byref(flags)))
        return flags.value

    def status_async(self, d_flags, stream=None):
        """Copy the same flags into the device int32 tensor `d_flags`,
        stream-ordered, without waiting for the device."""
        import torch
        st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        check(self.lib.uocr_hip_moe_layer_status_async(self.handle, d_flags.data_ptr(), st))

    def alloc_workspace(self, seq, device="cuda"):
        import torch
        n = self.workspace_size(seq)
        return torch.empty(n + 256, dtype=torch.uint8, device=device)

    def forward(self, x, out, workspace, ids=None, weights=None, stream=None):
        """x: torch [seq, hidden] bf16 or f32 (cuda); out: torch f32 [seq, hidden]."""
        import torch
        seq = x.shape[0]
        dt = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
        if x.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError("x must be bf16 or f32")
        ws_ptr = (workspace.data_ptr() + 255) // 256 * 256
        ws_bytes = workspace.numel() - (ws_ptr - workspace.data_ptr())
        st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        check(self.lib.uocr_hip_moe_layer_forward(
            self.handle, x.data_ptr(), dt, seq, out.data_ptr(),
            ids.data_ptr() if ids is not None else None,
            weights.data_ptr() if weights is not None else None,
            ws_ptr, ws_bytes, st))

    def forward_noalloc(self, x, out, ids=None, weights=None, stream=None):
        """forward() on the library's device scratch (no workspace argument,
        no allocation; calls on one device must not overlap)."""
        import torch
        dt = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
        if x.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError("x must be bf16 or f32")
        st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        check(self.lib.uocr_hip_moe_layer_forward_noalloc(
            self.handle, x.data_ptr(), dt, x.shape[0], out.data_ptr(),
            ids.data_ptr() if ids is not None else None,
            weights.data_ptr() if weights is not None else None, st))

    def set_timing(self, enable):
        check(self.lib.uocr_hip_moe_layer_set_timing(self.handle, 1 if enable else 0))

    def read_timing(self):
        ms = (C.c_float * len(STAGES))()
        n = C.c_int()
        check(self.lib.uocr_hip_moe_layer_read_timing(self.handle, ms, len(STAGES), C.byref(n)))
        return dict(zip(STAGES, list(ms))), n.value


# the layer takes every expert format the reference loads (INT4, BF16, F32)
MoELayer = MoELayerInt4
