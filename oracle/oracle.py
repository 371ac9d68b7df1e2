"""ctypes wrapper of the CPU oracle (liboracle.so) and of oracle/_ref.

TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, as the checker or the timed CPU
baseline. The product path (libuocr_hip) never touches it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libuocr_ref.so")
_lib = None
_ref = None

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


class QMatC(C.Structure):
    _fields_ = [("packed", C.c_void_p), ("scales", C.c_void_p), ("zeros", C.c_void_p),
                ("rows", C.c_int), ("cols", C.c_int), ("group_size", C.c_int)]


class DenseC(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int)]


class LayerC(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("shared_inter", C.c_int),
                ("n_experts", C.c_int), ("top_k", C.c_int), ("norm_topk_prob", C.c_int),
                ("routed_scaling_factor", C.c_float), ("scoring_sigmoid", C.c_int),
                ("router_bf16", C.c_void_p), ("gate", C.POINTER(QMatC)), ("up", C.POINTER(QMatC)),
                ("down", C.POINTER(QMatC)), ("shared_gate", QMatC), ("shared_up", QMatC),
                ("shared_down", QMatC), ("rms_weight", C.c_void_p), ("rms_eps", C.c_float),
                ("router_f32", C.c_void_p), ("shared_gate_w", DenseC), ("shared_up_w", DenseC),
                ("shared_down_w", DenseC), ("gate_w", C.POINTER(DenseC)), ("up_w", C.POINTER(DenseC)),
                ("down_w", C.POINTER(DenseC))]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_qmatrix_at.restype = C.c_float
        L.orc_qmatrix_at.argtypes = [C.POINTER(QMatC), C.c_int, C.c_int]
        L.orc_dequantize.argtypes = [C.POINTER(QMatC), f32p]
        for q in ("orc_quantize_int4_awq", "orc_quantize_int4_symmetric"):
            getattr(L, q).argtypes = [f32p, C.c_int, C.c_int, C.c_int, u8p, f32p, f32p]
        L.orc_matmul_int4.argtypes = [C.POINTER(QMatC), f32p, f32p, C.c_int]
        L.orc_matmul_t.argtypes = [f32p, f32p, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int]
        L.orc_matmul_t_bf16.argtypes = [f32p, u16p, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int]
        L.orc_softmax.argtypes = [f32p, C.c_int, C.c_int]
        L.orc_silu_mul.argtypes = [f32p, f32p, f32p, C.c_longlong]
        L.orc_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
        L.orc_fold_expert_input_scale.argtypes = [f32p, C.c_int, f32p, u16p, C.c_int, f32p]
        L.orc_scale_columns.argtypes = [f32p, C.c_int, C.c_int, f32p, f32p]
        L.orc_moe_gate.argtypes = [f32p, u16p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_float, C.c_int, i32p, f32p]
        L.orc_moe_gate_f32router.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                             C.c_int, C.c_float, C.c_int, i32p, f32p]
        L.orc_rswa_attention.argtypes = [f32p, f32p, f32p] + [C.c_int] * 7 + [f32p]
        L.orc_rswa_append.argtypes = [f32p, f32p, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int),
                                      C.c_int, C.c_int, C.c_int, f32p, f32p]
        L.orc_stable_group.argtypes = [i32p, C.c_int, C.c_int, C.c_int, i32p, i32p, i32p, C.c_void_p]
        L.orc_dense_matmul.argtypes = [C.POINTER(DenseC), f32p, f32p, C.c_int]
        L.orc_mlp_dense.argtypes = [C.POINTER(DenseC)] * 3 + [f32p, f32p, C.c_int]
        L.orc_moe_layer.argtypes = [C.POINTER(LayerC), f32p, C.c_int, C.c_void_p, C.c_int, C.c_int,
                                    i32p, f32p, f32p]
        _lib = L
    return _lib


def ref():
    """oracle/_ref/libuocr_ref.so (the reference's own quant.cpp + cpu_ops.cpp), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        R = C.CDLL(REF_LIB)
        R.ref_dequantize.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]
        R.ref_qat.restype = C.c_float
        R.ref_qat.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        for q in ("ref_quantize_awq", "ref_quantize_symmetric"):
            getattr(R, q).argtypes = [f32p, C.c_int, C.c_int, C.c_int, u8p, f32p, f32p]
        R.ref_matmul_t.argtypes = [f32p, f32p, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int]
        R.ref_matmul_t_bf16.argtypes = [f32p, u16p, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int]
        R.ref_softmax.argtypes = [f32p, C.c_int, C.c_int]
        R.ref_silu_mul.argtypes = [f32p, f32p, f32p, C.c_longlong]
        R.ref_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
        R.ref_f32_to_bf16.restype = C.c_uint16
        R.ref_f32_to_bf16.argtypes = [C.c_float]
        R.ref_bf16_to_f32.restype = C.c_float
        R.ref_bf16_to_f32.argtypes = [C.c_uint16]
        R.ref_rswa_new.restype = C.c_void_p
        R.ref_rswa_new.argtypes = [C.c_int, C.c_int, C.c_int]
        R.ref_rswa_free.argtypes = [C.c_void_p]
        R.ref_rswa_reset.argtypes = [C.c_void_p, C.c_int]
        R.ref_rswa_write_prefill.argtypes = [C.c_void_p, f32p, f32p, C.c_int]
        R.ref_rswa_append.argtypes = [C.c_void_p, f32p, f32p]
        for n in ("ref_rswa_len", "ref_rswa_ring_pos", "ref_rswa_capacity"):
            getattr(R, n).argtypes = [C.c_void_p]
        R.ref_rswa_copy_kv.argtypes = [C.c_void_p, f32p, f32p]
        R.ref_rswa_attention.argtypes = [C.c_void_p, f32p, C.c_int, C.c_int, f32p, C.c_int, C.c_int]
        _ref = R
    return _ref


def _qc(q, keep):
    p = np.ascontiguousarray(q.packed, np.uint8)
    s = np.ascontiguousarray(q.scales, np.float32)
    z = np.ascontiguousarray(q.zeros, np.float32)
    keep += [p, s, z]
    return QMatC(p.ctypes.data, s.ctypes.data, z.ctypes.data, q.rows, q.cols, q.group)


def qmat_c(q):
    keep = []
    return _qc(q, keep), keep


def dequantize(q):
    qc, keep = qmat_c(q)
    out = np.empty((q.rows, q.cols), np.float32)
    lib().orc_dequantize(C.byref(qc), out)
    return out


def matmul_int4(q, x):
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    qc, keep = qmat_c(q)
    y = np.empty((m, q.rows), np.float32)
    lib().orc_matmul_int4(C.byref(qc), x, y, m)
    return y


def moe_gate(x, router_bf16, top_k, norm=0, scaling=1.0, sigmoid=0):
    x = np.ascontiguousarray(x, np.float32)
    rows, hidden = x.shape
    E = router_bf16.shape[0]
    ids = np.empty((rows, top_k), np.int32)
    w = np.empty((rows, top_k), np.float32)
    lib().orc_moe_gate(x, np.ascontiguousarray(router_bf16, np.uint16), rows, hidden, E, top_k,
                       int(norm), float(scaling), int(sigmoid), ids, w)
    return ids, w


def moe_gate_f32router(x, router, top_k, norm=0, scaling=1.0, sigmoid=0):
    x = np.ascontiguousarray(x, np.float32)
    rows, hidden = x.shape
    E = router.shape[0]
    ids = np.empty((rows, top_k), np.int32)
    w = np.empty((rows, top_k), np.float32)
    lib().orc_moe_gate_f32router(x, np.ascontiguousarray(router, np.float32), rows, hidden, E,
                                 top_k, int(norm), float(scaling), int(sigmoid), ids, w)
    return ids, w


def stable_group(ids, n_experts):
    ids = np.ascontiguousarray(ids, np.int32)
    seq, k = ids.shape
    counts = np.empty(n_experts, np.int32)
    offs = np.empty(n_experts + 1, np.int32)
    perm = np.empty(seq * k, np.int32)
    lib().orc_stable_group(ids, seq, k, n_experts, counts, offs, perm, None)
    return counts, offs, perm


def rswa_attention(q, kcache, vcache, kv_len, q_start, heads, kv_heads, head_dim, causal):
    """RSWACache::attention (kv_cache.cpp:84-130) on an explicit cache
    [capacity, kv_heads, head_dim]; q [seq, heads, head_dim] -> out (same shape)."""
    q = np.ascontiguousarray(q, np.float32)
    seq = q.size // (heads * head_dim)
    out = np.empty_like(q)
    lib().orc_rswa_attention(q, np.ascontiguousarray(kcache, np.float32), np.ascontiguousarray(vcache, np.float32),
                             kv_len, seq, q_start, heads, kv_heads, head_dim, 1 if causal else 0, out)
    return out


class RswaCache:
    """One layer's R-SWA cache with the reference's host semantics
    (kv_cache.cpp:29-82): reset(P), write_prefill, append_decode."""

    def __init__(self, kv_heads, head_dim, window):
        self.kv_heads, self.head_dim, self.window = kv_heads, head_dim, window
        self.stride = kv_heads * head_dim

    def reset(self, prefill_len):
        self.prefill_len = prefill_len
        self.capacity = prefill_len + self.window
        self.k = np.zeros(self.capacity * self.stride, np.float32)
        self.v = np.zeros(self.capacity * self.stride, np.float32)
        self.len, self.ring_pos, self.ring_started = C.c_int(prefill_len), C.c_int(0), C.c_int(0)

    def write_prefill(self, k, v, seq):
        n = seq * self.stride
        self.k[:n] = np.asarray(k, np.float32).ravel()[:n]
        self.v[:n] = np.asarray(v, np.float32).ravel()[:n]
        self.len.value = seq
        self.prefill_len = seq

    def append(self, k, v):
        lib().orc_rswa_append(self.k, self.v, C.byref(self.len), C.byref(self.ring_pos), C.byref(self.ring_started),
                              self.prefill_len, self.window, self.stride,
                              np.ascontiguousarray(k, np.float32).ravel(), np.ascontiguousarray(v, np.float32).ravel())

    def attention(self, q, q_start, heads, causal):
        return rswa_attention(q, self.k, self.v, self.len.value, q_start, heads, self.kv_heads, self.head_dim, causal)


def fold_expert_input_scale(s, rms_weight, router_bf16):
    """weights.cpp:199-207 for the norm and the router: returns (rms_weight / s,
    f32 router with column c times s[c])."""
    s = np.ascontiguousarray(s, np.float32)
    rms = np.array(rms_weight, np.float32, copy=True)
    rb = np.ascontiguousarray(router_bf16, np.uint16)
    rf = np.empty(rb.shape, np.float32)
    lib().orc_fold_expert_input_scale(s, len(s), rms, rb, rb.shape[0], rf)
    return rms, rf


def scale_columns(w, s):
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(w)
    lib().orc_scale_columns(w, w.shape[0], w.shape[1], np.ascontiguousarray(s, np.float32), out)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(x, np.ascontiguousarray(w, np.float32), out, x.shape[0], x.shape[1], eps)
    return out


def _dc(d, keep):
    """orc_dense view of a synth.Dense (f32 or bf16-bits array)."""
    a = np.ascontiguousarray(d.data)
    keep.append(a)
    return DenseC(a.ctypes.data, 1 if a.dtype == np.uint16 else 0, a.shape[0], a.shape[1])


def dense_matmul(d, x):
    """WeightMatrix::matmul on an unquantised matrix (weights.cpp:51-60)."""
    keep = []
    dc = _dc(d, keep)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((x.shape[0], d.data.shape[0]), np.float32)
    lib().orc_dense_matmul(C.byref(dc), x, y, x.shape[0])
    return y


def mlp_dense(g, u, d, x):
    """mlp_forward (moe_decoder.cpp:45-60) on unquantised matrices."""
    keep = []
    gc, uc, dc = _dc(g, keep), _dc(u, keep), _dc(d, keep)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((x.shape[0], d.data.shape[0]), np.float32)
    lib().orc_mlp_dense(C.byref(gc), C.byref(uc), C.byref(dc), x, y, x.shape[0])
    return y


def layer_c(L):
    """orc_layer view of a synth.Layer (and the arrays it points into)."""
    keep = []
    E = L.n_experts
    dense_experts = getattr(L, "gate_w", None) is not None
    if dense_experts:
        gate = up = down = None
        gw = (DenseC * E)(*[_dc(m, keep) for m in L.gate_w])
        uw = (DenseC * E)(*[_dc(m, keep) for m in L.up_w])
        dw = (DenseC * E)(*[_dc(m, keep) for m in L.down_w])
        keep += [gw, uw, dw]
    else:
        gw = uw = dw = None
        gate = (QMatC * E)(*[_qc(q, keep) for q in L.gate])
        up = (QMatC * E)(*[_qc(q, keep) for q in L.up])
        down = (QMatC * E)(*[_qc(q, keep) for q in L.down])
        keep += [gate, up, down]
    empty = QMatC(None, None, None, 0, 0, 1)
    dempty = DenseC(None, 0, 0, 0)
    dense_shared = getattr(L, "shared_gate_w", None) is not None
    sg = _qc(L.shared_gate, keep) if L.n_shared and not dense_shared else empty
    su = _qc(L.shared_up, keep) if L.n_shared and not dense_shared else empty
    sd = _qc(L.shared_down, keep) if L.n_shared and not dense_shared else empty
    sgw = _dc(L.shared_gate_w, keep) if L.n_shared and dense_shared else dempty
    suw = _dc(L.shared_up_w, keep) if L.n_shared and dense_shared else dempty
    sdw = _dc(L.shared_down_w, keep) if L.n_shared and dense_shared else dempty
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
    lc = LayerC(L.hidden, L.inter, L.n_shared * L.inter, E, L.top_k, L.norm_topk_prob,
                L.routed_scaling_factor, L.scoring_sigmoid, router.ctypes.data, gate, up, down,
                sg, su, sd, rms.ctypes.data if rms is not None else None, L.rms_eps,
                rf.ctypes.data if rf is not None else None, sgw, suw, sdw, gw, uw, dw)
    return lc, keep


def moe_layer(L, h, sel=None, threads=1):
    """Reference CPU layer: routing for all rows, outputs for rows in `sel`
    (all rows when None). Returns ids, weights, out (unselected rows = NaN)."""
    h = np.ascontiguousarray(h, np.float32)
    seq = h.shape[0]
    lc, keep = layer_c(L)
    ids = np.empty((seq, L.top_k), np.int32)
    w = np.empty((seq, L.top_k), np.float32)
    out = np.full((seq, L.hidden), np.nan, np.float32)
    if sel is None:
        lib().orc_moe_layer(C.byref(lc), h, seq, None, 0, threads, ids, w, out)
    else:
        s = np.ascontiguousarray(sel, np.int32)
        lib().orc_moe_layer(C.byref(lc), h, seq, s.ctypes.data, len(s), threads, ids, w, out)
    return ids, w, out


def bf16_to_f32(h):
    return lib().orc_bf16_to_f32(int(h))


def f32_to_bf16(f):
    return lib().orc_f32_to_bf16(float(f))


def qmatrix_at(q, r, c):
    qc, keep = qmat_c(q)
    return lib().orc_qmatrix_at(C.byref(qc), r, c)


def _quantize(fn, w, group):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    ng = (cols + group - 1) // group
    packed = np.empty((rows, (cols + 1) // 2), np.uint8)
    scales = np.empty((rows, ng), np.float32)
    zeros = np.empty((rows, ng), np.float32)
    fn(w, rows, cols, group, packed, scales, zeros)
    return packed, scales, zeros


def quantize_int4_awq(w, group):
    return _quantize(lib().orc_quantize_int4_awq, w, group)


def quantize_int4_symmetric(w, group):
    return _quantize(lib().orc_quantize_int4_symmetric, w, group)


def matmul_t(x, w, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_matmul_t(x, w, None if b is None else b.ctypes.data, y, m, n, k)
    return y


def matmul_t_bf16(x, w_bits, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    m, k = x.shape
    n = w_bits.shape[0]
    y = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_matmul_t_bf16(x, w_bits, None if b is None else b.ctypes.data, y, m, n, k)
    return y


def softmax(x):
    y = np.array(x, np.float32, copy=True, order="C")
    lib().orc_softmax(y, y.shape[0], y.shape[1])
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    o = np.empty_like(g)
    lib().orc_silu_mul(g, u, o, g.size)
    return o
