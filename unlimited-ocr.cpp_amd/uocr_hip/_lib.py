"""ctypes loader and signatures for libuocr_hip.so."""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# UOCR_HIP_LIB overrides the in-tree library (used to compare builds)
_LIB_PATH = os.environ.get("UOCR_HIP_LIB") or os.path.join(os.path.dirname(_HERE), "lib", "libuocr_hip.so")
_lib = None

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
ENOMEM = -3
EWORKSPACE = -4
EHIP = -5
DTYPE_F32 = 0
DTYPE_BF16 = 1


class HipError(RuntimeError):
    """A libuocr_hip entry point returned a non-zero status."""

    def __init__(self, code, msg):
        super().__init__(f"libuocr_hip error {code}: {msg}")
        self.code = code


class QMatrixC(C.Structure):
    """uocr_hip_qmatrix (mirrors uocr::QuantizedMatrix, include/uocr/quant.h:16-32)."""

    _fields_ = [("packed", C.c_void_p), ("scales", C.c_void_p), ("zeros", C.c_void_p),
                ("rows", C.c_int), ("cols", C.c_int), ("group_size", C.c_int)]


class DenseMatrixC(C.Structure):
    """uocr_hip_dense_matrix (WeightMatrix BF16_EXT / F32, include/uocr/weights.h:18-46)."""

    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int)]


class LayerDescC(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
                ("top_k", C.c_int), ("n_shared", C.c_int), ("norm_topk_prob", C.c_int),
                ("routed_scaling_factor", C.c_float), ("scoring_sigmoid", C.c_int),
                ("router_bf16", C.c_void_p), ("gate", C.POINTER(QMatrixC)),
                ("up", C.POINTER(QMatrixC)), ("down", C.POINTER(QMatrixC)),
                ("shared_gate", C.POINTER(QMatrixC)), ("shared_up", C.POINTER(QMatrixC)),
                ("shared_down", C.POINTER(QMatrixC)), ("rms_weight", C.c_void_p),
                ("rms_eps", C.c_float), ("router_f32", C.c_void_p),
                ("shared_gate_w", C.POINTER(DenseMatrixC)), ("shared_up_w", C.POINTER(DenseMatrixC)),
                ("shared_down_w", C.POINTER(DenseMatrixC)), ("gate_w", C.POINTER(DenseMatrixC)),
                ("up_w", C.POINTER(DenseMatrixC)), ("down_w", C.POINTER(DenseMatrixC))]


def lib_path():
    return _LIB_PATH


# name -> (restype, argtypes); every entry is declared in include/uocr_hip/moe_capi.h
SIGNATURES = {
    "uocr_hip_last_error": (C.c_char_p, []),
    "uocr_hip_version": (C.c_char_p, []),
    "uocr_hip_moe_layer_create": (C.c_int, [C.POINTER(LayerDescC), C.POINTER(C.c_void_p)]),
    "uocr_hip_moe_layer_destroy": (C.c_int, [C.c_void_p]),
    "uocr_hip_moe_layer_device_bytes": (C.c_size_t, [C.c_void_p]),
    "uocr_hip_moe_layer_workspace_size": (C.c_size_t, [C.c_void_p, C.c_int]),
    "uocr_hip_moe_layer_path": (C.c_int, [C.c_void_p, C.c_int]),
    "uocr_hip_moe_layer_set_decode_kernel": (C.c_int, [C.c_void_p, C.c_int]),
    "uocr_hip_moe_layer_decode_kernel": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "uocr_hip_moe_layer_status": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int)]),
    "uocr_hip_moe_layer_status_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_router_overflow": (C.c_int, [C.c_int, C.POINTER(C.c_int)]),
    "uocr_hip_st_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "uocr_hip_st_close": (C.c_int, [C.c_void_p]),
    "uocr_hip_st_contains": (C.c_int, [C.c_void_p, C.c_char_p]),
    "uocr_hip_st_numel": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t)]),
    "uocr_hip_st_read_f32": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t]),
    "uocr_hip_st_read_u8": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t]),
    "uocr_hip_st_metadata": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "uocr_hip_gptq_group": (C.c_int, [C.c_void_p, C.c_int]),
    "uocr_hip_gptq_qmatrix": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int, C.c_int, C.c_int, C.POINTER(QMatrixC)]),
    "uocr_hip_fold_expert_input_scale": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "uocr_hip_scale_columns_f32": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "uocr_hip_rswa_attention_decode": (C.c_int, [C.c_void_p] * 3 + [C.c_int] * 4 + [C.c_void_p, C.c_void_p]),
    "uocr_hip_rswa_attention": (C.c_int, [C.c_void_p] * 3 + [C.c_int] * 7 + [C.c_void_p, C.c_void_p]),
    "uocr_hip_rswa_attention_devlen": (C.c_int, [C.c_void_p] * 4 + [C.c_int] * 6 + [C.c_void_p, C.c_void_p]),
    "uocr_hip_rswa_append_decode": (C.c_int, [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_void_p]),
    "uocr_hip_rswa_append_decode_batch": (C.c_int, [C.c_void_p] * 8 + [C.c_int] * 5 + [C.c_void_p]),
    "uocr_hip_rswa_attention_batch": (C.c_int, [C.c_void_p] * 5 + [C.c_int] * 5 + [C.c_void_p, C.c_void_p]),
    "uocr_hip_rswa_write_prefill_ragged": (C.c_int, [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_void_p]),
    "uocr_hip_rswa_attention_ragged": (C.c_int, [C.c_void_p] * 5 + [C.c_int] * 5 + [C.c_void_p, C.c_void_p]),
    "uocr_hip_fused_schedule_check": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.c_int]),
    "uocr_hip_moe_layer_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                              C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                              C.c_void_p]),
    "uocr_hip_moe_layer_forward_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                                      C.c_void_p, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_layer_set_timing": (C.c_int, [C.c_void_p, C.c_int]),
    "uocr_hip_moe_layer_read_timing": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int,
                                                  C.POINTER(C.c_int)]),
    "uocr_hip_moe_grouped_gate_up_int4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_grouped_down_int4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_experts_masked_int4": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_grouped_gate_up_bf16": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_grouped_down_bf16": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_experts_masked": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_gemm_int4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_gemm_int4_tc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "uocr_hip_moe_gemm_int4_tc_n": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    "uocr_hip_moe_gemm_int4_tc_nk": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_gemm_int4_tc_pipe": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    "uocr_hip_matmul_t_bf16": (C.c_int, [C.c_void_p] * 4 + [C.c_int] * 3 + [C.c_void_p]),
    "uocr_hip_matvec_bf16": (C.c_int, [C.c_void_p] * 4 + [C.c_int] * 2 + [C.c_void_p]),
    "uocr_hip_silu_mul": (C.c_int, [C.c_void_p] * 3 + [C.c_int, C.c_void_p]),
    "uocr_hip_add_scaled": (C.c_int, [C.c_void_p, C.c_void_p, C.c_float, C.c_int, C.c_void_p]),
    "uocr_hip_scatter_add_scaled": (C.c_int, [C.c_void_p] * 4 + [C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_gather_rows": (C.c_int, [C.c_void_p] * 3 + [C.c_int, C.c_int, C.c_void_p]),
    "uocr_hip_moe_router_topk": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                            C.c_float, C.c_int, C.c_void_p, C.c_void_p,
                                            C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                            C.c_void_p]),
}


def load():
    """Load libuocr_hip.so (built by __graft_entry__.build()); raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise FileNotFoundError(
            f"{_LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = C.CDLL(_LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    if rc != OK:
        raise HipError(rc, load().uocr_hip_last_error().decode())
    return rc
