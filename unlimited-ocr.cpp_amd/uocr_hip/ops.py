"""Reference operator mirrors (include/uocr/cuda_ops.h) on torch device tensors."""
from ._lib import check, load


def _stream(stream):
    import torch
    return stream if stream is not None else torch.cuda.current_stream().cuda_stream


def moe_router_topk(logits, top_k, norm_topk_prob, routed_scaling_factor, scoring_sigmoid,
                    ids, weights, assign_token, assign_w, count, cap, stream=None):
    """Mirror of uocr::cuda::moe_router_topk (cuda_ops.h:125-131)."""
    seq, n_experts = logits.shape
    check(load().uocr_hip_moe_router_topk(
        logits.data_ptr(), seq, n_experts, top_k, int(norm_topk_prob), float(routed_scaling_factor),
        int(scoring_sigmoid), ids.data_ptr(), weights.data_ptr(), assign_token.data_ptr(),
        assign_w.data_ptr(), count.data_ptr(), cap, _stream(stream)))


def moe_router_overflow(clear=True):
    """Sticky count > cap flag of moe_router_topk (synchronises the device)."""
    import ctypes as C
    f = C.c_int(0)
    check(load().uocr_hip_moe_router_overflow(1 if clear else 0, C.byref(f)))
    return f.value
