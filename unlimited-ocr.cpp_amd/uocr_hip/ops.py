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


class RefInt4Table:
    """Per-expert INT4 tables in the reference's device layout
    (GpuDecoder::upload_expert_table, src/engine/gpu_decoder.cu:316-358):
    packed [E, rows, ceil(cols/2)] u8, scales / zeros [E, rows, ng] f32."""

    def __init__(self, qmats, device):
        import numpy as np
        import torch
        q0 = qmats[0]
        self.rows, self.cols, self.group = q0.rows, q0.cols, q0.group
        self.ng = (q0.cols + q0.group - 1) // q0.group
        self.packed = torch.from_numpy(np.stack([q.packed for q in qmats])).to(device)
        self.scales = torch.from_numpy(np.stack([q.scales for q in qmats]).astype(np.float32)).to(device)
        self.zeros = torch.from_numpy(np.stack([q.zeros for q in qmats]).astype(np.float32)).to(device)
        self.pstride = self.rows * ((self.cols + 1) // 2)
        self.sstride = self.rows * self.ng

    def args(self):
        return [self.packed.data_ptr(), self.scales.data_ptr(), self.zeros.data_ptr(),
                self.pstride, self.sstride, self.ng]


def moe_grouped_gate_up_int4(x, gate, up, assign_token, count, cap, act, bn=16, bm=64, stream=None):
    """Mirror of uocr::cuda::moe_grouped_gate_up_int4 (cuda_ops.h:170-175)."""
    E = gate.packed.shape[0]
    check(load().uocr_hip_moe_grouped_gate_up_int4(
        x.data_ptr(), *gate.args(), *up.args(), assign_token.data_ptr(), count.data_ptr(), E, cap,
        gate.cols, gate.rows, gate.group, act.data_ptr(), bn, bm, _stream(stream)))


def moe_grouped_down_int4(act, down, assign_token, assign_w, count, cap, out, bn=16, bm=64, stream=None):
    """Mirror of uocr::cuda::moe_grouped_down_int4 (cuda_ops.h:177-181)."""
    E = down.packed.shape[0]
    check(load().uocr_hip_moe_grouped_down_int4(
        act.data_ptr(), *down.args(), assign_token.data_ptr(), assign_w.data_ptr(), count.data_ptr(), E, cap,
        down.rows, down.cols, down.group, out.data_ptr(), bn, bm, _stream(stream)))


def moe_experts_masked_int4(x, gate, up, down, assign_token, assign_w, count, cap, act, out, stream=None):
    """Mirror of uocr::cuda::moe_experts_masked_int4 (cuda_ops.h:145-155)."""
    E = gate.packed.shape[0]
    check(load().uocr_hip_moe_experts_masked_int4(
        x.data_ptr(), x.shape[0], *gate.args(), *up.args(), *down.args(), assign_token.data_ptr(),
        assign_w.data_ptr(), count.data_ptr(), E, cap, gate.cols, gate.rows, gate.group, act.data_ptr(),
        out.data_ptr(), _stream(stream)))


def _ptr_array(mats, device, stream=None):
    """Device table of the matrices' pointers. Its upload is ordered on torch's
    current stream; a launch on another `stream` first waits for that copy.
    The caller keeps the returned tensor alive until the launch has run."""
    import torch
    t = torch.tensor([m.data_ptr() for m in mats], dtype=torch.int64, device=device)
    if stream is not None:
        torch.cuda.current_stream(device).synchronize()
    return t


def moe_experts_masked(x, gate_w, up_w, down_w, assign_token, assign_w, count, cap, act, out, stream=None):
    """Mirror of uocr::cuda::moe_experts_masked (cuda_ops.h:139-143). gate_w /
    up_w / down_w: lists of per-expert bf16 device tensors."""
    dev = x.device
    pg, pu, pd = _ptr_array(gate_w, dev, stream), _ptr_array(up_w, dev, stream), _ptr_array(down_w, dev, stream)
    inter, hidden = gate_w[0].shape
    check(load().uocr_hip_moe_experts_masked(
        x.data_ptr(), x.shape[0], pg.data_ptr(), pu.data_ptr(), pd.data_ptr(), assign_token.data_ptr(),
        assign_w.data_ptr(), count.data_ptr(), len(gate_w), cap, hidden, inter, act.data_ptr(), out.data_ptr(),
        _stream(stream)))
    return pg, pu, pd  # keep alive until the stream has run


def moe_grouped_gate_up_bf16(x, gate_w, up_w, assign_token, count, cap, act, bn=16, bm=64, stream=None):
    """Mirror of uocr::cuda::moe_grouped_gate_up_bf16 (cuda_ops.h:192-195)."""
    dev = x.device
    pg, pu = _ptr_array(gate_w, dev, stream), _ptr_array(up_w, dev, stream)
    inter, hidden = gate_w[0].shape
    check(load().uocr_hip_moe_grouped_gate_up_bf16(
        x.data_ptr(), pg.data_ptr(), pu.data_ptr(), assign_token.data_ptr(), count.data_ptr(), len(gate_w), cap,
        hidden, inter, act.data_ptr(), bn, bm, _stream(stream)))
    return pg, pu


def moe_grouped_down_bf16(act, down_w, assign_token, assign_w, count, cap, out, bn=16, bm=64, stream=None):
    """Mirror of uocr::cuda::moe_grouped_down_bf16 (cuda_ops.h:197-200)."""
    dev = act.device
    pd = _ptr_array(down_w, dev, stream)
    hidden, inter = down_w[0].shape
    check(load().uocr_hip_moe_grouped_down_bf16(
        act.data_ptr(), pd.data_ptr(), assign_token.data_ptr(), assign_w.data_ptr(), count.data_ptr(), len(down_w),
        cap, hidden, inter, out.data_ptr(), bn, bm, _stream(stream)))
    return pd


def moe_gemm_int4(x, packed, scales, zeros, n, k, group, y, variant="", stream=None):
    """Mirror of uocr::cuda::moe_gemm_int4 and its _tc* variants (cuda_ops.h:204-239)."""
    lib = load()
    m = x.shape[0]
    base = [x.data_ptr(), packed.data_ptr(), scales.data_ptr(), zeros.data_ptr(), m, n, k, group, y.data_ptr()]
    if variant in ("", "_tc"):
        rc = getattr(lib, "uocr_hip_moe_gemm_int4" + variant)(*base, _stream(stream))
    elif variant in ("_tc_n", "_tc_pipe"):
        rc = getattr(lib, "uocr_hip_moe_gemm_int4" + variant)(*base, 16, _stream(stream))
    else:
        rc = lib.uocr_hip_moe_gemm_int4_tc_nk(*base, 16, 64, _stream(stream))
    check(rc)


def matmul_t_bf16(x, w_bits, y, bias=None, stream=None):
    """Mirror of uocr::cuda::matmul_t_bf16 (cuda_ops.h:31-32): y = x . W^T + bias,
    W bf16 bits (int16/uint16 tensor [n, k])."""
    m, k = x.shape
    n = w_bits.shape[0]
    check(load().uocr_hip_matmul_t_bf16(x.data_ptr(), w_bits.data_ptr(), bias.data_ptr() if bias is not None else None,
                                        y.data_ptr(), m, n, k, _stream(stream)))


def matvec_bf16(x, w_bits, y, bias=None, stream=None):
    """Mirror of uocr::cuda::matvec_bf16 (cuda_ops.h:41-42)."""
    n, k = w_bits.shape
    check(load().uocr_hip_matvec_bf16(x.data_ptr(), w_bits.data_ptr(), bias.data_ptr() if bias is not None else None,
                                      y.data_ptr(), n, k, _stream(stream)))


def silu_mul(gate, up, out, stream=None):
    """Mirror of uocr::cuda::silu_mul (cuda_ops.h:242-243)."""
    check(load().uocr_hip_silu_mul(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(), _stream(stream)))


def add_scaled(dst, src, scale, stream=None):
    """Mirror of uocr::cuda::add_scaled (cuda_ops.h:245-246)."""
    check(load().uocr_hip_add_scaled(dst.data_ptr(), src.data_ptr(), float(scale), dst.numel(), _stream(stream)))


def scatter_add_scaled(out, vals, row_idx, weights, stream=None):
    """Mirror of uocr::cuda::scatter_add_scaled (cuda_ops.h:248-250)."""
    rows, cols = vals.shape
    check(load().uocr_hip_scatter_add_scaled(out.data_ptr(), vals.data_ptr(), row_idx.data_ptr(), weights.data_ptr(),
                                             rows, cols, _stream(stream)))


def gather_rows(dst, src, row_idx, stream=None):
    """Mirror of uocr::cuda::gather_rows (cuda_ops.h:252-253)."""
    rows, cols = dst.shape
    check(load().uocr_hip_gather_rows(dst.data_ptr(), src.data_ptr(), row_idx.data_ptr(), rows, cols,
                                      _stream(stream)))
