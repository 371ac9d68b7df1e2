"""Writes tests/golden/ref_vectors.npz: input/output vectors of the reference's
own CPU code for the INT4 MoE path, produced by oracle/_ref/libuocr_ref.so
(compiled by oracle/Makefile from the reference's src/runtime/quant.cpp and
src/kernels/cpu_ops.cpp with the reference's Release flags).

Run in a container that has the reference tree:  python tests/golden/make_golden.py
The fixture is data only (seeded inputs and the reference's outputs); the GPU
box and the CPU tests read it without the reference tree.

Vectors (reference file:line of the function that produced each output):
  bf16      include/uocr/common.h:49-64     f32 -> bf16 bits (RNE, NaN, inf, ties)
  deq_*     src/runtime/quant.cpp:12-37     dequantize, odd column counts, zeros != 8
  qawq_*    src/runtime/quant.cpp:39-80     quantize_int4_awq
  qsym_*    src/runtime/quant.cpp:82-116    quantize_int4_symmetric
  mmt_*     src/kernels/cpu_ops.cpp:11-24   matmul_t (f32 weights, bias)
  mmb_*     src/kernels/cpu_ops.cpp:26-39   matmul_t_bf16 at the router shape [64, 1280]
  smx_*     src/kernels/cpu_ops.cpp:93-106  softmax (router logits, large/small/equal rows)
  silu_*    src/kernels/cpu_ops.cpp:108-113 silu_mul
  rms_*     src/kernels/cpu_ops.cpp:58-67   rmsnorm (eps 1e-6)
  mlpd_*    src/engine/moe_decoder.cpp:45-60 mlp_forward on unquantised matrices: a bf16 gate
            (matmul_t_bf16), an f32 up (matmul_t: the AWQ-folded form, weights.cpp:185-207),
            silu_mul, a bf16 down -- the reference's own functions composed as
            WeightMatrix::matmul dispatches them (weights.cpp:51-60)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def f32_to_bf16_bits(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def main():
    import oracle as O
    O.build()
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libuocr_ref.so is missing (needs the reference tree)")
    rng = np.random.default_rng(20261201)
    v = {}

    f = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(3.0),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38], np.float32),
        # exact ties on the 16-bit boundary: low half 0x8000 with even / odd upper half
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], np.uint32).view(np.float32),
    ])
    v["bf16_in"] = f
    v["bf16_out"] = np.array([R.ref_f32_to_bf16(float(x)) for x in f], np.uint16)

    for name, rows, cols, group, zp8 in [("a", 7, 77, 32, False), ("b", 16, 256, 128, True),
                                         ("c", 5, 33, 32, False)]:
        pr = (cols + 1) // 2
        ng = (cols + group - 1) // group
        packed = rng.integers(0, 256, (rows, pr), dtype=np.uint8)
        scales = np.abs(rng.standard_normal((rows, ng)).astype(np.float32)) * np.float32(0.01)
        zeros = np.full((rows, ng), 8.0, np.float32) if zp8 else \
            rng.integers(0, 16, (rows, ng)).astype(np.float32)
        out = np.empty((rows, cols), np.float32)
        R.ref_dequantize(packed, scales, zeros, rows, cols, group, out)
        v.update({f"deq_{name}_packed": packed, f"deq_{name}_scales": scales,
                  f"deq_{name}_zeros": zeros, f"deq_{name}_shape": np.array([rows, cols, group]),
                  f"deq_{name}_out": out})

    for kind, fn in (("qawq", R.ref_quantize_awq), ("qsym", R.ref_quantize_symmetric)):
        rows, cols, group = 9, 160, 32
        w = rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.05)
        w[0, :32] = 0.0          # constant group (scale fallback)
        w[1, 32:64] = 0.25       # constant non-zero group
        pr, ng = (cols + 1) // 2, cols // group
        packed = np.empty((rows, pr), np.uint8)
        scales = np.empty((rows, ng), np.float32)
        zeros = np.empty((rows, ng), np.float32)
        fn(w, rows, cols, group, packed, scales, zeros)
        v.update({f"{kind}_w": w, f"{kind}_shape": np.array([rows, cols, group]),
                  f"{kind}_packed": packed, f"{kind}_scales": scales, f"{kind}_zeros": zeros})

    m, n, k = 3, 17, 300
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.1)
    b = rng.standard_normal(n).astype(np.float32)
    y = np.empty((m, n), np.float32)
    R.ref_matmul_t(x, w, b.ctypes.data, y, m, n, k)
    v.update(mmt_x=x, mmt_w=w, mmt_b=b, mmt_y=y)

    m, n, k = 8, 64, 1280
    x = (rng.standard_normal((m, k)).astype(np.float32))
    wb = f32_to_bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02))
    y = np.empty((m, n), np.float32)
    R.ref_matmul_t_bf16(x, wb, None, y, m, n, k)
    v.update(mmb_x=x, mmb_w=wb, mmb_y=y)

    lg = rng.standard_normal((6, 64)).astype(np.float32)
    lg[1] *= 40.0                   # wide range: many exp underflow candidates
    lg[2] = 0.5                     # all equal
    lg[3, :] = -1e4
    lg[3, 5] = 30.0                 # one dominant expert
    lg[4] *= 1e-3
    sm = lg.copy()
    R.ref_softmax(sm, sm.shape[0], sm.shape[1])
    v.update(smx_in=lg, smx_out=sm)

    g = rng.standard_normal(2000).astype(np.float32) * np.float32(4.0)
    u = rng.standard_normal(2000).astype(np.float32)
    o = np.empty_like(g)
    R.ref_silu_mul(g, u, o, g.size)
    v.update(silu_g=g, silu_u=u, silu_out=o)

    x = rng.standard_normal((4, 1280)).astype(np.float32)
    x[3] *= 1e-4
    wr = rng.uniform(0.5, 2.0, 1280).astype(np.float32)
    o = np.empty_like(x)
    R.ref_rmsnorm(x, wr, o, 4, 1280, 1e-6)
    v.update(rms_x=x, rms_w=wr, rms_out=o)

    m, H, I = 3, 128, 96
    x = rng.standard_normal((m, H)).astype(np.float32)
    gb = f32_to_bf16_bits(rng.standard_normal((I, H)).astype(np.float32) * np.float32(0.05))
    uf = rng.standard_normal((I, H)).astype(np.float32) * np.float32(0.05)
    db = f32_to_bf16_bits(rng.standard_normal((H, I)).astype(np.float32) * np.float32(0.05))
    gy, uy, act, out = (np.empty((m, I), np.float32), np.empty((m, I), np.float32),
                        np.empty((m, I), np.float32), np.empty((m, H), np.float32))
    R.ref_matmul_t_bf16(x, gb, None, gy, m, I, H)
    R.ref_matmul_t(x, uf, None, uy, m, I, H)
    R.ref_silu_mul(gy, uy, act, m * I)
    R.ref_matmul_t_bf16(act, db, None, out, m, H, I)
    v.update(mlpd_x=x, mlpd_gate=gb, mlpd_up=uf, mlpd_down=db, mlpd_out=out)

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **v)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
