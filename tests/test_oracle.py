"""CPU tests that pin the oracle (oracle/moe_oracle.c) before it is trusted.

Each check compares the restatement with something other than itself:
  * tests/golden/ref_vectors.npz -- outputs of the reference's own compiled
    CPU code (quant.cpp, cpu_ops.cpp; written by tests/golden/make_golden.py);
  * oracle/_ref/libuocr_ref.so directly, when it is built (this container);
  * the known answers of the reference's tests/test_moe_gate.cpp:9-63;
  * brute force: exact rational arithmetic for the INT4 matvec's FMA chain
    (src/runtime/weights.cpp:51-72), float64 bounds, stable argsort for the
    grouping (src/engine/gpu_decoder.cu:602-609), greedy top-k by sorting.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
from uocr_hip import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gv():
    return np.load(GOLD)  # allow_pickle defaults to False


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(bits(a), bits(b))


def qmat(packed, scales, zeros, rows, cols, group):
    return synth.QMat(np.ascontiguousarray(packed), np.ascontiguousarray(scales, np.float32),
                      np.ascontiguousarray(zeros, np.float32), int(rows), int(cols), int(group))


# ---------------------------------------------------------------- bf16 (common.h:49-64)
def test_bf16_roundtrip_exhaustive():
    h = np.arange(65536, dtype=np.uint32)
    f = (h << 16).view(np.float32)
    got = np.array([O.bf16_to_f32(int(x)) for x in h[::257]], np.float32)
    assert same_bits(got, f[::257])
    # every finite bf16 value converts back to itself
    fin = np.isfinite(f)
    back = synth.f32_to_bf16_bits(f[fin])
    assert np.array_equal(back, h[fin].astype(np.uint16))


def test_bf16_golden(gv):
    got = np.array([O.f32_to_bf16(float(x)) for x in gv["bf16_in"]], np.uint16)
    ref = gv["bf16_out"]
    nan = np.isnan(gv["bf16_in"])
    assert np.array_equal(got[~nan], ref[~nan])
    # NaN stays NaN (exponent all ones, non-zero mantissa)
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all(got[nan] & 0x7F)


# ---------------------------------------------------------------- quant.cpp
@pytest.mark.parametrize("name", ["a", "b", "c"])
def test_dequantize_golden(gv, name):
    rows, cols, group = gv[f"deq_{name}_shape"]
    q = qmat(gv[f"deq_{name}_packed"], gv[f"deq_{name}_scales"], gv[f"deq_{name}_zeros"], rows, cols, group)
    out = O.dequantize(q)
    assert same_bits(out, gv[f"deq_{name}_out"])
    # closed form a1: (nibble - zero) * scale, low nibble = even column
    assert same_bits(q.dequantize(), out)
    for r, c in [(0, 0), (rows - 1, cols - 1), (rows // 2, 1)]:
        assert same_bits(O.qmatrix_at(q, r, c), out[r, c])


@pytest.mark.parametrize("kind", ["qawq", "qsym"])
def test_quantize_golden(gv, kind):
    w = gv[f"{kind}_w"]
    _, _, group = gv[f"{kind}_shape"]
    fn = O.quantize_int4_awq if kind == "qawq" else O.quantize_int4_symmetric
    p, s, z = fn(w, int(group))
    assert np.array_equal(p, gv[f"{kind}_packed"])
    assert same_bits(s, gv[f"{kind}_scales"]) and same_bits(z, gv[f"{kind}_zeros"])
    if kind == "qsym":
        assert np.all(z == 8.0)  # the layout every BASELINE config uses


# ---------------------------------------------------------------- cpu_ops.cpp
def test_matmul_t_golden(gv):
    assert same_bits(O.matmul_t(gv["mmt_x"], gv["mmt_w"], gv["mmt_b"]), gv["mmt_y"])


def test_matmul_t_bf16_golden(gv):
    y = O.matmul_t_bf16(gv["mmb_x"], gv["mmb_w"])
    assert same_bits(y, gv["mmb_y"])
    # sanity against float64: a sequential f32 chain of 1280 terms
    w = synth.bf16_bits_to_f32(gv["mmb_w"]).astype(np.float64)
    exact = gv["mmb_x"].astype(np.float64) @ w.T
    assert np.max(np.abs(exact - y)) < 1e-4


def test_softmax_golden(gv):
    assert same_bits(O.softmax(gv["smx_in"]), gv["smx_out"])


def test_silu_mul_golden(gv):
    assert same_bits(O.silu_mul(gv["silu_g"], gv["silu_u"]), gv["silu_out"])


def test_rmsnorm_golden(gv):
    assert same_bits(O.rmsnorm(gv["rms_x"], gv["rms_w"], 1e-6), gv["rms_out"])


def test_mlp_dense_golden(gv):
    """Unquantised shared MLP (bf16 gate, f32 up, bf16 down): the reference's
    own matmul_t_bf16 / matmul_t / silu_mul composed (mlpd_* golden vectors)."""
    g, u, d = synth.Dense(gv["mlpd_gate"]), synth.Dense(gv["mlpd_up"]), synth.Dense(gv["mlpd_down"])
    assert same_bits(O.mlp_dense(g, u, d, gv["mlpd_x"]), gv["mlpd_out"])
    # each matrix dispatches on its own dtype (weights.cpp:51-60)
    assert same_bits(O.dense_matmul(g, gv["mlpd_x"]), O.matmul_t_bf16(gv["mlpd_x"], gv["mlpd_gate"]))
    assert same_bits(O.dense_matmul(u, gv["mlpd_x"]), O.matmul_t(gv["mlpd_x"], gv["mlpd_up"]))
    # and the whole chain against float64
    x = gv["mlpd_x"].astype(np.float64)
    a = x @ g.to_f32().astype(np.float64).T
    b = x @ u.to_f32().astype(np.float64).T
    ref = (a / (1 + np.exp(-a)) * b) @ d.to_f32().astype(np.float64).T
    assert np.max(np.abs(O.mlp_dense(g, u, d, gv["mlpd_x"]) - ref)) < 1e-5


def test_moe_layer_dense_float64_brute_force():
    """bf16 routed experts + bf16 shared MLP (the reference's default layer)
    against float64 arithmetic on the same matrices."""
    L = synth.random_layer_bf16(34, hidden=256, inter=128, n_experts=16, top_k=4, n_shared=2)
    x = synth.bf16_normal(np.random.default_rng(5), (4, 256), 1.0)
    ids, w, out = O.moe_layer(L, x)

    def mlp(g, u, d, v):
        a = v @ g.to_f32().astype(np.float64).T
        b = v @ u.to_f32().astype(np.float64).T
        return (a / (1 + np.exp(-a)) * b) @ d.to_f32().astype(np.float64).T

    xd = x.astype(np.float64)
    ref = mlp(L.shared_gate_w, L.shared_up_w, L.shared_down_w, xd)
    for t in range(4):
        for j in range(4):
            e = ids[t, j]
            ref[t] += w[t, j] * mlp(L.gate_w[e], L.up_w[e], L.down_w[e], xd[t:t + 1])[0]
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-5


def test_against_ref_library_when_built():
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (no reference tree here)")
    rng = np.random.default_rng(11)
    lg = rng.standard_normal((32, 64)).astype(np.float32) * np.float32(8)
    sm = lg.copy()
    R.ref_softmax(sm, 32, 64)
    assert same_bits(O.softmax(lg), sm)
    x = rng.standard_normal((5, 1280)).astype(np.float32)
    w = synth.f32_to_bf16_bits(rng.standard_normal((64, 1280)).astype(np.float32) * np.float32(0.02))
    y = np.empty((5, 64), np.float32)
    R.ref_matmul_t_bf16(x, w, None, y, 5, 64, 1280)
    assert same_bits(O.matmul_t_bf16(x, w), y)


# ---------------------------------------------------------------- INT4 matvec (weights.cpp:51-72)
def _f32_round(fr):
    """Round an exact rational to the nearest binary32 (ties to even)."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * float(np.float32(float(q * ulp)))


def test_matmul_int4_exact_chain():
    """acc = fma(x[c] * (q - z), s, acc), c ascending -- emulated exactly."""
    rng = np.random.default_rng(5)
    rows, cols, group = 4, 70, 32
    q = synth.random_qmat(rng, rows, cols, group, scale_std=0.05)
    q.zeros[:] = rng.integers(0, 16, q.zeros.shape).astype(np.float32)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    y = O.matmul_int4(q, x)
    for i in range(2):
        for r in range(rows):
            acc = 0.0
            for c in range(cols):
                byte = int(q.packed[r, c // 2])
                nib = (byte >> 4) if c & 1 else (byte & 15)
                g = c // group
                qz = float(np.float32(nib) - q.zeros[r, g])
                t = float(np.float32(x[i, c]) * np.float32(qz))
                acc = _f32_round(Fraction(t) * Fraction(float(q.scales[r, g])) + Fraction(acc))
            assert np.float32(acc) == y[i, r], (i, r, acc, y[i, r])


def test_matmul_int4_float64_bound():
    rng = np.random.default_rng(6)
    q = synth.random_qmat(rng, 96, 1280, 32)
    x = synth.bf16_normal(rng, (3, 1280), 1.0)
    y = O.matmul_int4(q, x).astype(np.float64)
    exact = x.astype(np.float64) @ q.dequantize().astype(np.float64).T
    assert np.max(np.abs(y - exact)) < 1e-4
    assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 1e-5


# ---------------------------------------------------------------- moe_gate (moe_decoder.cpp:245-289)
def test_moe_gate_known_answers():
    """tests/test_moe_gate.cpp:9-63 of the reference."""
    router = np.eye(4, dtype=np.float32) * np.float32(5)
    ids, w = O.moe_gate_f32router(np.array([[2.0, 0.1, 0.1, 0.1]], np.float32), router, 2, norm=1)
    assert ids[0, 0] == 0
    assert abs(w[0].sum() - 1.0) < 1e-4 and w[0, 0] > w[0, 1]
    ids, w = O.moe_gate_f32router(np.array([[1.0, 0, 0, 0]], np.float32), np.eye(4, dtype=np.float32),
                                  2, norm=0, scaling=2.0)
    assert abs(w[0, 0] - 0.4754 * 2.0) < 2e-3
    assert abs(w[0].sum() - 0.6503 * 2.0) < 2e-3
    assert ids[0, 0] == 0 and ids[0, 1] == 1  # ties among experts 1..3 go to the lowest index


def _greedy(p, k):
    order = sorted(range(len(p)), key=lambda e: (-p[e], e))
    return order[:k]


@pytest.mark.parametrize("norm,scaling,sigmoid", [(0, 1.0, 0), (1, 1.0, 0), (1, 2.5, 0), (0, 1.0, 1)])
def test_moe_gate_composition(norm, scaling, sigmoid):
    """logits = matmul_t_bf16 (pinned above), softmax (pinned), greedy top-k by sort."""
    rng = np.random.default_rng(7 + norm)
    x = synth.bf16_normal(rng, (40, 1280), 1.0)
    wr = synth.f32_to_bf16_bits(rng.standard_normal((64, 1280)).astype(np.float32) * np.float32(0.02))
    ids, w = O.moe_gate(x, wr, 6, norm=norm, scaling=scaling, sigmoid=sigmoid)
    logits = O.matmul_t_bf16(x, wr)
    if sigmoid:
        p = (np.float32(1) / (np.float32(1) + np.exp(-logits.astype(np.float64)).astype(np.float32)))
    else:
        p = O.softmax(logits)
    for t in range(40):
        sel = _greedy(list(p[t]), 6)
        assert list(ids[t]) == sel
        pv = p[t, sel].astype(np.float32)
        if norm:
            s = np.float32(0)
            for v in pv:
                s = np.float32(s + v)
            exp_w = (pv / np.float32(s + np.float32(1e-20))) * np.float32(scaling)
        else:
            exp_w = pv * np.float32(scaling)
        if sigmoid:  # sigmoid's exp comes from glibc, numpy's may differ by 1 ulp
            assert np.allclose(w[t], exp_w, rtol=1e-6, atol=0)
        else:
            assert same_bits(w[t], exp_w)


def test_moe_gate_ties_lowest_index():
    logits_src = np.zeros((1, 8), np.float32)
    ids, _ = O.moe_gate_f32router(logits_src, np.eye(8, dtype=np.float32), 3)
    assert list(ids[0]) == [0, 1, 2]
    x = np.array([[0.0, 1.0, 1.0, 0.5, 1.0, 0, 0, 0]], np.float32)
    ids, _ = O.moe_gate_f32router(x, np.eye(8, dtype=np.float32), 4)
    assert list(ids[0]) == [1, 2, 4, 3]


# ---------------------------------------------------------------- grouping (gpu_decoder.cu:602-609)
@pytest.mark.parametrize("seq,E,k", [(1, 64, 6), (16, 64, 6), (333, 64, 6), (50, 8, 2)])
def test_stable_group_brute_force(seq, E, k):
    rng = np.random.default_rng(seq)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(seq)]).astype(np.int32)
    counts, offs, perm = O.stable_group(ids, E)
    assert np.array_equal(counts, np.bincount(ids.ravel(), minlength=E))
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(counts)]))
    flat_tok = np.repeat(np.arange(seq), k)
    assert np.array_equal(perm, flat_tok[np.argsort(ids.ravel(), kind="stable")])
    # the reference's loop: for t, for j: e_tokens[ids[t, j]].push_back(t)
    lists = [[] for _ in range(E)]
    for t in range(seq):
        for j in range(k):
            lists[ids[t, j]].append(t)
    assert np.array_equal(perm, np.array(sum(lists, []), np.int32))


# ---------------------------------------------------------------- whole layer (moe_decoder.cpp:76-113)
def test_moe_layer_float64_brute_force():
    L = synth.random_layer(31, hidden=256, inter=128, n_experts=16, top_k=4, n_shared=2, group=32)
    rng = np.random.default_rng(2)
    x = synth.bf16_normal(rng, (5, 256), 1.0)
    ids, w, out = O.moe_layer(L, x)
    ids_g, w_g = O.moe_gate(x, L.router_bf16, 4)
    assert np.array_equal(ids, ids_g) and same_bits(w, w_g)

    def mlp(g, u, d, v):
        a = v @ g.dequantize().astype(np.float64).T
        b = v @ u.dequantize().astype(np.float64).T
        return (a / (1 + np.exp(-a)) * b) @ d.dequantize().astype(np.float64).T

    xd = x.astype(np.float64)
    ref = mlp(L.shared_gate, L.shared_up, L.shared_down, xd)
    for t in range(5):
        for j in range(4):
            e = ids[t, j]
            ref[t] += w[t, j] * mlp(L.gate[e], L.up[e], L.down[e], xd[t:t + 1])[0]
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-5


def test_moe_layer_rmsnorm_residual():
    """out = h + moe(rmsnorm(h)) (moe_decoder.cpp:166-179)."""
    L = synth.random_layer(32, hidden=256, inter=128, n_experts=8, top_k=2, n_shared=0, group=32, rms=True)
    rng = np.random.default_rng(3)
    h = synth.bf16_normal(rng, (3, 256), 1.0)
    _, _, out = O.moe_layer(L, h)
    xn = O.rmsnorm(h, L.rms_weight, L.rms_eps)
    L.rms_weight = None
    _, _, moe = O.moe_layer(L, xn)
    assert same_bits(out, h + moe)


def test_moe_layer_subsample_rows_match_full():
    L = synth.random_layer(33, hidden=256, inter=128, n_experts=16, top_k=4, n_shared=2, group=32)
    x = synth.bf16_normal(np.random.default_rng(4), (9, 256), 1.0)
    ids, w, full = O.moe_layer(L, x, threads=2)
    sel = np.array([0, 4, 8], np.int32)
    ids2, w2, part = O.moe_layer(L, x, sel=sel)
    assert np.array_equal(ids, ids2) and same_bits(part[sel], full[sel])
    assert np.isnan(part[1]).all()


def test_contraction_pattern_sweep_vs_ref():
    """The reference build (GCC -O3 -march=native) fuses only some products:
    matmul_t_bf16 is one fma chain, while matmul_t and rmsnorm's sum of squares
    are vectorised products added in order with a fused scalar tail of n % 4
    terms. Sweep every tail length against oracle/_ref."""
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (no reference tree here)")
    rng = np.random.default_rng(1)
    for k in list(range(1, 34)) + [1279, 1280, 1281, 1282, 1283]:
        x = rng.standard_normal((3, k)).astype(np.float32)
        w = rng.standard_normal((9, k)).astype(np.float32)
        y = np.empty((3, 9), np.float32)
        R.ref_matmul_t(x, w, None, y, 3, 9, k)
        assert same_bits(O.matmul_t(x, w), y), k
        wb = synth.f32_to_bf16_bits(w)
        R.ref_matmul_t_bf16(x, wb, None, y, 3, 9, k)
        assert same_bits(O.matmul_t_bf16(x, wb), y), k
        rw = rng.uniform(0.5, 2, k).astype(np.float32)
        o = np.empty_like(x)
        R.ref_rmsnorm(x, rw, o, 3, k, 1e-6)
        assert same_bits(O.rmsnorm(x, rw, 1e-6), o), k
