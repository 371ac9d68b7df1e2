"""Shared test helpers: tolerances and metrics of the parity contract."""
import numpy as np

# outputs within rel_l2 <= 5e-3 and max-abs <= 2e-2 of the
# reference CPU path; routing ids (and here also weights) bit-exact.
REL_L2_TOL = 5e-3
MAX_ABS_TOL = 2e-2


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def subsample(ids, seq, n, seed=7):
    """Seeded token subsample that always includes tokens routed to the most
    and the least loaded experts (BASELINE.md CPU-baseline plan)."""
    if seq <= n:
        return np.arange(seq, dtype=np.int32)
    counts = np.bincount(ids.ravel(), minlength=ids.max() + 1)
    live = np.nonzero(counts)[0]
    most, least = live[np.argmax(counts[live])], live[np.argmin(counts[live])]
    must = {int(np.nonzero((ids == most).any(1))[0][0]), int(np.nonzero((ids == least).any(1))[0][0])}
    rng = np.random.default_rng(seed)
    rest = [t for t in rng.permutation(seq) if t not in must][: n - len(must)]
    return np.array(sorted(must | set(int(t) for t in rest)), dtype=np.int32)


def awq_layer(seed, group=32, n_experts=16, top_k=6, n_shared=2, hidden=1280, inter=896,
              router_bias=None, quantizer="awq"):
    """A layer whose experts come from the reference's own quantizer
    (quantize_int4_awq, src/runtime/quant.cpp:39-80, via the pinned oracle):
    f32 weights ~N(0, 0.02) with a per-row offset, so zeros span [0, 15] and
    scales are arbitrary f32 values (not bf16-valued)."""
    import oracle as O
    from uocr_hip import synth

    rng = np.random.default_rng(seed)
    fn = O.quantize_int4_awq if quantizer == "awq" else O.quantize_int4_symmetric

    def qm(rows, cols):
        w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
        w += (rng.standard_normal((rows, 1), dtype=np.float32) * np.float32(0.015))
        packed, scales, zeros = fn(w, group)
        return synth.QMat(packed, scales, zeros, rows, cols, group)

    router = rng.standard_normal((n_experts, hidden), dtype=np.float32) * np.float32(0.02)
    if router_bias is not None:
        router[:, 0] = np.asarray(router_bias, np.float32)
    L = synth.Layer(hidden, inter, n_experts, top_k, n_shared, group, synth.f32_to_bf16_bits(router), [], [], [])
    for _ in range(n_experts):
        L.gate.append(qm(inter, hidden))
        L.up.append(qm(inter, hidden))
        L.down.append(qm(hidden, inter))
    if n_shared:
        L.shared_gate = qm(n_shared * inter, hidden)
        L.shared_up = qm(n_shared * inter, hidden)
        L.shared_down = qm(hidden, n_shared * inter)
    return L
