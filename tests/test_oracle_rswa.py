"""Pins of the oracle's R-SWA restatement (oracle/moe_oracle.c orc_rswa_*).

Against the reference's own RSWACache (src/scheduler/kv_cache.cpp compiled
into oracle/_ref): cache contents, length and ring position after prefill
writes and appends across the warmup -> ring transition, and attention
outputs bit for bit (decode and causal prefill, GQA, head dims with and
without a head_dim % 4 tail). Independently of _ref: the ring's row placement
against a direct model of kv_cache.h's layout comment (reference region 0..P-1
fixed, ring P..P+W-1 circular), and attention against a float64 two-pass
softmax (test_kv_ring_buffer.cpp's naive form).
"""
import numpy as np
import pytest

import oracle as O


def rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def ref_cache(R, kv_heads, hd, W, P, prefill, steps):
    c = R.ref_rswa_new(kv_heads, hd, W)
    R.ref_rswa_reset(c, P)
    if prefill is not None:
        R.ref_rswa_write_prefill(c, prefill[0], prefill[1], prefill[0].shape[0])
    for k, v in steps:
        R.ref_rswa_append(c, k, v)
    return c


@pytest.mark.parametrize("kv_heads,heads,hd", [(10, 10, 128), (2, 8, 64), (1, 4, 6), (3, 3, 256), (2, 4, 96)])
def test_rswa_against_reference_build(kv_heads, heads, hd):
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(hd * 7 + heads)
    W, P = 16, 37
    st = kv_heads * hd
    pre = (rand(rng, P, st), rand(rng, P, st))
    steps = [(rand(rng, st), rand(rng, st)) for _ in range(W + 11)]  # warmup, then 11 ring overwrites
    c = ref_cache(R, kv_heads, hd, W, P, pre, [])
    mine = O.RswaCache(kv_heads, hd, W)
    mine.reset(P)
    mine.write_prefill(pre[0], pre[1], P)
    for i, (k, v) in enumerate(steps):
        R.ref_rswa_append(c, k, v)
        mine.append(k, v)
        assert R.ref_rswa_len(c) == mine.len.value and R.ref_rswa_ring_pos(c) == mine.ring_pos.value, i
        if i in (W - 2, W - 1, W, W + 10):
            K = np.empty(R.ref_rswa_capacity(c) * st, np.float32)
            V = np.empty_like(K)
            R.ref_rswa_copy_kv(c, K, V)
            np.testing.assert_array_equal(K, mine.k)
            np.testing.assert_array_equal(V, mine.v)
            kv_len = mine.len.value
            for seq, q_start, causal in ((1, kv_len - 1, 0), (4, kv_len - 9, 1), (3, 5, 1)):
                q = rand(rng, seq, heads * hd)
                a = np.empty_like(q)
                R.ref_rswa_attention(c, q, seq, q_start, a, heads, causal)
                b = mine.attention(q, q_start, heads, causal)
                np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    R.ref_rswa_free(c)


def test_ring_row_placement():
    """kv_cache.h: rows 0..P-1 fixed; decode rows grow to P+W, then row
    P + ring_pos is overwritten circularly."""
    kvh, hd, W, P = 1, 4, 5, 3
    c = O.RswaCache(kvh, hd, W)
    c.reset(P)
    c.write_prefill(np.full((P, hd), -1, np.float32), np.full((P, hd), -2, np.float32), P)
    expect = {r: -1.0 for r in range(P)}
    for i in range(3 * W + 2):
        c.append(np.full(hd, i, np.float32), np.full(hd, i, np.float32))
        row = P + i if i < W else P + (i - W) % W
        expect[row] = float(i)
        got = c.k.reshape(-1, hd)[:, 0]
        for r, val in expect.items():
            assert got[r] == val, (i, r)
        assert c.len.value == min(P + i + 1, P + W)


@pytest.mark.parametrize("kv_heads,heads,hd,causal", [(10, 10, 128, 0), (2, 8, 64, 1), (1, 2, 6, 1)])
def test_attention_against_two_pass_softmax_f64(kv_heads, heads, hd, causal):
    rng = np.random.default_rng(heads + hd)
    cap, kv_len, seq, q_start = 70, 61, 5, 50
    K = rand(rng, cap, kv_heads, hd)
    V = rand(rng, cap, kv_heads, hd)
    q = rand(rng, seq, heads, hd)
    out = O.rswa_attention(q, K, V, kv_len, q_start, heads, kv_heads, hd, causal).reshape(seq, heads, hd)
    g = heads // kv_heads
    for s in range(seq):
        lim = min(kv_len, q_start + s + 1) if causal else kv_len
        for h in range(heads):
            k = K[:lim, h // g].astype(np.float64)
            v = V[:lim, h // g].astype(np.float64)
            sc = k @ q[s, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            want = (p / p.sum()) @ v
            np.testing.assert_allclose(out[s, h], want, rtol=2e-5, atol=2e-6)
