"""GPU parity of the R-SWA mirrors against the oracle's RSWACache restatement
(itself pinned bit-exact to the reference build, tests/test_oracle_rswa.py).

Cache writes (append, batched append, ragged prefill scatter) and the ring
state must be bit-exact; attention outputs within 1e-4 abs (the reference's
own GPU test allows 1e-3, tests/test_rswa_cuda.cu:96, for its __expf kernel).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _t():
    import torch
    return torch


def dev_f32(a, dev):
    return _t().from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def dev_i32(a, dev):
    return _t().from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def lib():
    from uocr_hip import _lib
    return _lib.load()


def ok(rc):
    from uocr_hip._lib import check
    check(rc)


_alive = []  # device temporaries a queued kernel still reads


def ptr(t):
    _alive.append(t)
    if len(_alive) > 4096:
        _t().cuda.synchronize()
        del _alive[:-64]
    return C.c_void_p(t.data_ptr())


def rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("kv_heads,heads,hd", [(10, 10, 128), (2, 8, 64), (3, 6, 256), (4, 4, 96)])
def test_decode_append_ring_and_attention(dev, kv_heads, heads, hd):
    """The reference test's flow (test_rswa_cuda.cu:51-101) on the device cache:
    prefill P rows, then appends through the warmup -> ring transition with the
    device-side state, attention after each checkpoint."""
    torch = _t()
    print(f"[rswa] decode kv_heads={kv_heads} heads={heads} hd={hd}", flush=True)
    rng = np.random.default_rng(hd + heads)
    W, P = 32, 57
    st = kv_heads * hd
    ref = O.RswaCache(kv_heads, hd, W)
    ref.reset(P)
    pk, pv = rand(rng, P, st), rand(rng, P, st)
    ref.write_prefill(pk, pv, P)
    kc, vc = dev_f32(ref.k, dev), dev_f32(ref.v, dev)
    d_len = dev_i32([P], dev)
    d_ring = dev_i32([0], dev)
    out = torch.empty(heads * hd, dtype=torch.float32, device=dev)
    for i in range(W + 21):
        k, v = rand(rng, st), rand(rng, st)
        ref.append(k, v)
        ok(lib().uocr_hip_rswa_append_decode(ptr(dev_f32(k, dev)), ptr(dev_f32(v, dev)), ptr(kc), ptr(vc),
                                             ptr(d_len), ptr(d_ring), P, W, kv_heads, hd, None))
        if i in (W - 2, W - 1, W, W + 20):
            torch.cuda.synchronize()
            assert d_len.item() == ref.len.value and d_ring.item() == ref.ring_pos.value, i
            assert np.array_equal(kc.cpu().numpy(), ref.k) and np.array_equal(vc.cpu().numpy(), ref.v), i
            q = rand(rng, heads * hd)
            L = ref.len.value
            ok(lib().uocr_hip_rswa_attention_decode(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), L, heads, kv_heads, hd,
                                                    ptr(out), None))
            torch.cuda.synchronize()
            want = ref.attention(q, L - 1, heads, False)
            err = np.abs(out.cpu().numpy() - want).max()
            print(f"[rswa] step {i}: kv_len={L} max_err={err:.2e}", flush=True)
            assert err <= TOL


@pytest.mark.parametrize("hd,kv_heads,heads", [(128, 10, 10), (64, 2, 8)])
def test_causal_prefill_and_devlen(dev, hd, kv_heads, heads):
    torch = _t()
    rng = np.random.default_rng(7 + hd)
    cap, kv_len = 300, 260
    K, V = rand(rng, cap, kv_heads, hd), rand(rng, cap, kv_heads, hd)
    kc, vc = dev_f32(K, dev), dev_f32(V, dev)
    for seq, q_start, causal in ((260, 0, 1), (17, 243, 1), (9, 100, 0)):
        q = rand(rng, seq, heads, hd)
        out = torch.empty(seq * heads * hd, dtype=torch.float32, device=dev)
        ok(lib().uocr_hip_rswa_attention(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), kv_len, seq, q_start, heads,
                                         kv_heads, hd, causal, ptr(out), None))
        torch.cuda.synchronize()
        want = O.rswa_attention(q, K, V, kv_len, q_start, heads, kv_heads, hd, causal).ravel()
        assert np.abs(out.cpu().numpy() - want).max() <= TOL, (seq, q_start, causal)
        # devlen: the same with the length read on the device
        out.zero_()
        ok(lib().uocr_hip_rswa_attention_devlen(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), ptr(dev_i32([kv_len], dev)),
                                                seq, q_start, heads, kv_heads, hd, causal, ptr(out), None))
        torch.cuda.synchronize()
        assert np.abs(out.cpu().numpy() - want).max() <= TOL, ("devlen", seq, q_start, causal)


def test_empty_cache_gives_zeros(dev):
    torch = _t()
    heads, hd = 4, 64
    kc = torch.zeros(8 * heads * hd, dtype=torch.float32, device=dev)
    out = torch.full((heads * hd,), 7.0, dtype=torch.float32, device=dev)
    q = torch.ones(heads * hd, dtype=torch.float32, device=dev)
    ok(lib().uocr_hip_rswa_attention_decode(ptr(q), ptr(kc), ptr(kc), 0, heads, heads, hd, ptr(out), None))
    torch.cuda.synchronize()
    assert (out == 0).all()


def test_batched_append_and_attention(dev):
    """Requests in slots of a batched cache with their own prefill lengths;
    batched appends in a permuted slot order, through each slot's ring
    transition (rswa_attention.cu:385-424, 84-140)."""
    torch = _t()
    rng = np.random.default_rng(11)
    kv_heads, heads, hd, W = 10, 10, 128, 8
    P = [5, 30, 1, 17, 12]
    n, cap = len(P), max(P) + W
    st = kv_heads * hd
    refs = []
    kbase = np.zeros((n, cap, st), np.float32)
    vbase = np.zeros((n, cap, st), np.float32)
    for s in range(n):
        r = O.RswaCache(kv_heads, hd, W)
        r.reset(P[s])
        pk, pv = rand(rng, P[s], st), rand(rng, P[s], st)
        r.write_prefill(pk, pv, P[s])
        kbase[s, :P[s]], vbase[s, :P[s]] = pk, pv
        refs.append(r)
    kc, vc = dev_f32(kbase, dev), dev_f32(vbase, dev)
    d_len, d_ring, d_pre = dev_i32(P, dev), dev_i32([0] * n, dev), dev_i32(P, dev)
    for step in range(W + 6):
        slots = rng.permutation(n)[: 3 + step % 3]
        k, v = rand(rng, len(slots), st), rand(rng, len(slots), st)
        for b, s in enumerate(slots):
            refs[s].append(k[b], v[b])
        ok(lib().uocr_hip_rswa_append_decode_batch(ptr(dev_f32(k, dev)), ptr(dev_f32(v, dev)), ptr(kc), ptr(vc),
                                                   ptr(d_len), ptr(d_ring), ptr(d_pre), ptr(dev_i32(slots, dev)),
                                                   len(slots), cap, W, kv_heads, hd, None))
    torch.cuda.synchronize()
    kh, vh = kc.cpu().numpy(), vc.cpu().numpy()
    for s in range(n):
        assert d_len[s].item() == refs[s].len.value and d_ring[s].item() == refs[s].ring_pos.value, s
        assert np.array_equal(kh[s].ravel()[: refs[s].k.size], refs[s].k), s
        assert np.array_equal(vh[s].ravel()[: refs[s].v.size], refs[s].v), s
    slots = np.array([3, 0, 4, 1, 2, 0], np.int32)
    q = rand(rng, len(slots), heads, hd)
    out = torch.empty(q.size, dtype=torch.float32, device=dev)
    ok(lib().uocr_hip_rswa_attention_batch(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), ptr(d_len),
                                           ptr(dev_i32(slots, dev)), len(slots), cap, heads, kv_heads, hd, ptr(out),
                                           None))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(len(slots), heads * hd)
    for b, s in enumerate(slots):
        want = refs[s].attention(q[b], refs[s].len.value - 1, heads, False).ravel()
        assert np.abs(got[b] - want).max() <= TOL, b


def test_ragged_prefill_write_and_attention(dev):
    """Three requests packed back to back (gpu_decoder.cu:1044): scatter of the
    K/V rows into their slots, then causal attention per request."""
    torch = _t()
    rng = np.random.default_rng(13)
    kv_heads, heads, hd, cap = 4, 8, 128, 80
    lens = [5, 40, 17]
    slots = [2, 0, 1]
    st = kv_heads * hd
    d_slots = np.concatenate([[s] * n for s, n in zip(slots, lens)]).astype(np.int32)
    d_pos = np.concatenate([np.arange(n) for n in lens]).astype(np.int32)
    total = int(sum(lens))
    k, v, q = rand(rng, total, st), rand(rng, total, st), rand(rng, total, heads, hd)
    kc = torch.zeros(3 * cap * st, dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    ok(lib().uocr_hip_rswa_write_prefill_ragged(ptr(dev_f32(k, dev)), ptr(dev_f32(v, dev)), ptr(kc), ptr(vc),
                                                ptr(dev_i32(d_slots, dev)), ptr(dev_i32(d_pos, dev)), total, cap,
                                                kv_heads, hd, None))
    out = torch.empty(q.size, dtype=torch.float32, device=dev)
    ok(lib().uocr_hip_rswa_attention_ragged(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), ptr(dev_i32(d_slots, dev)),
                                            ptr(dev_i32(d_pos, dev)), total, cap, heads, kv_heads, hd, ptr(out), None))
    torch.cuda.synchronize()
    kh = kc.cpu().numpy().reshape(3, cap, st)
    vh = vc.cpu().numpy().reshape(3, cap, st)
    got = out.cpu().numpy().reshape(total, heads * hd)
    t0 = 0
    for s, n in zip(slots, lens):
        assert np.array_equal(kh[s, :n], k[t0:t0 + n]) and np.array_equal(vh[s, :n], v[t0:t0 + n])
        want = O.rswa_attention(q[t0:t0 + n], kh[s], vh[s], n, 0, heads, kv_heads, hd, True).reshape(n, -1)
        assert np.abs(got[t0:t0 + n] - want).max() <= TOL, s
        t0 += n


def test_rejects_unsupported_head_dim(dev):
    from uocr_hip._lib import HipError
    torch = _t()
    x = torch.zeros(64, dtype=torch.float32, device=dev)
    with pytest.raises(HipError, match="head_dim"):
        ok(lib().uocr_hip_rswa_attention_decode(ptr(x), ptr(x), ptr(x), 1, 1, 1, 6, ptr(x), None))


@pytest.mark.parametrize("kv_heads,heads,hd,kv_len", [(10, 10, 128, 1128), (3, 6, 256, 1000), (2, 8, 64, 700)])
def test_long_cache_key_split(dev, kv_heads, heads, hd, kv_len):
    """Decode rows over long caches: few (row, head) workgroups, so the keys
    are split over several workgroups and merged (flash-decoding); the
    single-cache, device-length and batched entry points against the oracle."""
    torch = _t()
    rng = np.random.default_rng(kv_len + hd)
    print(f"[rswa] key split kv_heads={kv_heads} heads={heads} hd={hd} kv_len={kv_len}", flush=True)
    K, V = rand(rng, kv_len, kv_heads, hd), rand(rng, kv_len, kv_heads, hd)
    kc, vc = dev_f32(K, dev), dev_f32(V, dev)
    q = rand(rng, 1, heads, hd)
    want = O.rswa_attention(q, K, V, kv_len, 0, heads, kv_heads, hd, False).ravel()
    out = torch.empty(heads * hd, dtype=torch.float32, device=dev)
    ok(lib().uocr_hip_rswa_attention_decode(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), kv_len, heads, kv_heads, hd,
                                            ptr(out), None))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - want).max() <= TOL
    out.zero_()
    ok(lib().uocr_hip_rswa_attention_devlen(ptr(dev_f32(q, dev)), ptr(kc), ptr(vc), ptr(dev_i32([kv_len], dev)),
                                            1, kv_len - 1, heads, kv_heads, hd, 1, ptr(out), None))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - want).max() <= TOL
    # batched: slots of one cache array with lengths from 1 to the capacity
    lens = [kv_len, 1, kv_len // 3, kv_len - 5]
    n, st = len(lens), kv_heads * hd
    kb = rand(rng, n, kv_len, st)
    vb = rand(rng, n, kv_len, st)
    slots = np.array([2, 0, 3, 1, 0], np.int32)
    qb = rand(rng, len(slots), heads, hd)
    outb = torch.empty(qb.size, dtype=torch.float32, device=dev)
    ok(lib().uocr_hip_rswa_attention_batch(ptr(dev_f32(qb, dev)), ptr(dev_f32(kb, dev)), ptr(dev_f32(vb, dev)),
                                           ptr(dev_i32(lens, dev)), ptr(dev_i32(slots, dev)), len(slots), kv_len,
                                           heads, kv_heads, hd, ptr(outb), None))
    torch.cuda.synchronize()
    got = outb.cpu().numpy().reshape(len(slots), heads * hd)
    for b, s in enumerate(slots):
        Ks = kb[s].reshape(kv_len, kv_heads, hd)
        Vs = vb[s].reshape(kv_len, kv_heads, hd)
        wb = O.rswa_attention(qb[b:b + 1], Ks, Vs, lens[s], 0, heads, kv_heads, hd, False).ravel()
        assert np.abs(got[b] - wb).max() <= TOL, (b, s)
