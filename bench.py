"""Benchmark: one Unlimited-OCR INT4 MoE layer on one MI355X.

Headline (`value`): BASELINE config 1 -- batched decode, 16 tokens, one INT4
g32 MoE layer (router + top-6 of 64 + 2 shared experts + combine) -- as
tokens/s with inputs and weights resident in HBM. Each timed step runs the layer
on the next of R distinct weight replicas, so the ~128 MB layer is streamed
from HBM rather than from the 256 MB Infinity Cache.

Roofline: the dominant kernel is the single-launch decode kernel (streamed
from 6 tokens, fused below; router, experts and combine in one launch;
algorithmic bytes = the layer's: touched experts' weights + shared expert +
router + activations), or, where that path does not apply, the gate/up expert
pass. Its average duration comes from HIP events stamped on that kernel's own dispatch
(hipExtLaunchKernelGGL start/stop events on the layer's stream, enabled by
uocr_hip_moe_layer_set_timing) over a second pass of the same steps;
achieved = algorithmic bytes per launch / that duration. traffic = HBM bytes per
launch from the committed rocprofv3 --pmc summary under profiles/.

Extra configs (0, 2, 3, 4) are reported under "configs" in the same line.
cpu_baseline: the CPU oracle (a restatement of the reference's CPU path) on the
host cores, bounded sample of config 1.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "unlimited-ocr.cpp_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16/f16


def layer_bytes(L, counts, seq):
    """Algorithmic HBM bytes of one layer call: every touched expert's weights
    once (INT4: packed nibbles + bf16-sized scales, zero point implicit; bf16:
    2 bytes per weight), the shared expert (INT4 or bf16), router, bf16 input
    and f32 output."""
    H, I, G = L.hidden, L.inter, L.group
    if getattr(L, "gate_w", None) is not None:
        gu_e, dn_e = 2 * I * H * 2, H * I * 2
    else:
        gu_e = 2 * (I * H // 2 + I * (H // G) * 2)
        dn_e = H * I // 2 + H * (I // G) * 2
    U = int((counts > 0).sum())
    S = L.n_shared
    if getattr(L, "shared_gate_w", None) is not None:
        shared_gu, shared_dn = S * 2 * I * H * 2, S * H * I * 2
    else:
        shared_gu, shared_dn = S * gu_e, S * dn_e
    io = seq * H * 2 + seq * H * 4 + L.n_experts * H * 2
    dense_shared = getattr(L, "shared_gate_w", None) is not None
    # an unquantised shared MLP runs in its own stage (dense.hip), an INT4 one
    # inside the routed passes
    return {"U": U, "gate_up": U * gu_e + (0 if dense_shared else shared_gu) + seq * H * 2,
            "down": U * dn_e + (0 if dense_shared else shared_dn),
            "shared": shared_gu + shared_dn if dense_shared else 0,
            "total": U * (gu_e + dn_e) + shared_gu + shared_dn + io}


def layer_flops(L, seq):
    H, I = L.hidden, L.inter
    per_tok = L.top_k * 3 * 2 * I * H + 3 * 2 * (L.n_shared * I) * H + 2 * L.n_experts * H
    return seq * per_tok, seq * (L.top_k + L.n_shared) * 2 * 2 * I * H


FORMATS = {
    "int4": "INT4 routed experts and INT4 shared MLP (BASELINE's synthetic layer)",
    "bf16_shared": "INT4 routed experts, bf16 shared MLP (the reference's real INT4 layer: "
                   "weights.cpp:289-292 keeps the shared MLP unquantised)",
    "bf16": "bf16 routed experts and bf16 shared MLP (the reference's default expert format, config.h:111)",
    "f32_input": "INT4 layer as int4, hidden states passed as f32 (the engine's normed2, gpu_decoder.cu:537-560)",
    "f32_router": "INT4 layer as int4 with an f32 router (the AWQ-folded router, weights.cpp:199-207: the bf16 "
                  "router times a per-column scale in [0.5, 2)), routed by the uncontracted f32 chain",
}


def make_layer(cfg, seed, group, fmt, bias=None, rms=False):
    from uocr_hip import synth
    if fmt == "bf16":
        return synth.random_layer_bf16(seed, router_bias=bias, rms=rms)
    L = synth.random_layer(seed, group=group, router_bias=bias, rms=rms)
    if fmt == "bf16_shared":
        synth.with_bf16_shared(L, seed + 1)
    if fmt == "f32_router":
        import numpy as np
        s = np.random.default_rng(seed + 2).uniform(0.5, 2.0, L.hidden).astype(np.float32)
        w = (L.router_bf16.astype(np.uint32) << 16).view(np.float32)
        L.router_f32 = (w * s[None, :]).astype(np.float32)
    return L


def run_config(cfg, steps, warmup, replicas, group=32, graph=False, fmt="int4"):
    import numpy as np
    import torch
    from uocr_hip import MoELayerInt4, synth

    dev = torch.device("cuda:0")
    if cfg == 4:
        wl = synth.make_config(4, group=group)
        if fmt != "int4":
            wl.layers = [make_layer(4, 1234 + 100 + i, group, fmt, rms=True) for i in range(len(wl.layers))]
        layers_np = wl.layers
        stack = True
    else:
        base = synth.make_config(cfg, group=group)
        bias = synth.zipf_bias() if cfg == 3 else None
        if fmt not in ("int4", "f32_input"):
            base.layers = [make_layer(cfg, 1234 + 10 + cfg, group, fmt, bias=bias)]
        layers_np = [base.layers[0]]
        for r in range(1, replicas):
            layers_np.append(make_layer(cfg, 9000 + 100 * cfg + r, group, fmt, bias=bias))
        wl = base
        stack = False
    seq = wl.seq
    layers = [MoELayerInt4(L) for L in layers_np]
    x = torch.from_numpy(wl.x).to(dev)
    x_f32 = stack or fmt == "f32_input"
    x_in = x.float() if x_f32 else x.to(torch.bfloat16)
    outs = [torch.empty(seq, wl.layers[0].hidden, dtype=torch.float32, device=dev) for _ in range(2)]
    ids = [torch.empty(seq, 6, dtype=torch.int32, device=dev) for _ in layers]
    wts = [torch.empty(seq, 6, dtype=torch.float32, device=dev) for _ in layers]
    ws = layers[0].alloc_workspace(seq, dev)

    def step(i):
        if stack:  # 12 layers: h <- h + moe(rmsnorm(h))
            h = x_in
            for li, lay in enumerate(layers):
                lay.forward(h, outs[li % 2], ws, ids[li], wts[li])
                h = outs[li % 2]
        else:
            li = i % len(layers)
            layers[li].forward(x_in, outs[0], ws, ids[li], wts[li])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    def timed(use_graph):
        """ms per step, eagerly launched or replayed from a hipGraph. A graph
        holds one call per weight replica (every replica once per replay, so the
        weights still stream from HBM, not from the memory-side cache)."""
        per = 1 if stack else len(layers)
        g = None
        if use_graph:
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for i in range(per):
                    step(i)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            with torch.cuda.graph(g):
                for i in range(per):
                    step(i)
            g.replay()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        n = max(1, steps // per) if g is not None else steps
        e0.record()
        for i in range(n):
            if g is not None:
                g.replay()
            else:
                step(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (n * per if g is not None else n)

    ms = timed(graph)
    ms_eager = ms if not graph else (timed(False) if not stack else None)

    # per-stage durations (HIP events around each launch), same step sequence
    # (stack: per layer call, over all layers)
    stage = None
    for lay in layers:
        lay.set_timing(True)
        lay.read_timing()
    tot = {}
    n = 0
    for i in range(steps):
        step(i)
        for lay in (layers if stack else [layers[i % len(layers)]]):
            st, c = lay.read_timing()
            for k, v in st.items():
                tot[k] = tot.get(k, 0.0) + v
            n += c
    for lay in layers:
        lay.set_timing(False)
    stage = {k: v / max(n, 1) for k, v in tot.items() if v > 0}

    torch.cuda.synchronize()
    counts = [np.bincount(t.cpu().numpy().ravel(), minlength=64) for t in ids]
    # one more call of replica 0 (the seeded layer the CPU leg checks): its
    # routing and outputs (stack: the 12-layer output and layer 0's routing)
    step(0)
    torch.cuda.synchronize()
    gpu_check = {"ids": ids[0].cpu().numpy(),
                 "out": outs[(len(layers) - 1) % 2 if stack else 0].cpu().numpy()}
    res = {"config": cfg, "workload": wl.name, "seq": seq, "group": group, "format": fmt,
           "format_note": FORMATS[fmt], "ms_per_step": ms, "graph": bool(graph)}
    if ms_eager is not None and graph:
        res["ms_per_step_eager"] = ms_eager
    if stack:
        tb = sum(layer_bytes(L, c, seq)["total"] for L, c in zip(layers_np, counts))
        res.update(tokens_per_s=seq / (ms * 1e-3), layers=len(layers), stage_ms=stage,
                   hbm_gbs=tb / (ms * 1e-3) / 1e9, hbm_frac=tb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
        if stage and "fused" in stage:
            # one single-launch decode call per layer: its bytes are the layer's
            kind = layers[0].decode_kernel(seq, "f32")
            res["decode_kernel"] = kind
            lb = tb / len(layers)
            res["dominant"] = {"kernel": f"decode_{kind}_kernel<{128 // group}, 10, 7, false, true> (wide mode, one per layer)",
                               "ms": stage["fused"], "bytes": lb, "gbs": lb / (stage["fused"] * 1e-3) / 1e9,
                               "traffic_file": f"decode_{kind}_config4_traffic.md" if group == 32 and fmt == "int4" else None,
                               "profile_file": "decode_layer_config4_kernel_stats.md" if fmt == "int4" else None}
    else:
        lb = [layer_bytes(L, c, seq) for L, c in zip(layers_np, counts)]
        avg = {k: float(np.mean([b[k] for b in lb])) for k in lb[0]}
        fl, fl_gu = layer_flops(layers_np[0], seq)
        res.update(tokens_per_s=seq / (ms * 1e-3), touched_experts=avg["U"],
                   layer_hbm_gbs=avg["total"] / (ms * 1e-3) / 1e9,
                   layer_tflops=fl / (ms * 1e-3) / 1e12, stage_ms=stage,
                   gate_up_bytes=avg["gate_up"], gate_up_flops=fl_gu)
        if stage and "fused" in stage:
            # one kernel for the whole layer: its algorithmic bytes are the
            # layer's (touched experts only, although from 12 tokens the dense
            # gate/up pass reads every expert by design)
            fu = stage["fused"] * 1e-3
            fb = avg["total"] - avg["shared"]  # the fused launch's own bytes
            kind = layers[0].decode_kernel(seq, "f32" if x_f32 else "bf16")
            gpt = 128 // group
            res["decode_kernel"] = kind
            res["dominant"] = {"kernel": f"decode_{kind}_kernel<{gpt}, 10, 7, false{', true' if kind == 'stream' and x_f32 else ''}> (router + experts + combine)",
                               "ms": stage["fused"], "bytes": fb,
                               "gbs": fb / fu / 1e9,
                               "traffic_file": f"decode_{kind}_config{cfg}_traffic.md" if fmt == "int4" else None,
                               "profile_file": f"decode_layer_config{cfg}_kernel_stats.md" if fmt == "int4" else None}
        elif stage:
            gu = stage["gate_up"] * 1e-3
            res["gate_up_gbs"] = avg["gate_up"] / gu / 1e9
            res["gate_up_tflops"] = fl_gu / gu / 1e12
            res["gate_up_hbm_frac"] = res["gate_up_gbs"] / HBM_PEAK_GBS
            res["gate_up_mfma_frac"] = res["gate_up_tflops"] / MFMA_PEAK_TFLOPS
            if getattr(layers_np[0], "gate_w", None) is not None:  # bf16 experts (dense.hip)
                big = seq >= 256
                res["dominant"] = {"kernel": "dense_tiled_kernel<true> (gate+up)" if big else
                                   "dense_skinny_kernel<4, 10, true, 0> (gate+up)", "ms": stage["gate_up"],
                                   "bytes": avg["gate_up"], "gbs": res["gate_up_gbs"], "flops": fl_gu,
                                   "tflops": res["gate_up_tflops"], "mfma_frac": res["gate_up_mfma_frac"],
                                   "hbm_frac": res["gate_up_hbm_frac"]}
            elif seq >= 256:  # prefill path: the large-tile MFMA kernel, MFMA-bound
                res["dominant"] = {"kernel": f"experts_prefill_big_kernel<{128 // group}, true, 10> (gate+up)",
                                   "ms": stage["gate_up"], "flops": fl_gu, "tflops": res["gate_up_tflops"],
                                   "mfma_frac": res["gate_up_mfma_frac"],
                                   "profile_file": {2: "experts_prefill_config2_kernel_stats.md",
                                                    3: "experts_prefill_config3_kernel_stats.md"}.get(cfg) if group == 32 else None}
            else:
                res["dominant"] = {"kernel": "expert_decode_kernel<4, 10, true> (gate+up)", "ms": stage["gate_up"],
                                   "bytes": avg["gate_up"], "gbs": res["gate_up_gbs"], "traffic_file": None}
    # the fused decode kernel's sticky status (bit 0: a bounded cross-workgroup
    # wait timed out, bit 1: an exact pick outside the candidates): any set bit
    # means some timed call returned NaN rows, so the measurement is void
    flags = 0
    for lay in layers:
        flags |= lay.status(clear=True)
    res["status_flags"] = flags
    if flags:
        print(f"bench.py: config {cfg}: layer status flags {flags:#x} (a fused call timed out or "
              "picked outside its candidates; its outputs were NaN)", file=sys.stderr)
    for lay in layers:
        lay.close()
    res["_check"] = (wl, gpu_check)
    return res


def _cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def subsample(ids, seq, n, seed=7):
    """Seeded token subsample that always includes tokens routed to the most
    and the least loaded experts (the BASELINE CPU-baseline plan)."""
    import numpy as np
    if seq <= n:
        return np.arange(seq, dtype=np.int32)
    counts = np.bincount(ids.ravel(), minlength=ids.max() + 1)
    live = np.nonzero(counts)[0]
    most, least = live[np.argmax(counts[live])], live[np.argmin(counts[live])]
    must = {int(np.nonzero((ids == most).any(1))[0][0]), int(np.nonzero((ids == least).any(1))[0][0])}
    rng = np.random.default_rng(seed)
    rest = [t for t in rng.permutation(seq) if t not in must][: n - len(must)]
    return np.array(sorted(must | set(int(t) for t in rest)), dtype=np.int32)


def cpu_leg(res, min_seconds=2.0, stack_tokens=8):
    """The CPU reference path (the oracle: the restated reference CPU code) on
    the GPU box's host, for the config `res` measured. Threading is the
    reference's: the routed experts run token by token on one thread
    (moe_decoder.cpp:76-113; the INT4 matvec has no OpenMP, weights.cpp:51-72;
    a bf16 expert's matvec has m = 1, so its row-parallel loop runs one
    iteration), the router and a bf16 shared MLP run as batch GEMMs with the
    reference's OpenMP rule (cpu_ops.cpp:11-39, OpenMP over rows above 2^18
    MACs), the INT4 shared MLP serially. Routing is computed and compared on
    all T tokens; outputs on a seeded subsample of S = min(T, 64) tokens that
    includes tokens of the most and least loaded experts (config 4: S =
    `stack_tokens` tokens through all 12 layers, since a token's path through
    the stack depends only on its own rows). The call is repeated until
    `min_seconds` have passed."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    wl, gpu = res.pop("_check")
    T = wl.seq
    x = wl.x.astype(np.float32)
    L0 = wl.layers[0]
    ids_all, w_all, _ = O.moe_layer(L0, x, sel=np.zeros(0, np.int32))
    routing_exact = bool(np.array_equal(ids_all, gpu["ids"]))
    stack = len(wl.layers) > 1
    S = min(T, stack_tokens if stack else 64)
    sel = subsample(ids_all, T, S)

    def once():
        if stack:
            h = x[sel]
            for L in wl.layers:
                _, _, h = O.moe_layer(L, h)
            return h
        return O.moe_layer(L0, x, sel=sel)[2][sel]

    n, t0 = 0, time.perf_counter()
    while True:
        got = once()
        n += 1
        if time.perf_counter() - t0 >= min_seconds:
            break
    dt = (time.perf_counter() - t0) / n
    want = gpu["out"][sel].astype(np.float64)
    err = got.astype(np.float64) - want
    dense = getattr(L0, "shared_gate_w", None) is not None or getattr(L0, "gate_w", None) is not None
    nproc = os.cpu_count() or 1
    return {"value": S / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "threads_note": ("routed experts on one thread; the router" + (" and the bf16 shared MLP" if dense else "") +
                             f" OpenMP row-parallel (OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS')})"),
            "nproc": nproc, "cpu_model": _cpu_model(),
            "sample": (f"{S} of {T} tokens through {len(wl.layers)} layers" if stack else f"{S} of {T} tokens") +
                      f", x{n} calls, {dt * n:.1f} s",
            "routing_bit_exact_all_tokens": routing_exact,
            "gpu_vs_cpu": {"rel_l2": float(np.linalg.norm(err) / np.linalg.norm(got)),
                           "max_abs": float(np.abs(err).max())},
            "note": "reported baseline, not the target"}


def measured_traffic(name):
    """HBM bytes per launch of the dominant kernel from its committed
    rocprofv3 --pmc summary under profiles/ (FETCH_SIZE + WRITE_SIZE, each
    scaled by the copy-kernel calibration it records); None when absent."""
    try:
        for ln in open(os.path.join(ROOT, "profiles", name)):
            if ln.startswith("traffic_bytes_per_launch:"):
                return float(ln.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_probe(nbytes, reps=5):
    """A plain device copy of `nbytes` bytes, `reps` times: the calibration
    kernel for the FETCH_SIZE / WRITE_SIZE counters (reads and writes nbytes)."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "reps": reps}))


def run_mirrors(steps, warmup, replicas=6):
    """Config 1 through the reference's operator calls one for one (the path of
    an engine that swaps each CUDA call for its mirror, GpuDecoder::mlp_block's
    device branch, src/engine/gpu_decoder.cu:537-657): router GEMV
    (matmul_t_bf16) -> moe_router_topk -> zero out -> moe_experts_masked_int4
    on the reference's table layout; the INT4 shared MLP as moe_gemm_int4 x 3
    + silu_mul; out += shared (add_scaled). Weight replicas as in config 1."""
    import numpy as np
    import torch
    from uocr_hip import ops, synth
    dev = torch.device("cuda:0")
    wl = synth.make_config(1)
    T, H, I = wl.seq, wl.layers[0].hidden, wl.layers[0].inter
    layers = [wl.layers[0]] + [synth.random_layer(9000 + 100 + r) for r in range(1, replicas)]
    reps = []
    for L in layers:
        g, u, d = (ops.RefInt4Table(q, dev) for q in (L.gate, L.up, L.down))
        sq = [(torch.from_numpy(q.packed).to(dev), torch.from_numpy(q.scales).to(dev), torch.from_numpy(q.zeros).to(dev),
               q.rows, q.cols, q.group) for q in (L.shared_gate, L.shared_up, L.shared_down)]
        router = torch.from_numpy(L.router_bf16.view(np.int16)).to(dev)
        reps.append((g, u, d, sq, router))
    x = torch.from_numpy(wl.x).to(dev)
    E, K, SI = 64, 6, layers[0].n_shared * I
    logits = torch.empty(T, E, device=dev)
    ids = torch.empty(T, K, dtype=torch.int32, device=dev)
    w = torch.empty(T, K, device=dev)
    at = torch.empty(E, T, dtype=torch.int32, device=dev)
    aw = torch.empty(E, T, device=dev)
    cnt = torch.empty(E, dtype=torch.int32, device=dev)
    act = torch.empty(E, T, I, device=dev)
    out = torch.empty(T, H, device=dev)
    sg, su, sa = (torch.empty(T, SI, device=dev) for _ in range(3))
    so = torch.empty(T, H, device=dev)

    def step(i):
        g, u, d, sq, router = reps[i % len(reps)]
        ops.matmul_t_bf16(x, router, logits)
        ops.moe_router_topk(logits, K, False, 1.0, False, ids, w, at, aw, cnt, T)
        out.zero_()
        ops.moe_experts_masked_int4(x, g, u, d, at, aw, cnt, T, act, out)
        ops.moe_gemm_int4(x, *sq[0][:3], sq[0][3], sq[0][4], sq[0][5], sg)
        ops.moe_gemm_int4(x, *sq[1][:3], sq[1][3], sq[1][4], sq[1][5], su)
        ops.silu_mul(sg, su, sa)
        ops.moe_gemm_int4(sa, *sq[2][:3], sq[2][3], sq[2][4], sq[2][5], so)
        ops.add_scaled(out, so, 1.0)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": "config1_decode_t16_g32 via the operator mirrors", "ms_per_step": ms,
            "tokens_per_s": T / (ms * 1e-3),
            "sequence": "matmul_t_bf16, moe_router_topk, zero, moe_experts_masked_int4, moe_gemm_int4 x3, silu_mul, add_scaled",
            "note": "hipEvent-timed on torch's current stream; the mirrors run a 64x64-tile MFMA kernel, the fused layer "
                    "call is the fast path"}


def run_rswa_prefill(steps, warmup, batch=4, rows=1000, heads=10, kv_heads=10, head_dim=128):
    """Ragged multi-request R-SWA prefill attention (uocr_hip_rswa_attention_ragged,
    cuda_ops.h:109-124): `batch` requests of `rows` query rows each, row t of a
    request attending its rows [0, t] (causal). Work: 4 * head_dim flops per
    (query row, key row, head) for the scores and the weighted sum."""
    import ctypes as C
    import torch
    from uocr_hip import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    cap = rows + 128
    stride = kv_heads * head_dim
    g = torch.Generator(device=dev).manual_seed(6)
    kc = torch.randn(batch * cap * stride, device=dev, generator=g)
    vc = torch.randn(batch * cap * stride, device=dev, generator=g)
    total = batch * rows
    q = torch.randn(total * heads * head_dim, device=dev, generator=g)
    out = torch.empty_like(q)
    slots = torch.arange(batch, dtype=torch.int32, device=dev).repeat_interleave(rows)
    pos = torch.arange(rows, dtype=torch.int32, device=dev).repeat(batch)
    P = lambda t: C.c_void_p(t.data_ptr())

    def call():
        rc = lib.uocr_hip_rswa_attention_ragged(P(q), P(kc), P(vc), P(slots), P(pos), total, cap, heads, kv_heads,
                                                head_dim, P(out), None)
        if rc:
            raise RuntimeError(lib.uocr_hip_last_error().decode())
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    pairs = batch * rows * (rows + 1) // 2
    flops = 4.0 * head_dim * heads * pairs
    return {"workload": f"rswa_prefill_ragged_{batch}x{rows}_h{heads}_d{head_dim}", "ms_per_step": ms,
            "kernel": "rswa_kernel (uocr_hip_rswa_attention_ragged)", "flops": flops,
            "tflops": flops / (ms * 1e-3) / 1e12,
            "note": "f32 VALU online softmax, one workgroup per (row, head); no MFMA query tiling"}


def run_rswa(steps, warmup, batch=16, prefill=1000, window=128, heads=10, kv_heads=10, head_dim=128, replicas=2):
    """R-SWA decode attention (uocr_hip_rswa_attention_batch) at the decoder's
    shapes: `batch` requests with full caches (prefill + window rows), one
    query row each. HBM-bound: every (request, head) streams its K and V rows.
    `replicas` cache copies (alternating) keep the caches out of the 256 MB
    Infinity Cache."""
    import ctypes as C
    import torch
    from uocr_hip import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    cap = prefill + window
    stride = kv_heads * head_dim
    g = torch.Generator(device=dev).manual_seed(5)
    caches = [(torch.randn(batch * cap * stride, device=dev, generator=g),
               torch.randn(batch * cap * stride, device=dev, generator=g)) for _ in range(replicas)]
    q = torch.randn(batch * heads * head_dim, device=dev, generator=g)
    out = torch.empty_like(q)
    d_len = torch.full((batch,), cap, dtype=torch.int32, device=dev)
    slots = torch.arange(batch, dtype=torch.int32, device=dev)
    P = lambda t: C.c_void_p(t.data_ptr())

    def call(i):
        kc, vc = caches[i % replicas]
        rc = lib.uocr_hip_rswa_attention_batch(P(q), P(kc), P(vc), P(d_len), P(slots), batch, cap, heads, kv_heads,
                                               head_dim, P(out), None)
        if rc:
            raise RuntimeError(lib.uocr_hip_last_error().decode())
    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        call(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    nbytes = batch * heads * cap * head_dim * 4 * 2 + 2 * batch * heads * head_dim * 4
    return {"workload": f"rswa_decode_batch{batch}_kv{cap}_h{heads}_d{head_dim}", "ms_per_step": ms,
            "kernel": "rswa_kernel<128> (uocr_hip_rswa_attention_batch)", "bytes": nbytes,
            "gbs": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "note": "hipEvent-timed on torch's current stream (the library launches on the default stream)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=6)
    ap.add_argument("--extra", default="0,2,3,4,rswa,rswa_prefill,mirrors",
                    help="extra configs to report: 0,2,3,4, rswa (R-SWA decode attention) and mirrors (config 1 "
                         "through the operator mirrors); '' = none")
    ap.add_argument("--graph", default="",
                    help="decode configs (0, 1) replayed from a hipGraph, as a decode engine runs its step; "
                         "their eager rate is reported beside it (config 4 always runs as a graph)")
    ap.add_argument("--formats", default="1:bf16_shared,1:bf16,3:bf16,1:f32_input,1:f32_router,4:f32_router",
                    help="extra (config:format) lines; formats: " + ", ".join(FORMATS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="run one configuration only, CFG or CFG:FORMAT (e.g. 4, 1:bf16_shared), and print its "
                         "record (for per-kernel profiles); config 4 runs at --group")
    ap.add_argument("--group", type=int, default=32)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run a plain copy of BYTES bytes (counter calibration)")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the MoE path is benchmarked on a "
              "single MI355X; multi-GPU expert parallelism is design-only)", file=sys.stderr)
        sys.exit(2)

    graph_cfgs = {v.strip() for v in args.graph.split(",") if v.strip()}
    if args.only:
        c, _, fmt = args.only.partition(":")
        c, fmt = int(c), fmt or "int4"
        if c == 4:
            r = run_config(4, max(args.steps // 10, 5), 3, 1, group=args.group, graph=True, fmt=fmt)
        else:
            reps = 2 if fmt == "bf16" else (3 if c >= 2 else args.replicas)
            r = run_config(c, args.steps, args.warmup, reps, group=args.group, graph=str(c) in graph_cfgs, fmt=fmt)
        r["cpu_baseline"] = None if args.no_cpu else cpu_leg(r)
        r.pop("_check", None)
        print(json.dumps(r))
        return
    main_res = run_config(1, args.steps, args.warmup, args.replicas, graph="1" in graph_cfgs)
    cpu = None if args.no_cpu else cpu_leg(main_res, min_seconds=10.0)
    main_res.pop("_check", None)
    extras = {}

    def extra(key, r):
        r["cpu_baseline"] = None if args.no_cpu else cpu_leg(r)
        r.pop("_check", None)
        extras[key] = r

    for c in [v.strip() for v in args.extra.split(",") if v.strip()]:
        if c == "rswa":
            extras["rswa"] = run_rswa(max(args.steps // 2, 20), 5)
            continue
        if c == "rswa_prefill":
            extras["rswa_prefill"] = run_rswa_prefill(10, 2)
            continue
        if c == "mirrors":
            extras["mirrors"] = run_mirrors(max(args.steps // 2, 20), 5)
            continue
        c = int(c)
        if c == 4:
            for g in (32, 128):
                extra(f"4_g{g}", run_config(4, max(args.steps // 10, 5), 3, 1, group=g, graph=True))
        else:
            extra(str(c), run_config(c, max(args.steps // (5 if c >= 2 else 1), 20),
                                     max(args.warmup // 4, 3), 3 if c >= 2 else args.replicas,
                                     graph=str(c) in graph_cfgs))
    for item in [v.strip() for v in args.formats.split(",") if v.strip()]:
        c, fmt = item.split(":")
        c = int(c)
        if c == 4:
            r = run_config(4, max(args.steps // 10, 5), 3, 1, graph=True, fmt=fmt)
        else:
            # bf16 experts: a layer is ~450 MB, so 2 replicas already exceed the memory-side cache
            reps = 2 if fmt == "bf16" else (3 if c >= 2 else args.replicas)
            r = run_config(c, max(args.steps // (5 if c >= 2 else 1), 20), max(args.warmup // 4, 3), reps,
                           graph=str(c) in graph_cfgs, fmt=fmt)
        extra(f"{c}_{fmt}", r)
    dom = main_res["dominant"]
    line = {
        "metric": "INT4 MoE layer tokens/s (batch-16 decode, config 1)",
        "value": main_res["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded INT4 g32 experts, bf16 N(0,1) hidden states)",
        "config": {"workload": "config1_decode_t16_g32", "tokens": 16, "hidden": 1280,
                   "experts": "64 routed top-6 + 2 shared", "inter": 896, "group": 32,
                   "weight_replicas": args.replicas},
        "roofline": {"bound": "hbm", "kernel": dom["kernel"],
                     "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["gbs"] / HBM_PEAK_GBS, "traffic": measured_traffic(dom["traffic_file"]),
                     "avg_launch_ms": dom["ms"], "algorithmic_bytes": dom["bytes"]},
        "layer_hbm_frac": main_res["layer_hbm_gbs"] / HBM_PEAK_GBS,
        "stage_ms": main_res["stage_ms"],
        "cpu_baseline": cpu,
        "configs": extras,
    }
    line["status_flags"] = main_res.get("status_flags")
    print(json.dumps(line))


if __name__ == "__main__":
    main()
