"""Seeded synthetic MoE layers and inputs for the benchmark configurations.

Shapes follow Unlimited-OCR's decoder (include/uocr/config.h:18-33): hidden 1280,
64 routed experts of width 896, top-6 softmax routing without renormalisation,
2 shared experts (one SwiGLU MLP of width 1792, src/runtime/weights.cpp:352).
Weights are INT4 with the reference's symmetric layout: nibbles uniform in
[0, 15], zero point 8, one scale per group of `group` columns drawn as
|N(0, 0.003)| rounded to bf16 and stored as f32 (include/uocr/quant.h:16-32).
The router is bf16 N(0, 0.02); inputs are bf16-valued.
"""
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

HIDDEN = 1280
INTER = 896
N_EXPERTS = 64
TOP_K = 6
N_SHARED = 2


def f32_to_bf16_bits(a):
    """Round-to-nearest-even f32 -> bf16 bits (include/uocr/common.h:56-64)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    b = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return b.astype(np.uint16)


def bf16_bits_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(a):
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


@dataclass
class QMat:
    """Reference-layout INT4 matrix (uocr::QuantizedMatrix)."""
    packed: np.ndarray   # uint8 [rows, ceil(cols/2)]
    scales: np.ndarray   # f32 [rows, ceil(cols/group)]
    zeros: np.ndarray    # f32 [rows, ceil(cols/group)]
    rows: int
    cols: int
    group: int

    def dequantize(self):
        lo = (self.packed & 0x0F).astype(np.float32)
        hi = (self.packed >> 4).astype(np.float32)
        q = np.empty((self.rows, self.packed.shape[1] * 2), np.float32)
        q[:, 0::2] = lo
        q[:, 1::2] = hi
        q = q[:, : self.cols]
        g = np.arange(self.cols) // self.group
        return (q - self.zeros[:, g]) * self.scales[:, g]


@dataclass
class Dense:
    """Unquantised matrix as the reference holds it (WeightMatrix BF16_EXT /
    F32): `data` is uint16 bf16 bits or float32, shape [rows, cols]."""
    data: np.ndarray

    @property
    def rows(self):
        return self.data.shape[0]

    @property
    def cols(self):
        return self.data.shape[1]

    def to_f32(self):
        return bf16_bits_to_f32(self.data) if self.data.dtype == np.uint16 else np.asarray(self.data, np.float32)


@dataclass
class Layer:
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    n_shared: int
    group: int
    router_bf16: np.ndarray            # uint16 [E, H]
    gate: list                         # [E] QMat [I, H]
    up: list
    down: list                         # [E] QMat [H, I]
    shared_gate: Optional[QMat] = None  # [S*I, H]
    shared_up: Optional[QMat] = None
    shared_down: Optional[QMat] = None  # [H, S*I]
    rms_weight: Optional[np.ndarray] = None
    rms_eps: float = 1e-6
    norm_topk_prob: int = 0
    routed_scaling_factor: float = 1.0
    scoring_sigmoid: int = 0
    router_f32: Optional[np.ndarray] = None  # f32 [E, H]; replaces router_bf16 (AWQ-folded router)
    # unquantised shared MLP (the reference's form, weights.cpp:289-292); replaces shared_*
    shared_gate_w: Optional[Dense] = None
    shared_up_w: Optional[Dense] = None
    shared_down_w: Optional[Dense] = None
    # unquantised routed experts (config.h:111); replace gate/up/down
    gate_w: Optional[list] = None
    up_w: Optional[list] = None
    down_w: Optional[list] = None
    _keep: list = field(default_factory=list, repr=False)


def random_qmat(rng, rows, cols, group, scale_std=0.003):
    packed = rng.integers(0, 256, size=(rows, (cols + 1) // 2), dtype=np.uint8)
    ng = (cols + group - 1) // group
    scales = bf16_round(np.abs(rng.standard_normal((rows, ng), dtype=np.float32) * np.float32(scale_std)))
    zeros = np.full((rows, ng), 8.0, np.float32)
    return QMat(packed, scales, zeros, rows, cols, group)


def random_layer(seed, hidden=HIDDEN, inter=INTER, n_experts=N_EXPERTS, top_k=TOP_K,
                 n_shared=N_SHARED, group=32, router_bias=None, rms=False):
    """One seeded INT4 MoE layer. `router_bias` (length n_experts) is written
    into router column 0 (used with an input whose channel 0 is 1.0)."""
    rng = np.random.default_rng(seed)
    router = rng.standard_normal((n_experts, hidden), dtype=np.float32) * np.float32(0.02)
    if router_bias is not None:
        router[:, 0] = np.asarray(router_bias, np.float32)
    L = Layer(hidden, inter, n_experts, top_k, n_shared, group, f32_to_bf16_bits(router), [], [], [])
    for _ in range(n_experts):
        L.gate.append(random_qmat(rng, inter, hidden, group))
        L.up.append(random_qmat(rng, inter, hidden, group))
        L.down.append(random_qmat(rng, hidden, inter, group))
    if n_shared:
        si = n_shared * inter
        L.shared_gate = random_qmat(rng, si, hidden, group)
        L.shared_up = random_qmat(rng, si, hidden, group)
        L.shared_down = random_qmat(rng, hidden, si, group)
    if rms:
        L.rms_weight = rng.uniform(0.5, 2.0, size=hidden).astype(np.float32)
    return L


def random_dense_bf16(rng, rows, cols, std=0.02):
    """bf16 N(0, std) matrix (a BF16_EXT checkpoint tensor)."""
    return Dense(f32_to_bf16_bits(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)))


def with_bf16_shared(L, seed, std=0.02):
    """L with its shared MLP replaced by bf16 matrices of the same shapes, as the
    reference loads it (load_linear(..., quantize=false), weights.cpp:289-292)."""
    rng = np.random.default_rng(seed)
    si = L.n_shared * L.inter
    L.shared_gate_w = random_dense_bf16(rng, si, L.hidden, std)
    L.shared_up_w = random_dense_bf16(rng, si, L.hidden, std)
    L.shared_down_w = random_dense_bf16(rng, L.hidden, si, std)
    L.shared_gate = L.shared_up = L.shared_down = None
    return L


def random_layer_bf16(seed, hidden=HIDDEN, inter=INTER, n_experts=N_EXPERTS, top_k=TOP_K,
                      n_shared=N_SHARED, router_bias=None, rms=False, std=0.02):
    """A layer in the reference's default format (config.h:111): bf16 routed
    experts and a bf16 shared MLP, bf16 router N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    router = rng.standard_normal((n_experts, hidden), dtype=np.float32) * np.float32(0.02)
    if router_bias is not None:
        router[:, 0] = np.asarray(router_bias, np.float32)
    L = Layer(hidden, inter, n_experts, top_k, n_shared, 32, f32_to_bf16_bits(router), [], [], [])
    L.gate_w = [random_dense_bf16(rng, inter, hidden, std) for _ in range(n_experts)]
    L.up_w = [random_dense_bf16(rng, inter, hidden, std) for _ in range(n_experts)]
    L.down_w = [random_dense_bf16(rng, hidden, inter, std) for _ in range(n_experts)]
    if n_shared:
        si = n_shared * inter
        L.shared_gate_w = random_dense_bf16(rng, si, hidden, std)
        L.shared_up_w = random_dense_bf16(rng, si, hidden, std)
        L.shared_down_w = random_dense_bf16(rng, hidden, si, std)
    if rms:
        L.rms_weight = rng.uniform(0.5, 2.0, size=hidden).astype(np.float32)
    return L


def bf16_normal(rng, shape, std):
    return bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


# Zipf(1.1) router bias for config 3: with x[:, 0] = 1 the logit of expert e gains
# ZIPF_BETA * log((e + 1) ** -1.1); ZIPF_BETA was calibrated so the most popular
# expert receives > 1000 of 4096 tokens (see tests/test_synth.py).
ZIPF_BETA = 1.5


def zipf_bias(n_experts=N_EXPERTS, s=1.1, beta=ZIPF_BETA):
    return (beta * -s * np.log(np.arange(1, n_experts + 1))).astype(np.float32)


@dataclass
class Workload:
    name: str
    seq: int
    layers: list          # list[Layer]
    x: np.ndarray         # f32 (bf16-valued) [seq, hidden]
    note: str = ""


def make_config(cfg, group=32, seed=1234, n_layers=None):
    """Build BASELINE config `cfg` (0..4). Returns a Workload."""
    rng = np.random.default_rng(seed + 1000 * cfg)
    if cfg == 0:
        return Workload("decode_t1", 1, [random_layer(seed + 10, group=group)],
                        bf16_normal(rng, (1, HIDDEN), 1.0), "single decode token")
    if cfg == 1:
        return Workload("decode_t16", 16, [random_layer(seed + 11, group=group)],
                        bf16_normal(rng, (16, HIDDEN), 1.0), "batched decode, 16 tokens")
    if cfg == 2:
        x = np.concatenate([bf16_normal(rng, (900, HIDDEN), 0.5), bf16_normal(rng, (124, HIDDEN), 1.0)])
        return Workload("prefill_t1024", 1024, [random_layer(seed + 12, group=group)], x,
                        "900 visual rows N(0,0.5) + 124 text rows N(0,1)")
    if cfg == 3:
        x = bf16_normal(rng, (4096, HIDDEN), 1.0)
        x[:, 0] = 1.0
        return Workload("prefill_t4096_zipf", 4096,
                        [random_layer(seed + 13, group=group, router_bias=zipf_bias())], x,
                        "Zipf(1.1) expert popularity via router column 0")
    if cfg == 4:
        n = 12 if n_layers is None else n_layers
        layers = [random_layer(seed + 100 + i, group=group, rms=True) for i in range(n)]
        return Workload(f"stack12_t64_g{group}", 64, layers, bf16_normal(rng, (64, HIDDEN), 1.0),
                        "RMSNorm + MoE + residual per layer")
    raise ValueError(cfg)
