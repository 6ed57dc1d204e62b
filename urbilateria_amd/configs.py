"""Layer geometry and the five benchmark workloads.

``LayerSpec`` mirrors the fields the reference's MoE layers carry: ``MoeGeometry``
(src/models/glm/moe_geometry.rs:3-9: top_k, n_group, topk_group, normalize,
routed_scaling_factor) plus the projection formats of ``WeightMatrix``
(src/model/weight.rs:54-61) and the composition of the calling adapter:

* ``COMPOSE_QWEN36`` -- execute_streamed_moe / execute_batched_moe
  (src/models/qwen3_6/runtime.rs:1067-1243): FP32 router GEMV + BF16 logits, softmax top-k,
  BF16 route weights, Qwen SwiGLU experts with BF16 boundaries, BF16 combine in ascending
  expert id.
* ``COMPOSE_GLM`` -- RuntimeMoeLayer::forward (src/models/glm/runtime/moe.rs:138-176): ordered
  f64 router GEMV, softmax top-k or sigmoid noaux_tc, GatedMlp experts, f64 combine in ranking
  order on top of the shared expert.
* ``COMPOSE_DSV41`` -- the MX-activation mode of DeepSeek-V4.1 MoeWeights::forward
  (src/models/deepseek_v41/runtime.rs:1963-2019): FP32 router GEMV, sqrt-softplus routing,
  experts with FP32-accumulated projections whose SwiGLU output is scaled by the route weight
  before the BF16 step and the down projection, f32 ascending-id sum plus the shared expert.
* ``COMPOSE_DSV4`` -- DeepSeek-V4 MoeWeights::forward{,_batch}
  (src/models/deepseek_v4/runtime.rs:2484-2828): as ``COMPOSE_DSV41`` with the ordered f64
  router GEMV and 128-value activation blocks; its first layers route by a tid2eid table
  (``HostLayer.hash_experts``) instead of the scores.
* ``COMPOSE_HY4`` -- the MX-activation mode, Hy4 MoeWeights::forward
  (src/models/hy4/runtime.rs:1371-1447): ordered f64 router GEMV, every MX projection fed by
  simulate_e4m3_activation(x, 32), routed experts with BF16 gate/up and a bounded SwiGLU
  (``swiglu_limit``), BF16 expert outputs, f32 combine in ascending expert id plus the shared
  expert, rounded to BF16.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import synth

FMT_BF16, FMT_MXFP4, FMT_MXFP8 = 0, 1, 2
ROUTER_SOFTMAX_TOPK, ROUTER_SIGMOID_NOAUX_TC, ROUTER_SQRT_SOFTPLUS = 0, 1, 2
COMPOSE_QWEN36, COMPOSE_GLM, COMPOSE_HY4, COMPOSE_DSV41, COMPOSE_DSV4 = 0, 1, 2, 3, 4
FORMAT_NAMES = {FMT_BF16: "bf16", FMT_MXFP4: "mxfp4", FMT_MXFP8: "mxfp8"}


@dataclass(frozen=True)
class LayerSpec:
    hidden: int
    n_experts: int
    top_k: int
    intermediate: int
    shared_intermediate: int = 0
    expert_format: int = FMT_BF16
    shared_format: int = FMT_BF16
    router: int = ROUTER_SOFTMAX_TOPK
    composition: int = COMPOSE_GLM
    n_group: int = 1
    topk_group: int = 1
    normalize: bool = True
    routed_scaling_factor: float = 1.0
    swiglu_limit: float = 0.0   # COMPOSE_HY4 routed experts


def matrix_bytes(fmt: int, rows: int, cols: int) -> Tuple[int, int]:
    """(payload bytes, scale bytes) of one [rows, cols] matrix."""
    if fmt == FMT_BF16:
        return rows * cols * 2, 0
    groups = rows * ((cols + 31) // 32)
    if fmt == FMT_MXFP4:
        return rows * ((cols + 1) // 2), groups
    return rows * cols, groups


def expert_bytes(spec: LayerSpec) -> int:
    H, I = spec.hidden, spec.intermediate
    t = 0
    for r, c in ((I, H), (I, H), (H, I)):
        a, b = matrix_bytes(spec.expert_format, r, c)
        t += a + b
    return t


def shared_bytes(spec: LayerSpec) -> int:
    if not spec.shared_intermediate:
        return 0
    H, I = spec.hidden, spec.shared_intermediate
    t = 0
    for r, c in ((I, H), (I, H), (H, I)):
        a, b = matrix_bytes(spec.shared_format, r, c)
        t += a + b
    return t


@dataclass(frozen=True)
class Workload:
    name: str
    spec: LayerSpec
    tokens: Tuple[int, ...]
    zipf_s: Optional[float] = None
    description: str = ""
    hash_vocab: int = 0   # > 0: routed by a synthetic tid2eid table of this many token ids
    # How the Zipf(zipf_s) correction bias is fitted (``workload_bias``):
    #   "marginals"  one bias per expert, fitted so that each expert's selection frequency is its
    #                inclusion probability in a top-k draw without replacement from the Zipf
    #                popularity (the popularity model of a Zipf-skewed router);
    #   "slope"      b_e = beta ln p_e, beta set so the log-log slope of selection frequency
    #                against rank is -zipf_s;
    #   "top_share"  b_e = beta ln p_e, beta set so the hottest expert takes zipf_top_share of
    #                the tokens.
    zipf_fit: str = "marginals"
    zipf_top_share: float = 0.0


# The five benchmark configurations (shapes, routers, formats and value distributions).
WORKLOADS: Dict[str, Workload] = {
    "c1_bf16_decode": Workload(
        "c1_bf16_decode",
        LayerSpec(hidden=2048, n_experts=128, top_k=8, intermediate=768,
                  expert_format=FMT_BF16, router=ROUTER_SOFTMAX_TOPK,
                  composition=COMPOSE_QWEN36),
        (1,), description="BF16 layer H2048 E128 top-8 softmax I768, decode 1 token"),
    "c2_bf16_prefill": Workload(
        "c2_bf16_prefill",
        LayerSpec(hidden=2048, n_experts=128, top_k=8, intermediate=768,
                  expert_format=FMT_BF16, router=ROUTER_SOFTMAX_TOPK,
                  composition=COMPOSE_QWEN36),
        (128,), description="BF16 layer H2048 E128 top-8 softmax I768, prefill 128 tokens"),
    "c3_mxfp4_decode": Workload(
        "c3_mxfp4_decode",
        LayerSpec(hidden=7168, n_experts=256, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_BF16,
                  router=ROUTER_SIGMOID_NOAUX_TC, composition=COMPOSE_GLM, n_group=8,
                  topk_group=4, normalize=True, routed_scaling_factor=1.0),
        (1, 32), description="MXFP4 H7168 E256 sigmoid group-limited top-8 (8 groups, top-4) "
                             "I2048 + BF16 shared, decode 1 and 32 tokens"),
    "c4_mxfp8": Workload(
        "c4_mxfp8",
        LayerSpec(hidden=6144, n_experts=160, top_k=8, intermediate=2048,
                  expert_format=FMT_MXFP8, router=ROUTER_SOFTMAX_TOPK,
                  composition=COMPOSE_GLM),
        (1, 512), description="MXFP8 H6144 E160 softmax top-8 I2048, decode 1, prefill 512"),
    "c5_mxfp4_zipf_prefill": Workload(
        "c5_mxfp4_zipf_prefill",
        LayerSpec(hidden=7168, n_experts=384, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_BF16,
                  router=ROUTER_SIGMOID_NOAUX_TC, composition=COMPOSE_GLM, n_group=1,
                  topk_group=1, normalize=True, routed_scaling_factor=1.0),
        (1024,), zipf_s=1.1,
        description="MXFP4 H7168 E384 sigmoid top-8 with a per-expert bias giving Zipf(1.1) "
                    "expert popularity (top-8 without replacement) I2048 + BF16 shared, "
                    "prefill 1024"),
    # The same layer with a one-parameter bias b_e = beta ln p_e.  "flat": beta fitted to the
    # log-log slope of the whole frequency curve, where the Gaussian tail of the logits
    # dominates and the head stays flat (hottest expert ~160 of 1024 tokens).  "hot": beta set
    # so the hottest expert takes ~850 of 1024 tokens, which also concentrates the rest on ~55
    # experts.
    "c5_mxfp4_zipf_flat": Workload(
        "c5_mxfp4_zipf_flat",
        LayerSpec(hidden=7168, n_experts=384, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_BF16,
                  router=ROUTER_SIGMOID_NOAUX_TC, composition=COMPOSE_GLM, n_group=1,
                  topk_group=1, normalize=True, routed_scaling_factor=1.0),
        (1024,), zipf_s=1.1, zipf_fit="slope",
        description="MXFP4 H7168 E384 sigmoid top-8 + single-beta Zipf(1.1) bias fitted to "
                    "the frequency slope I2048 + BF16 shared, prefill 1024"),
    "c5_mxfp4_zipf_hot": Workload(
        "c5_mxfp4_zipf_hot",
        LayerSpec(hidden=7168, n_experts=384, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_BF16,
                  router=ROUTER_SIGMOID_NOAUX_TC, composition=COMPOSE_GLM, n_group=1,
                  topk_group=1, normalize=True, routed_scaling_factor=1.0),
        (1024,), zipf_s=1.1, zipf_fit="top_share", zipf_top_share=850.0 / 1024.0,
        description="MXFP4 H7168 E384 sigmoid top-8 + single-beta Zipf(1.1) bias, hottest "
                    "expert ~850 of 1024 tokens, I2048 + BF16 shared, prefill 1024"),
}

# The MX-activation mode on the shapes of c4_mxfp8 and c5_mxfp4_zipf_prefill: Hy4's
# composition (E4M3 activations per
# 32 values into every MX projection, BF16 boundaries, bounded SwiGLU with limit 7, f32
# ascending-id combine) and DeepSeek-V4.1's (the same activations, FP32-accumulated
# projections, route weight applied before the down projection, sqrt-softplus router).  The
# shared expert of the c5 shape is MXFP4 here: the mode feeds MX weights only.
MX_ACTIVATION_WORKLOADS: Dict[str, Workload] = {
    "c4_mxfp8_mx_activation": Workload(
        "c4_mxfp8_mx_activation",
        LayerSpec(hidden=6144, n_experts=160, top_k=8, intermediate=2048,
                  expert_format=FMT_MXFP8, router=ROUTER_SOFTMAX_TOPK,
                  composition=COMPOSE_HY4, swiglu_limit=7.0),
        (1, 512), description="MXFP8 H6144 E160 softmax top-8 I2048, MX activations (Hy4 "
                              "composition), decode 1, prefill 512"),
    "c5_mxfp4_mx_activation": Workload(
        "c5_mxfp4_mx_activation",
        LayerSpec(hidden=7168, n_experts=384, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_MXFP4,
                  router=ROUTER_SIGMOID_NOAUX_TC, composition=COMPOSE_HY4, n_group=1,
                  topk_group=1, normalize=True, routed_scaling_factor=1.0, swiglu_limit=7.0),
        (1024,), zipf_s=1.1,
        description="MXFP4 H7168 E384 sigmoid top-8 + Zipf(1.1) bias I2048 + MXFP4 shared, MX "
                    "activations (Hy4 composition), prefill 1024"),
    "c5_mxfp4_dsv41": Workload(
        "c5_mxfp4_dsv41",
        LayerSpec(hidden=7168, n_experts=384, top_k=8, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_MXFP4,
                  router=ROUTER_SQRT_SOFTPLUS, composition=COMPOSE_DSV41,
                  routed_scaling_factor=1.5, swiglu_limit=7.0),
        (1, 1024), zipf_s=1.1,
        description="MXFP4 H7168 E384 sqrt-softplus top-8 + Zipf(1.1) bias I2048 + MXFP4 shared, "
                    "MX activations (DeepSeek-V4.1 composition), decode 1, prefill 1024"),
}


# The Qwen3.6 release MoE geometry (src/models/qwen3_6/expert_store.rs:180-190: H 2048, 256
# experts of I 512, BF16) with its sigmoid-gated BF16 shared expert (I 512), top-8: the full
# QWEN36 composition the c1/c2 shapes leave the shared expert out of.
QWEN36_RELEASE_WORKLOADS: Dict[str, Workload] = {
    "qwen36_release": Workload(
        "qwen36_release",
        LayerSpec(hidden=2048, n_experts=256, top_k=8, intermediate=512,
                  shared_intermediate=512, expert_format=FMT_BF16, shared_format=FMT_BF16,
                  router=ROUTER_SOFTMAX_TOPK, composition=COMPOSE_QWEN36),
        (1, 128), description="Qwen3.6 release MoE: BF16 H2048 E256 softmax top-8 I512 + gated "
                              "BF16 shared expert I512, decode 1, prefill 128"),
}


# The DeepSeek-V4 Flash MoE geometry (the reference's tests/fixtures/
# deepseek_v4_flash_0731_config.json: hidden 4096, 256 routed experts of I 2048, top-6, one
# shared expert, routed_scaling_factor 1.5, swiglu_limit 10, FP4 experts, sqrt-softplus scores,
# 3 hash layers over a 129280-token vocabulary) in the DSV4 composition; the shared expert is
# synthesized in MXFP4 like the routed ones.
DSV4_WORKLOADS: Dict[str, Workload] = {
    "dsv4_flash": Workload(
        "dsv4_flash",
        LayerSpec(hidden=4096, n_experts=256, top_k=6, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_MXFP4,
                  router=ROUTER_SQRT_SOFTPLUS, composition=COMPOSE_DSV4,
                  routed_scaling_factor=1.5, swiglu_limit=10.0),
        (1, 1024), zipf_s=1.1,
        description="DeepSeek-V4 Flash MoE: MXFP4 H4096 E256 sqrt-softplus top-6 + Zipf(1.1) "
                    "bias I2048 + MXFP4 shared, 128-value MX activations, decode 1, prefill "
                    "1024"),
    "dsv4_flash_hash": Workload(
        "dsv4_flash_hash",
        LayerSpec(hidden=4096, n_experts=256, top_k=6, intermediate=2048,
                  shared_intermediate=2048, expert_format=FMT_MXFP4, shared_format=FMT_MXFP4,
                  router=ROUTER_SQRT_SOFTPLUS, composition=COMPOSE_DSV4,
                  routed_scaling_factor=1.5, swiglu_limit=10.0),
        (1, 1024), hash_vocab=129280,
        description="DeepSeek-V4 Flash hash layer: as dsv4_flash, experts from a synthetic "
                    "129280 x 6 tid2eid table indexed by uniform token ids"),
}


def workload(name: str) -> Workload:
    """A benchmark configuration or one of its variants, by name."""
    for table in (WORKLOADS, QWEN36_RELEASE_WORKLOADS, DSV4_WORKLOADS):
        if name in table:
            return table[name]
    return MX_ACTIVATION_WORKLOADS[name]



@dataclass
class HostLayer:
    """Packed host weights of one layer, in the reference's on-disk layouts."""
    spec: LayerSpec
    router_weight: np.ndarray                       # [E, H] uint16 BF16 bits
    experts: List[List[Tuple[np.ndarray, Optional[np.ndarray]]]]  # [E][gate, up, down]
    shared: Optional[List[Tuple[np.ndarray, Optional[np.ndarray]]]] = None
    correction_bias: Optional[np.ndarray] = None     # [E] f32
    shared_expert_gate: Optional[np.ndarray] = None  # [H] uint16 BF16 (QWEN36 shared expert)
    hash_experts: Optional[np.ndarray] = None        # [vocab, k] int64 tid2eid (sqrt-softplus)


def hash_table(vocab: int, n_experts: int, top_k: int,
               base_seed: int = synth.BASE_SEED) -> np.ndarray:
    """A synthetic tid2eid table [vocab, top_k] (int64): row v holds the distinct expert ids
    (a_v + j * b_v) mod E, j < top_k, with seeded a_v and a seeded stride b_v coprime to E."""
    E = n_experts
    keys = synth.splitmix64(synth.stream_seed("tid2eid", base_seed), 0, 2 * vocab)
    start = (keys[0::2] % np.uint64(E)).astype(np.int64)
    stride = (keys[1::2] % np.uint64(E)).astype(np.int64) | 1
    while True:  # step each stride until coprime with E (E = 1: any stride)
        bad = np.gcd(stride, E) != 1
        if E == 1 or not bad.any():
            break
        stride[bad] += 1
    j = np.arange(top_k, dtype=np.int64)
    return np.ascontiguousarray((start[:, None] + j[None, :] * stride[:, None]) % E)


def _matrix(fmt: int, name: str, rows: int, cols: int, base_seed: int):
    if fmt == FMT_BF16:
        return synth.bf16_matrix(name, rows, cols, 0.02, base_seed), None
    if fmt == FMT_MXFP4:
        return synth.mxfp4_matrix(name, rows, cols, base_seed)
    return synth.mxfp8_matrix(name, rows, cols, base_seed)


def make_host_layer(spec: LayerSpec, base_seed: int = synth.BASE_SEED,
                    bias: Optional[np.ndarray] = None, hash_vocab: int = 0) -> HostLayer:
    """Generates a layer on the host (numpy).  Practical for small shapes only; full-size
    layers are generated on the device by ``urbilateria_amd.device.make_device_layer``."""
    H, I, E = spec.hidden, spec.intermediate, spec.n_experts
    router = synth.bf16_matrix("router", E, H, 0.02, base_seed)
    experts = []
    for e in range(E):
        experts.append([
            _matrix(spec.expert_format, f"expert.{e}.gate", I, H, base_seed),
            _matrix(spec.expert_format, f"expert.{e}.up", I, H, base_seed),
            _matrix(spec.expert_format, f"expert.{e}.down", H, I, base_seed),
        ])
    shared = None
    if spec.shared_intermediate:
        Is = spec.shared_intermediate
        shared = [
            _matrix(spec.shared_format, "shared.gate", Is, H, base_seed),
            _matrix(spec.shared_format, "shared.up", Is, H, base_seed),
            _matrix(spec.shared_format, "shared.down", H, Is, base_seed),
        ]
    gate = None
    if spec.shared_intermediate and spec.composition == COMPOSE_QWEN36:
        gate = synth.bf16_matrix("shared.expert_gate", 1, H, 0.02, base_seed).reshape(H)
    table = hash_table(hash_vocab, E, spec.top_k, base_seed) if hash_vocab else None
    return HostLayer(spec, router, experts, shared, bias, gate, table)


def zipf_bias(n_experts: int, s: float, beta: float, base_seed: int = synth.BASE_SEED) -> np.ndarray:
    """Correction bias b_e = beta * ln(p_e) with p_e proportional to rank_e^-s; ranks come
    from a seeded permutation of the expert ids."""
    keys = synth.splitmix64(synth.stream_seed("zipf.rank", base_seed), 0, n_experts)
    rank = np.empty(n_experts, np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(1, n_experts + 1)
    p = rank.astype(np.float64) ** (-s)
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def calibrate_zipf_beta(n_experts: int, top_k: int, s: float, logit_std: np.ndarray,
                        tokens: int = 4096, base_seed: int = synth.BASE_SEED,
                        router: int = ROUTER_SIGMOID_NOAUX_TC, top_target: float = 0.0) -> float:
    """Bisection on beta so the log-log slope of expert selection frequency against popularity
    rank is -s (top_target > 0: so the hottest expert is selected by that share of tokens).  Router logits are drawn as independent N(0, logit_std[e]^2), the distribution
    a BF16 N(0, 0.02) router produces on N(0, 1) activations (logit_std[e] = ||w_e||); the
    selection score is the router's: sigmoid, or sqrt(softplus) for ROUTER_SQRT_SOFTPLUS."""
    z = synth.normals(synth.stream_seed("zipf.calibration", base_seed), tokens * n_experts)
    logits = z.reshape(tokens, n_experts).astype(np.float64) * logit_std[None, :]
    if router == ROUTER_SQRT_SOFTPLUS:
        gates = np.sqrt(np.logaddexp(0.0, logits))
    else:
        gates = 1.0 / (1.0 + np.exp(-logits))
    keys = synth.splitmix64(synth.stream_seed("zipf.rank", base_seed), 0, n_experts)
    rank = np.empty(n_experts, np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(1, n_experts + 1)

    def slope(beta: float) -> float:
        bias = zipf_bias(n_experts, s, beta, base_seed).astype(np.float64)
        sel = gates + bias[None, :]
        top = np.argpartition(-sel, top_k - 1, axis=1)[:, :top_k]
        freq = np.bincount(top.ravel(), minlength=n_experts).astype(np.float64)
        ok = freq > 0
        return float(np.polyfit(np.log(rank[ok]), np.log(freq[ok]), 1)[0])

    def top_share(beta: float) -> float:
        bias = zipf_bias(n_experts, s, beta, base_seed).astype(np.float64)
        sel = gates + bias[None, :]
        top = np.argpartition(-sel, top_k - 1, axis=1)[:, :top_k]
        return float(np.bincount(top.ravel(), minlength=n_experts).max()) / tokens

    lo, hi = 0.0, 4.0
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        if (top_share(mid) < top_target) if top_target else (slope(mid) > -s):
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def zipf_popularity(n_experts: int, s: float,
                    base_seed: int = synth.BASE_SEED) -> Tuple[np.ndarray, np.ndarray]:
    """(rank [E], popularity p [E]): ranks 1..E from a seeded permutation of the expert ids,
    p_e proportional to rank_e^-s, normalised."""
    keys = synth.splitmix64(synth.stream_seed("zipf.rank", base_seed), 0, n_experts)
    rank = np.empty(n_experts, np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(1, n_experts + 1)
    p = rank.astype(np.float64) ** (-s)
    return rank, p / p.sum()


def zipf_inclusion(p: np.ndarray, top_k: int, points: int = 2000) -> np.ndarray:
    """Inclusion probability of each item in a draw of top_k items without replacement, each
    draw picking a remaining item with probability proportional to p (successive sampling).

    Exact up to quadrature: with independent clocks X_f ~ Exp(p_f), the draw order is the
    clock order, so pi_e = integral over t of P(fewer than top_k other clocks fired by t)
    d(1 - exp(-p_e t)).  The count of other fired clocks is Poisson-binomial; its
    distribution truncated at top_k comes from prefix and suffix products over the items,
    leaving item e out.  The t grid is geometric, 'points' cells (2000: within 1e-6 of the
    exact value at 384 items, top-8)."""
    p = np.asarray(p, np.float64)
    p = p / p.sum()
    E, K = len(p), top_k
    if K >= E:
        return np.ones(E)
    edges = np.concatenate([[0.0], np.geomspace(1e-6 / p.max(), 60.0 / p.min(), points)])
    mids = np.concatenate([[edges[1] / 2], np.sqrt(edges[2:] * edges[1:-1]), [edges[-1] * 2]])
    q = -np.expm1(-np.outer(p, mids))            # clock f fired by the cell's midpoint

    def step(d, qf):
        n = d * (1.0 - qf)[:, None]
        n[:, 1:] += d[:, :-1] * qf[:, None]
        n[:, K] += d[:, K] * qf                   # index K: K or more fired
        return n

    M = len(mids)
    pre = np.zeros((E + 1, M, K + 1))
    pre[0, :, 0] = 1.0
    for f in range(E):
        pre[f + 1] = step(pre[f], q[f])
    suf = np.zeros((E + 1, M, K + 1))
    suf[E, :, 0] = 1.0
    for f in range(E - 1, -1, -1):
        suf[f] = step(suf[f + 1], q[f])
    cum = np.cumsum(suf[1:, :, :K], axis=2)
    below = np.zeros((E, M))
    for i in range(K):
        below += pre[:E, :, i] * cum[:, :, K - 1 - i]
    cdf = -np.expm1(-np.outer(p, np.concatenate([edges, [np.inf]])))
    return (below * np.diff(cdf, axis=1)).sum(axis=1)


def router_scores(router: int, logits: np.ndarray) -> np.ndarray:
    """The selection score a biased router ranks by (before the bias): sigmoid for noaux_tc
    (src/math/routing.rs:62-67), sqrt(softplus) for sqrt-softplus
    (src/models/deepseek_v4/math.rs:480-487)."""
    if router == ROUTER_SQRT_SOFTPLUS:
        return np.sqrt(np.logaddexp(0.0, logits))
    return 1.0 / (1.0 + np.exp(-logits))


def calibration_scores(spec: LayerSpec, tokens: int,
                       base_seed: int = synth.BASE_SEED) -> np.ndarray:
    """Selection scores [tokens, E] of calibration tokens: logits drawn independently as
    N(0, ||w_e||^2), the distribution the layer's seeded BF16 router row w_e gives on N(0, 1)
    activations (the rows are near-orthogonal: |cos| ~ 1/sqrt(H))."""
    w = synth.bf16_to_f32(synth.bf16_matrix("router", spec.n_experts, spec.hidden, 0.02,
                                            base_seed)).astype(np.float64)
    std = np.sqrt((w * w).sum(axis=1))
    z = synth.normals(synth.stream_seed("zipf.calibration", base_seed),
                      tokens * spec.n_experts).astype(np.float64)
    return router_scores(spec.router, z.reshape(tokens, spec.n_experts) * std[None, :])


def fit_selection_bias(scores: np.ndarray, top_k: int, target: np.ndarray,
                       iters: int = 40, damping: float = 0.5) -> Tuple[np.ndarray, np.ndarray]:
    """A per-expert bias b [E] under which top-k selection by scores + b picks expert e in
    about target[e] of the rows (sum(target) = rows * top_k).  Damped Jacobi iteration: given
    the others' biases, expert e is picked in row n exactly when s_ne + b_e exceeds the k-th
    largest biased score among the other experts (the row's (k+1)-th largest when e is picked,
    its k-th otherwise), so each step sets every b_e to the value that meets its target with
    the other biases held, and moves halfway there.  Returns (bias, counts under it)."""
    N, E = scores.shape
    K = top_k
    b = np.zeros(E)
    cols = np.arange(E)
    t = np.clip(np.asarray(target, np.float64), 0.5, N - 0.5)
    lo = np.floor(t).astype(np.int64)
    counts = None
    for _ in range(iters + 1):
        sel = scores + b[None, :]
        part = np.partition(sel, (E - K - 1, E - K), axis=1)
        kth, k1th = part[:, E - K], part[:, E - K - 1]
        picked = sel >= kth[:, None]
        counts = picked.sum(axis=0)
        d = scores - np.where(picked, k1th[:, None], kth[:, None])  # picked iff d + b_e > 0
        ds = -np.sort(-d, axis=0)
        c = 0.5 * (ds[np.clip(lo - 1, 0, N - 1), cols] + ds[np.clip(lo, 0, N - 1), cols])
        b = b + damping * (-c - b)
    return b, counts


_BIAS_CACHE: Dict[str, Tuple[dict, np.ndarray]] = {}
ZIPF_CALIBRATION_TOKENS = 8192


def workload_bias(w: Workload) -> Tuple[Optional[dict], Optional[np.ndarray]]:
    """(fit record, correction bias [E] f32) of a Zipf workload, as the benchmark runs it
    (None, None without a Zipf bias).  The record names the fit and, for "marginals", the
    targets and the calibration's own head counts; for the single-beta fits, beta."""
    if not w.zipf_s:
        return None, None
    if w.name not in _BIAS_CACHE:
        spec = w.spec
        if w.zipf_fit == "marginals":
            rank, p = zipf_popularity(spec.n_experts, w.zipf_s)
            pi = zipf_inclusion(p, spec.top_k)
            N = ZIPF_CALIBRATION_TOKENS
            scores = calibration_scores(spec, N)
            bias, counts = fit_selection_bias(scores, spec.top_k, N * pi)
            ok = counts > 0
            info = {"fit": "marginals", "zipf_s": w.zipf_s, "calibration_tokens": N,
                    "target_top_share": float(pi.max()),
                    "calibration_top_share": float(counts.max() / N),
                    "max_abs_count_error": float(np.abs(counts - N * pi).max()),
                    "calibration_slope": float(np.polyfit(np.log(rank[ok]),
                                                          np.log(counts[ok]), 1)[0])}
            _BIAS_CACHE[w.name] = (info, bias.astype(np.float32))
        else:
            std = np.full(spec.n_experts, 0.02 * np.sqrt(spec.hidden))
            top = w.zipf_top_share if w.zipf_fit == "top_share" else 0.0
            beta = calibrate_zipf_beta(spec.n_experts, spec.top_k, w.zipf_s, std,
                                       router=spec.router, top_target=top)
            _BIAS_CACHE[w.name] = ({"fit": w.zipf_fit, "zipf_s": w.zipf_s, "beta": beta},
                                   zipf_bias(spec.n_experts, w.zipf_s, beta))
    info, bias = _BIAS_CACHE[w.name]
    return dict(info), bias.copy()


def with_tokens(w: Workload, tokens: int) -> Tuple[LayerSpec, int]:
    return w.spec, tokens


def small_spec(spec: LayerSpec, hidden: int = 64, n_experts: int = 8, intermediate: int = 32,
               top_k: Optional[int] = None) -> LayerSpec:
    """A reduced copy of a spec for fast parity tests (keeps formats and routing rules)."""
    k = min(spec.top_k, n_experts) if top_k is None else top_k
    groups = spec.n_group if spec.n_group > 1 and n_experts % spec.n_group == 0 and \
        n_experts // spec.n_group >= 2 else 1
    return replace(spec, hidden=hidden, n_experts=n_experts, intermediate=intermediate,
                   top_k=k, n_group=groups, topk_group=min(spec.topk_group, groups),
                   shared_intermediate=(intermediate if spec.shared_intermediate else 0))
