"""ctypes bindings for the CPU oracle (``liburb_oracle.so``).

TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this module.
The oracle restates inspirewind/Urbilateria 0.2.4's CPU path; each C function cites the Rust
function it follows (see ``urb_oracle.h``).
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liburb_oracle.so")

OK, SHAPE, INVALID_SCALE, NONFINITE, INVALID_GEOMETRY = 0, 1, 2, 3, 4
FMT_BF16, FMT_MXFP4, FMT_MXFP8, FMT_F32 = 0, 1, 2, 3
ROUTER_SOFTMAX_TOPK, ROUTER_SIGMOID_NOAUX_TC, ROUTER_SQRT_SOFTPLUS = 0, 1, 2
COMPOSE_QWEN36, COMPOSE_GLM, COMPOSE_HY4, COMPOSE_DSV41, COMPOSE_DSV4 = 0, 1, 2, 3, 4

_STATUS_NAMES = {OK: "ok", SHAPE: "shape", INVALID_SCALE: "invalid_scale",
                 NONFINITE: "nonfinite", INVALID_GEOMETRY: "invalid_geometry"}


class OracleError(Exception):
    def __init__(self, status: int):
        super().__init__(f"oracle status {status} ({_STATUS_NAMES.get(status, '?')})")
        self.status = status


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    sz = ctypes.c_size_t
    lib.urbo_decode_e8m0.argtypes = [ctypes.c_uint8, ctypes.POINTER(ctypes.c_float)]
    lib.urbo_decode_e2m1.argtypes = [ctypes.c_uint8]
    lib.urbo_decode_e2m1.restype = ctypes.c_float
    lib.urbo_decode_e4m3fn.argtypes = [ctypes.c_uint8]
    lib.urbo_decode_e4m3fn.restype = ctypes.c_float
    lib.urbo_encode_e4m3fn_finite.argtypes = [ctypes.c_float]
    lib.urbo_encode_e4m3fn_finite.restype = ctypes.c_uint8
    lib.urbo_power_of_two_ceiling.argtypes = [ctypes.c_float]
    lib.urbo_power_of_two_ceiling.restype = ctypes.c_float
    lib.urbo_simulate_e4m3_activation.argtypes = [P, sz, sz]
    lib.urbo_round_to_bf16.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float)]
    lib.urbo_round_to_bf16_in_place.argtypes = [P, sz]
    lib.urbo_validate.argtypes = [ctypes.c_int, P, P, sz, sz]
    lib.urbo_row.argtypes = [ctypes.c_int, P, P, sz, sz, sz, P]
    lib.urbo_matvec_rows.argtypes = [ctypes.c_int, P, P, sz, sz, sz, sz, P, P]
    lib.urbo_bf16_matvec_rows_fp32.argtypes = [P, sz, sz, sz, sz, P, P]
    lib.urbo_mxfp4_matvec_rows_fp32.argtypes = [P, P, sz, sz, sz, sz, P, P]
    lib.urbo_mxfp8_matvec_rows_f64.argtypes = [P, P, sz, sz, sz, sz, P, P]
    lib.urbo_route_softmax_top_k.argtypes = [P, sz, sz, P, P]
    lib.urbo_route_sqrt_softplus.argtypes = [P, P, sz, sz, ctypes.c_float, P, P, P]
    lib.urbo_route_sqrt_softplus_hashed.argtypes = [P, P, P, sz, sz, ctypes.c_float, P, P, P]
    lib.urbo_route_noaux_tc.argtypes = [P, P, sz, sz, sz, sz, ctypes.c_int, ctypes.c_float,
                                        P, P, P]
    lib.urbo_silu.argtypes = [ctypes.c_float]
    lib.urbo_silu.restype = ctypes.c_float
    lib.urbo_moe_forward.argtypes = [P, P, ctypes.c_uint32, P, P, P, P, ctypes.c_int]
    lib.urbo_moe_forward_tokens.argtypes = [P, P, P, ctypes.c_uint32, P, P, P, P, ctypes.c_int]
    lib.urbo_dsv4_expert.argtypes = [ctypes.c_int, P, ctypes.c_uint32, ctypes.c_uint32, P,
                                     ctypes.c_uint32, ctypes.c_float, P, P, ctypes.c_int]
    lib.urbo_physical_cores.argtypes = []
    lib.urbo_physical_cores.restype = ctypes.c_int
    lib.urbo_cpu_order.argtypes = [P, sz]
    lib.urbo_cpu_order.restype = sz
    lib.urbo_set_pinning.argtypes = [ctypes.c_int]
    lib.urbo_set_pinning.restype = ctypes.c_int
    return lib


_lib = _load()


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(status: int):
    if status != OK:
        raise OracleError(status)


# ---------------------------------------------------------------- element functions
def decode_e8m0(code: int) -> float:
    out = ctypes.c_float()
    _check(_lib.urbo_decode_e8m0(code, ctypes.byref(out)))
    return np.float32(out.value)


def decode_e2m1(code: int) -> np.float32:
    return np.float32(_lib.urbo_decode_e2m1(code))


def decode_e4m3fn(code: int) -> np.float32:
    return np.float32(_lib.urbo_decode_e4m3fn(code))


def encode_e4m3fn_finite(value: float) -> int:
    return int(_lib.urbo_encode_e4m3fn_finite(float(np.float32(value))))


def power_of_two_ceiling(value: float) -> np.float32:
    return np.float32(_lib.urbo_power_of_two_ceiling(float(np.float32(value))))


def simulate_e4m3_activation(values: np.ndarray, block: int) -> np.ndarray:
    out = np.ascontiguousarray(values, dtype=np.float32).copy()
    _check(_lib.urbo_simulate_e4m3_activation(_ptr(out), out.size, block))
    return out


def round_to_bf16(value: float) -> np.float32:
    out = ctypes.c_float()
    _check(_lib.urbo_round_to_bf16(float(np.float32(value)), ctypes.byref(out)))
    return np.float32(out.value)


def round_to_bf16_in_place(values: np.ndarray) -> int:
    """Rounds in place; returns the status (values before the first failure are rounded)."""
    assert values.dtype == np.float32 and values.flags["C_CONTIGUOUS"]
    return _lib.urbo_round_to_bf16_in_place(_ptr(values), values.size)


def silu(value: float) -> np.float32:
    return np.float32(_lib.urbo_silu(float(np.float32(value))))


# ---------------------------------------------------------------- matrices
def validate(fmt: int, data: np.ndarray, scales: Optional[np.ndarray], rows: int, cols: int) -> int:
    return _lib.urbo_validate(fmt, _ptr(data), _ptr(scales), rows, cols)


def row(fmt: int, data, scales, rows: int, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    _check(_lib.urbo_row(fmt, _ptr(data), _ptr(scales), rows, cols, r, _ptr(out)))
    return out


def matvec_rows(fmt: int, data, scales, rows: int, cols: int, x: np.ndarray,
                start: int = 0, count: Optional[int] = None) -> np.ndarray:
    count = rows - start if count is None else count
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(count, np.float32)
    _check(_lib.urbo_matvec_rows(fmt, _ptr(data), _ptr(scales), rows, cols, start, count,
                                 _ptr(x), _ptr(out)))
    return out


def bf16_matvec_rows_fp32(data: np.ndarray, rows: int, cols: int, x: np.ndarray,
                          start: int = 0, count: Optional[int] = None) -> np.ndarray:
    count = rows - start if count is None else count
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(count, np.float32)
    _check(_lib.urbo_bf16_matvec_rows_fp32(_ptr(data), rows, cols, start, count, _ptr(x),
                                           _ptr(out)))
    return out


def mxfp4_matvec_rows_fp32(packed, scales, rows: int, cols: int, x: np.ndarray,
                           start: int = 0, count: Optional[int] = None) -> np.ndarray:
    count = rows - start if count is None else count
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(count, np.float32)
    _check(_lib.urbo_mxfp4_matvec_rows_fp32(_ptr(packed), _ptr(scales), rows, cols, start,
                                            count, _ptr(x), _ptr(out)))
    return out


def mxfp8_matvec_rows_f64(codes, scales, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, np.float32)
    _check(_lib.urbo_mxfp8_matvec_rows_f64(_ptr(codes), _ptr(scales), rows, cols, 0, rows,
                                           _ptr(x), _ptr(out)))
    return out


# ---------------------------------------------------------------- routers
def route_softmax_top_k(logits: np.ndarray, top_k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    _check(_lib.urbo_route_softmax_top_k(_ptr(logits), logits.size, top_k, _ptr(ids), _ptr(w)))
    return ids, w


def route_sqrt_softplus(logits, bias, top_k: int, scale: float, hash_experts=None):
    """route_sqrt_softplus; ``hash_experts`` (top_k ids, table order) replaces the ranking."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    h = None if hash_experts is None else np.ascontiguousarray(hash_experts, dtype=np.int64)
    if h is not None and h.size != top_k:
        raise OracleError(SHAPE)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    sel = np.empty(top_k, np.float32)
    _check(_lib.urbo_route_sqrt_softplus_hashed(_ptr(logits), _ptr(b), _ptr(h), logits.size,
                                                top_k, float(scale), _ptr(ids), _ptr(w),
                                                _ptr(sel)))
    return ids, w, sel


def route_noaux_tc(logits, bias, top_k: int, n_group: int, topk_group: int, normalize: bool,
                   scale: float):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    sel = np.empty(top_k, np.float32)
    _check(_lib.urbo_route_noaux_tc(_ptr(logits), _ptr(bias), logits.size, top_k, n_group,
                                    topk_group, int(normalize), float(scale), _ptr(ids), _ptr(w),
                                    _ptr(sel)))
    return ids, w, sel


# ---------------------------------------------------------------- one MoE layer
class _Matrix(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


class _Layer(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_uint32), ("n_experts", ctypes.c_uint32),
        ("top_k", ctypes.c_uint32), ("intermediate", ctypes.c_uint32),
        ("shared_intermediate", ctypes.c_uint32),
        ("expert_format", ctypes.c_int32), ("shared_format", ctypes.c_int32),
        ("router", ctypes.c_int32), ("composition", ctypes.c_int32),
        ("n_group", ctypes.c_uint32), ("topk_group", ctypes.c_uint32),
        ("normalize", ctypes.c_int32), ("routed_scaling_factor", ctypes.c_float),
        ("router_weight", ctypes.c_void_p), ("correction_bias", ctypes.c_void_p),
        ("experts", ctypes.c_void_p), ("shared", ctypes.c_void_p),
        ("swiglu_limit", ctypes.c_float),
        ("shared_expert_gate", ctypes.c_void_p),
        ("hash_experts", ctypes.c_void_p), ("hash_vocab", ctypes.c_uint32),
        ("router_weight_f32", ctypes.c_void_p),
    ]


@dataclass
class OracleResult:
    output: np.ndarray   # [T, H] f32
    ids: np.ndarray      # [T, k] ranking order
    weights: np.ndarray  # [T, k]
    logits: np.ndarray   # [T, E]


def moe_forward(spec, experts: Sequence, router_weight: np.ndarray, x: np.ndarray,
                correction_bias: Optional[np.ndarray] = None, shared: Optional[Sequence] = None,
                threads: int = 1, shared_expert_gate: Optional[np.ndarray] = None,
                token_ids: Optional[np.ndarray] = None, hash_experts: Optional[np.ndarray] = None,
                router_weight_f32: Optional[np.ndarray] = None) -> OracleResult:
    """Runs one layer.  ``spec`` carries the layer geometry (attributes hidden, n_experts,
    top_k, intermediate, shared_intermediate, expert_format, shared_format, router, composition,
    n_group, topk_group, normalize, routed_scaling_factor, swiglu_limit).  ``experts[e]`` is a triple of
    (data, scales) pairs for gate, up and down; ``shared`` likewise or None.  ``hash_experts``
    [vocab, k] routes token t by row ``token_ids[t]``; ``router_weight_f32`` [E, H] replaces the
    BF16 router of a DeepSeek-V4 layer."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    H, E, K = spec.hidden, spec.n_experts, spec.top_k
    keep = []
    mats = (_Matrix * (E * 3))()
    for e in range(E):
        if experts[e] is None:  # not supplied: the oracle reports SHAPE if routing needs it
            continue
        for m in range(3):
            d, s = experts[e][m]
            keep += [d, s]
            mats[e * 3 + m] = _Matrix(_ptr(d), _ptr(s))
    sh = None
    if shared is not None:
        sh = (_Matrix * 3)()
        for m in range(3):
            d, s = shared[m]
            keep += [d, s]
            sh[m] = _Matrix(_ptr(d), _ptr(s))
    rwt = np.ascontiguousarray(router_weight)
    bias = None if correction_bias is None else np.ascontiguousarray(correction_bias, np.float32)
    sgate = None if shared_expert_gate is None else np.ascontiguousarray(shared_expert_gate)
    hx = None if hash_experts is None else np.ascontiguousarray(hash_experts, np.int64)
    tok = None if token_ids is None else np.ascontiguousarray(token_ids, np.uint32)
    rf32 = None if router_weight_f32 is None else np.ascontiguousarray(router_weight_f32,
                                                                       np.float32)
    if tok is not None and tok.size != T:
        raise OracleError(SHAPE)
    layer = _Layer(H, E, K, spec.intermediate, spec.shared_intermediate, spec.expert_format,
                   spec.shared_format, spec.router, spec.composition, spec.n_group,
                   spec.topk_group, int(spec.normalize), float(spec.routed_scaling_factor),
                   _ptr(rwt), _ptr(bias), ctypes.addressof(mats),
                   None if sh is None else ctypes.addressof(sh),
                   float(getattr(spec, "swiglu_limit", 0.0)), _ptr(sgate), _ptr(hx),
                   0 if hx is None else hx.shape[0], _ptr(rf32))
    y = np.empty((T, H), np.float32)
    ids = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    logits = np.empty((T, E), np.float32)
    status = _lib.urbo_moe_forward_tokens(ctypes.byref(layer), _ptr(x), _ptr(tok), T, _ptr(y),
                                          _ptr(ids), _ptr(w), _ptr(logits), threads)
    _check(status)
    return OracleResult(y, ids, w, logits)


def _mats(triple):
    mats = (_Matrix * 3)()
    keep = []
    for m in range(3):
        d, s = triple[m]
        keep += [d, s]
        mats[m] = _Matrix(_ptr(d), _ptr(s))
    return mats, keep


def gated_mlp(fmt: int, triple, hidden: int, intermediate: int, x: np.ndarray,
              threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    mats, keep = _mats(triple)
    y = np.empty((x.shape[0], hidden), np.float32)
    _lib.urbo_gated_mlp.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32,
                                    ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32,
                                    ctypes.c_void_p, ctypes.c_int]
    _check(_lib.urbo_gated_mlp(fmt, ctypes.addressof(mats), hidden, intermediate, _ptr(x),
                               x.shape[0], _ptr(y), threads))
    return y


def physical_cores() -> int:
    """recommended_worker_threads (src/execution.rs:254-263): physical cores in the allowed set."""
    return int(_lib.urbo_physical_cores())


def cpu_order() -> list:
    """The allowed logical CPUs, one per physical core first (src/execution.rs:270-330)."""
    buf = (ctypes.c_int * 8192)()
    n = _lib.urbo_cpu_order(buf, 8192)
    return [buf[i] for i in range(min(n, 8192))]


def set_pinning(enable: bool) -> bool:
    """Pin pool worker i to cpu_order()[i] (the reference pool's start_handler); returns the
    previous setting."""
    return bool(_lib.urbo_set_pinning(int(enable)))


def set_mxfp8_fma_host(fma_host: bool) -> bool:
    """MXFP8 matvec kernel of layer calls: the AVX2+FMA host's compact kernel (True, default)
    or the ordered-f64 kernel of other hosts.  Returns the previous setting."""
    return bool(_lib.urbo_set_mxfp8_fma_host(int(fma_host)))


def bounded_swiglu(gate, up, limit: float) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(gate)
    _lib.urbo_bounded_swiglu.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_float, ctypes.c_void_p]
    _check(_lib.urbo_bounded_swiglu(_ptr(gate), _ptr(up), gate.size, float(limit), _ptr(out)))
    return out


def hy4_expert(fmt: int, triple, hidden: int, intermediate: int, x: np.ndarray,
               swiglu_limit: float, threads: int = 1) -> np.ndarray:
    """Hy4 MX-activation expert on [n, hidden] (quantized inside): the routed expert for
    swiglu_limit > 0, the shared DenseMlp for swiglu_limit == 0."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    mats, keep = _mats(triple)
    y = np.empty((x.shape[0], hidden), np.float32)
    _lib.urbo_hy4_expert.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32,
                                     ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32,
                                     ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
    _check(_lib.urbo_hy4_expert(fmt, ctypes.addressof(mats), hidden, intermediate, _ptr(x),
                                x.shape[0], float(swiglu_limit), _ptr(y), threads))
    return y


def dsv41_expert(fmt: int, triple, hidden: int, intermediate: int, x: np.ndarray,
                 swiglu_limit: float, route_weights=None, threads: int = 1) -> np.ndarray:
    """DeepSeek-V4.1 MX-activation expert on [n, hidden] (quantized inside); route_weights [n]
    scale the SwiGLU output before the down projection, None for the shared expert."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    mats, keep = _mats(triple)
    y = np.empty((x.shape[0], hidden), np.float32)
    rw = None if route_weights is None else np.ascontiguousarray(route_weights, np.float32)
    _lib.urbo_dsv41_expert.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32,
                                       ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32,
                                       ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int]
    _check(_lib.urbo_dsv41_expert(fmt, ctypes.addressof(mats), hidden, intermediate, _ptr(x),
                                  x.shape[0], float(swiglu_limit), _ptr(rw), _ptr(y), threads))
    return y


def dsv4_expert(fmt: int, triple, hidden: int, intermediate: int, x: np.ndarray,
                swiglu_limit: float, route_weights=None, threads: int = 1) -> np.ndarray:
    """DeepSeek-V4 expert on [n, hidden]: MX weights read x quantized per 128 values (inside)
    and round to BF16; BF16 and F32 weights read x as it is."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    mats, keep = _mats(triple)
    y = np.empty((x.shape[0], hidden), np.float32)
    rw = None if route_weights is None else np.ascontiguousarray(route_weights, np.float32)
    _check(_lib.urbo_dsv4_expert(fmt, ctypes.addressof(mats), hidden, intermediate, _ptr(x),
                                 x.shape[0], float(swiglu_limit), _ptr(rw), _ptr(y), threads))
    return y


def qwen_expert(triple, hidden: int, intermediate: int, x: np.ndarray,
                threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    mats, keep = _mats(triple)
    y = np.empty((x.shape[0], hidden), np.float32)
    _lib.urbo_qwen_expert.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                      ctypes.c_int]
    _check(_lib.urbo_qwen_expert(ctypes.addressof(mats), hidden, intermediate, _ptr(x),
                                 x.shape[0], _ptr(y), threads))
    return y


def zc_rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, round_bf16: bool = True) -> np.ndarray:
    """zero_centered_rms_norm of every row of x [n, H], then (round_bf16) the Qwen3.6 runtime's
    BF16 cast (src/models/qwen3_8/norm.rs:38-52; src/models/qwen3_6/runtime.rs:1053-1057)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(x)
    _lib.urbo_zc_rms_norm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_size_t, ctypes.c_float, ctypes.c_int,
                                      ctypes.c_void_p]
    _check(_lib.urbo_zc_rms_norm(_ptr(x), _ptr(weight), x.shape[0], x.shape[1], float(eps),
                                 int(round_bf16), _ptr(out)))
    return out


def add_residual_bf16(residual: np.ndarray, update: np.ndarray) -> np.ndarray:
    """add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494)."""
    out = np.array(residual, dtype=np.float32, copy=True, order="C")
    update = np.ascontiguousarray(update, dtype=np.float32)
    _lib.urbo_add_residual_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    _check(_lib.urbo_add_residual_bf16(_ptr(out), _ptr(update), out.size))
    return out
