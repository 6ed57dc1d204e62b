"""ctypes binding of the C ABI in ``include/urb_moe.h`` (``liburb_moe.so``) and of the device
workload generator (``liburb_synth.so``).

The shared libraries are built in-tree by ``__graft_entry__.build()``.  Loading fails loudly
when they are missing: there is no CPU fallback for any entry point.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
MOE_LIB = os.path.join(_HERE, "liburb_moe.so")
SYNTH_LIB = os.path.join(_HERE, "liburb_synth.so")

OK, ERR_SHAPE, ERR_INVALID_SCALE, ERR_NONFINITE, ERR_INVALID_GEOMETRY = 0, 1, 2, 3, 4
ERR_DEVICE, ERR_OUT_OF_MEMORY, ERR_ARGUMENT = 5, 6, 7
SOURCE_HOST, SOURCE_DEVICE_COPY, SOURCE_DEVICE_BORROW = 0, 1, 2

# Every symbol include/urb_moe.h declares.
EXPORTS = ("urb_moe_create", "urb_moe_destroy", "urb_moe_forward", "urb_moe_route",
           "urb_moe_sync", "urb_dequant_rows", "urb_moe_memory", "urb_status_string",
           "urb_moe_profile", "urb_moe_profile_read", "urb_pack_matrix", "urb_quantize_e4m3",
           "urb_expert_views", "urb_moe_forward_block", "urb_zc_rms_norm_bf16",
           "urb_moe_set_expert", "urb_moe_forward_tokens", "urb_moe_route_tokens",
           "urb_quantize_e4m3_blocks", "urb_gemm_placement", "urb_moe_forward_noalloc",
           "urb_inspect_matrix")
STAGES = ("router", "route", "permute", "gate_up", "down", "shared_gate_up", "shared_down",
          "combine")
SYNTH_EXPORTS = ("urb_synth_bf16", "urb_synth_activations", "urb_synth_fp4", "urb_synth_fp8",
                 "urb_synth_e8m0", "urb_probe_mfma_16x16x32", "urb_probe_cvt_bf16",
                 "urb_probe_mfma_scale_16x16x128", "urb_probe_split_bf16")


class UrbError(RuntimeError):
    """A non-OK urb_status, carrying the code (1..4 mirror the reference's error enums)."""

    def __init__(self, status: int, where: str = ""):
        msg = _status_string(status)
        super().__init__(f"{where}: urb_status {status} ({msg})" if where else msg)
        self.status = status


class Matrix(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


class Desc(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_uint32), ("n_experts", ctypes.c_uint32),
        ("top_k", ctypes.c_uint32), ("intermediate", ctypes.c_uint32),
        ("shared_intermediate", ctypes.c_uint32),
        ("expert_format", ctypes.c_int), ("shared_format", ctypes.c_int),
        ("router", ctypes.c_int), ("composition", ctypes.c_int),
        ("n_group", ctypes.c_uint32), ("topk_group", ctypes.c_uint32),
        ("normalize", ctypes.c_int32), ("routed_scaling_factor", ctypes.c_float),
        ("max_tokens", ctypes.c_uint32), ("swiglu_limit", ctypes.c_float),
    ]


DTYPES = {"BF16": 0, "F16": 1, "F32": 2, "F8_E4M3": 3, "I8": 4, "U8": 5, "F8_E8M0": 6}


class TensorMeta(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("ndim", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 2), ("data_len", ctypes.c_uint64)]


class Weights(ctypes.Structure):
    _fields_ = [("router_weight", ctypes.c_void_p), ("correction_bias", ctypes.c_void_p),
                ("experts", ctypes.c_void_p), ("shared", ctypes.c_void_p),
                ("shared_expert_gate", ctypes.c_void_p),
                ("hash_experts", ctypes.c_void_p), ("hash_vocab", ctypes.c_uint32)]


_moe = None
_synth = None


def _status_string(status: int) -> str:
    try:
        return moe_lib().urb_status_string(status).decode()
    except Exception:
        return "unknown"


def moe_lib() -> ctypes.CDLL:
    global _moe
    if _moe is None:
        if not os.path.exists(MOE_LIB):
            raise RuntimeError(f"{MOE_LIB} is not built: run __graft_entry__.build() "
                               "(the MoE path has no CPU fallback)")
        lib = ctypes.CDLL(MOE_LIB)
        P, u32 = ctypes.c_void_p, ctypes.c_uint32
        lib.urb_moe_create.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(Weights), ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_void_p)]
        lib.urb_moe_create.restype = ctypes.c_int
        lib.urb_moe_destroy.argtypes = [P]
        lib.urb_moe_destroy.restype = None
        lib.urb_moe_forward.argtypes = [P, P, u32, P, P, P, P]
        lib.urb_moe_forward.restype = ctypes.c_int
        lib.urb_moe_route.argtypes = [P, P, u32, P, P, P, P]
        lib.urb_moe_route.restype = ctypes.c_int
        lib.urb_moe_forward_noalloc.argtypes = [P, P, u32, P, P, P, P]
        lib.urb_moe_forward_noalloc.restype = ctypes.c_int
        lib.urb_moe_forward_tokens.argtypes = [P, P, P, u32, P, P, P, P]
        lib.urb_moe_forward_tokens.restype = ctypes.c_int
        lib.urb_moe_route_tokens.argtypes = [P, P, P, u32, P, P, P, P]
        lib.urb_moe_route_tokens.restype = ctypes.c_int
        lib.urb_moe_sync.argtypes = [P, P]
        lib.urb_moe_sync.restype = ctypes.c_int
        lib.urb_dequant_rows.argtypes = [ctypes.c_int, P, P, u32, u32, u32, u32, P, P]
        lib.urb_dequant_rows.restype = ctypes.c_int
        lib.urb_moe_memory.argtypes = [P, ctypes.POINTER(ctypes.c_size_t),
                                       ctypes.POINTER(ctypes.c_size_t)]
        lib.urb_moe_memory.restype = ctypes.c_int
        lib.urb_moe_profile.argtypes = [P, ctypes.c_int]
        lib.urb_moe_profile.restype = ctypes.c_int
        lib.urb_moe_profile_read.argtypes = [P, P, P]
        lib.urb_moe_profile_read.restype = ctypes.c_int
        lib.urb_pack_matrix.argtypes = [ctypes.c_int, P, P, u32, u32, P, P, P]
        lib.urb_pack_matrix.restype = ctypes.c_int
        lib.urb_quantize_e4m3.argtypes = [P, u32, u32, P, P, P]
        lib.urb_quantize_e4m3.restype = ctypes.c_int
        lib.urb_quantize_e4m3_blocks.argtypes = [P, u32, u32, u32, P, P, P]
        lib.urb_quantize_e4m3_blocks.restype = ctypes.c_int
        lib.urb_moe_set_expert.argtypes = [P, u32, P, P]
        lib.urb_moe_set_expert.restype = ctypes.c_int
        lib.urb_moe_forward_block.argtypes = [P, P, P, ctypes.c_float, u32, P, P, P, P]
        lib.urb_moe_forward_block.restype = ctypes.c_int
        lib.urb_zc_rms_norm_bf16.argtypes = [P, P, u32, u32, ctypes.c_float, P, P]
        lib.urb_zc_rms_norm_bf16.restype = ctypes.c_int
        lib.urb_expert_views.argtypes = [ctypes.c_int, u32, u32, u32, P, P, P, P, P]
        lib.urb_expert_views.restype = ctypes.c_int
        lib.urb_inspect_matrix.argtypes = [P, P, ctypes.c_int, u32, u32,
                                           ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(ctypes.c_uint64)]
        lib.urb_inspect_matrix.restype = ctypes.c_int
        lib.urb_gemm_placement.argtypes = [ctypes.c_int, ctypes.c_int, u32, u32, u32, u32, P, P,
                                           u32]
        lib.urb_gemm_placement.restype = u32
        lib.urb_status_string.argtypes = [ctypes.c_int]
        lib.urb_status_string.restype = ctypes.c_char_p
        for f in EXPORTS:
            if getattr(lib, f).argtypes is None:
                raise RuntimeError(f"{f}: no ctypes signature")
        _moe = lib
    return _moe


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(SYNTH_LIB)
        P, sz, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64
        lib.urb_synth_bf16.argtypes = [u64, sz, ctypes.c_double, ctypes.c_double, P, P]
        lib.urb_synth_activations.argtypes = [u64, sz, P, P]
        lib.urb_synth_fp4.argtypes = [u64, sz, P, P]
        lib.urb_synth_fp8.argtypes = [u64, sz, P, P]
        lib.urb_synth_e8m0.argtypes = [u64, sz, P, P]
        lib.urb_probe_mfma_16x16x32.argtypes = [P, P, P, P]
        lib.urb_probe_cvt_bf16.argtypes = [ctypes.c_int, P, P, ctypes.c_int, P, P]
        lib.urb_probe_mfma_scale_16x16x128.argtypes = [ctypes.c_int, P, P, P, P, P, P]
        lib.urb_probe_split_bf16.argtypes = [P, ctypes.c_int, P, P, P]
        for f in SYNTH_EXPORTS:
            # without argtypes ctypes would pass a device pointer as a 32-bit int
            if getattr(lib, f).argtypes is None:
                raise RuntimeError(f"{f}: no ctypes signature")
            getattr(lib, f).restype = ctypes.c_int
        _synth = lib
    return _synth


def check(status: int, where: str = "") -> None:
    if status != OK:
        raise UrbError(status, where)


def inspect_matrix(weight: dict, scale: Optional[dict], rows: int, cols: int,
                   packed_name: bool = False):
    """urb_inspect_matrix on safetensors header entries ({"dtype", "shape", "data_offsets"} or
    {"dtype", "shape", "data_len"}): (urb_format, resident bytes); raises UrbError."""
    def meta(e):
        shape = list(e["shape"])
        n = e["data_len"] if "data_len" in e else e["data_offsets"][1] - e["data_offsets"][0]
        return TensorMeta(DTYPES.get(e["dtype"], 7), len(shape),
                          (ctypes.c_uint64 * 2)(*(shape + [0, 0])[:2]), n)
    w = meta(weight)
    s = meta(scale) if scale is not None else None
    fmt, rb = ctypes.c_int(), ctypes.c_uint64()
    check(moe_lib().urb_inspect_matrix(ctypes.byref(w), None if s is None else ctypes.byref(s),
                                       int(packed_name), rows, cols, ctypes.byref(fmt),
                                       ctypes.byref(rb)), "urb_inspect_matrix")
    return fmt.value, rb.value
