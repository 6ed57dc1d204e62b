"""Seeded synthetic workloads for the MoE layer (host/numpy side).

Generator definition (shared bit for bit with the device generator in ``csrc/urb_synth.hip``):

* PRNG: SplitMix64 exactly as the reference's ``SplitMix64`` (src/generation.rs:419-440).  The
  n-th output of a stream with seed ``s`` is ``mix(s + (n + 1) * 0x9e3779b97f4a7c15)``, so any
  element can be generated independently.  ``unit_f64`` is ``(u >> 11) * 2**-53``.
* One stream per tensor: ``seed = base_seed ^ fnv1a64(tensor_name)``.
* Normals: Box-Muller on draws ``2i`` and ``2i + 1``:
  ``z = sqrt(-2 ln(1 - u0)) * cos(2 pi u1)`` in f64, then ``mean + std * z`` cast to f32.
* BF16 tensors: normals rounded to BF16 with round-to-nearest-even.
* MXFP4: nibble ``i`` = draw ``i`` & 0xF, two nibbles per byte, low nibble first; E8M0 scales
  from the stream ``<name>.scales``: ``119 + draw % 7`` (2^-8 .. 2^-2).
* MXFP8: E4M3 = nearest-even finite E4M3 encoding of ``clamp(N(0,1), +-448)``; scales as MXFP4.
"""

from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
MIX1 = np.uint64(0xBF58476D1CE4E5B9)
MIX2 = np.uint64(0x94D049BB133111EB)
BASE_SEED = 0x5EED2026
SCALE_LO, SCALE_SPAN = 119, 7


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_seed(name: str, base_seed: int = BASE_SEED) -> int:
    return (base_seed ^ fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs ``start .. start+count`` of the SplitMix64 stream seeded with ``seed``."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * MIX1
        z = (z ^ (z >> np.uint64(27))) * MIX2
        return z ^ (z >> np.uint64(31))


def unit_f64(u: np.ndarray) -> np.ndarray:
    return (u >> np.uint64(11)).astype(np.float64) * (1.0 / float(1 << 53))


def normals(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    d = splitmix64(seed, 0, 2 * count)
    u0 = unit_f64(d[0::2])
    u1 = unit_f64(d[1::2])
    z = np.sqrt(-2.0 * np.log(1.0 - u0)) * np.cos(2.0 * np.pi * u1)
    return (mean + std * z).astype(np.float32)


def bf16_rne_bits(values: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even BF16 bits of finite f32 values."""
    b = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_values(values: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_rne_bits(values))


def encode_e4m3fn(values: np.ndarray) -> np.ndarray:
    """Nearest-even finite E4M3FN code of f32 values, saturating at +-448."""
    v = np.clip(np.asarray(values, dtype=np.float32), -448.0, 448.0)
    mag = np.abs(v)
    sub = np.rint(mag * np.float32(512.0)).astype(np.uint32)  # exact 2^-9 grid below 2^-6
    bits = mag.view(np.uint32)
    rounded = (bits + np.uint32((1 << 19) - 1) + ((bits >> np.uint32(20)) & np.uint32(1))) \
        & np.uint32(0xFFF00000)
    exponent = (rounded >> np.uint32(23)) & np.uint32(0xFF)
    exponent = np.where(exponent > 120, exponent - np.uint32(120), np.uint32(0))
    normal = np.minimum((exponent << np.uint32(3)) | ((rounded >> np.uint32(20)) & np.uint32(7)),
                        np.uint32(0x7E))
    code = np.where(mag < np.float32(2.0 ** -6), sub, normal)
    code = np.where((np.signbit(v)) & (code != 0), code | np.uint32(0x80), code)
    code = np.where(mag == 0, np.uint32(0), code)
    return code.astype(np.uint8)


def e8m0_scales(name: str, rows: int, cols: int, base_seed: int = BASE_SEED) -> np.ndarray:
    groups = (cols + 31) // 32
    d = splitmix64(stream_seed(name + ".scales", base_seed), 0, rows * groups)
    return (np.uint64(SCALE_LO) + d % np.uint64(SCALE_SPAN)).astype(np.uint8).reshape(rows, groups)


def mxfp4_matrix(name: str, rows: int, cols: int, base_seed: int = BASE_SEED):
    assert cols % 2 == 0
    d = splitmix64(stream_seed(name, base_seed), 0, rows * cols)
    nib = (d & np.uint64(0xF)).astype(np.uint8).reshape(rows, cols)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << np.uint8(4))).astype(np.uint8)
    return np.ascontiguousarray(packed), e8m0_scales(name, rows, cols, base_seed)


def mxfp8_matrix(name: str, rows: int, cols: int, base_seed: int = BASE_SEED):
    z = normals(stream_seed(name, base_seed), rows * cols, 0.0, 1.0)
    codes = encode_e4m3fn(z).reshape(rows, cols)
    return np.ascontiguousarray(codes), e8m0_scales(name, rows, cols, base_seed)


def bf16_matrix(name: str, rows: int, cols: int, std: float = 0.02,
                base_seed: int = BASE_SEED) -> np.ndarray:
    z = normals(stream_seed(name, base_seed), rows * cols, 0.0, std)
    return bf16_rne_bits(z).reshape(rows, cols)


def activations(name: str, tokens: int, hidden: int, base_seed: int = BASE_SEED) -> np.ndarray:
    """N(0, 1) activations rounded to BF16, returned as f32 values [tokens, hidden]."""
    z = normals(stream_seed(name, base_seed), tokens * hidden, 0.0, 1.0)
    return bf16_values(z).reshape(tokens, hidden)
