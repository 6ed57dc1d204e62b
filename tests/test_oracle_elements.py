"""Pins the oracle's element decoders/encoders against the reference's known-answer tests,
closed forms and an independent library (torch's float8/bfloat16 conversions)."""

import json
import math
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def fbits(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


def test_e8m0_all_codes_are_powers_of_two():
    # src/math/mxfp.rs:2217-2224: decode(code) == 2^(code-127) for every finite code.
    for code in range(255):
        assert bits(O.decode_e8m0(code)) == bits(math.ldexp(1.0, code - 127)), code
    with pytest.raises(O.OracleError) as e:
        O.decode_e8m0(255)
    assert e.value.status == O.INVALID_SCALE


def test_e8m0_code_zero_is_the_midpoint_subnormal():
    assert bits(O.decode_e8m0(0)) == 0x00400000


def test_real_checkpoint_prefix_kat():
    k = KATS["e4m3_e8m0_prefix"]
    assert O.decode_e4m3fn(k["e4m3_code"]) == k["e4m3_value"]
    assert O.decode_e8m0(k["e8m0_code"]) == k["e8m0_value"]
    assert np.float32(O.decode_e4m3fn(k["e4m3_code"]) * O.decode_e8m0(k["e8m0_code"])) == k["product"]


def _e2m1_closed_form(code: int) -> float:
    # OCP MX E2M1: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0; exponent 0 is
    # subnormal (m * 0.5).
    s = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    v = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
    return s * v


def test_e2m1_table_matches_ocp_definition():
    for code in range(16):
        expect = _e2m1_closed_form(code)
        got = O.decode_e2m1(code)
        assert got == expect, code
    # code 8 decodes to +0.0, not -0.0 (src/math/mxfp.rs:73-79)
    assert bits(float(O.decode_e2m1(8))) == 0


def test_mxfp4_low_nibble_first_kat():
    k = KATS["mxfp4_low_nibble_first"]
    packed = np.array(k["packed"], np.uint8)
    scales = np.array(k["scales"], np.uint8)
    r = O.row(O.FMT_MXFP4, packed, scales, k["rows"], k["cols"], 0)
    assert [bits(float(v)) for v in r] == [bits(v) for v in k["row"]]
    assert O.validate(O.FMT_MXFP4, packed, np.array(k["invalid_scales"], np.uint8), 1, 2) == O.INVALID_SCALE


def test_e4m3_all_codes_match_torch_float8_e4m3fn():
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        got = float(O.decode_e4m3fn(c))
        if c & 0x7F == 0x7F:
            assert math.isnan(got) and math.isnan(ref[c])
        else:
            assert bits(got) == bits(float(ref[c])), hex(c)


def _e4m3_table():
    return np.array([O.decode_e4m3fn(c) for c in range(256)], np.float32)


def _nearest_finite_code(v: float, table) -> int:
    # Brute force: smallest distance over every finite code, ties to the even code
    # (the reference's exhaustive check, src/math/mxfp.rs:2958-2981 / :279-298).
    best, bestd = 0, math.inf
    v = min(max(v, -448.0), 448.0)
    for c in range(0xFF):
        d = table[c]
        if not math.isfinite(d):
            continue
        dist = abs(float(d) - v)
        if dist < bestd or (dist == bestd and c % 2 == 0 and best % 2 == 1):
            best, bestd = c, dist
    return best


def test_e4m3_encoder_matches_exhaustive_nearest_even():
    table = _e4m3_table()
    vals = [float(table[c]) for c in range(0xFF) if math.isfinite(table[c])]
    for c in range(0x7E):
        mid = float(np.float32((table[c] + table[c + 1]) * np.float32(0.5)))
        vals += [mid, -mid]
    rng = np.random.default_rng(7)
    vals += list(rng.standard_normal(2000).astype(np.float32) * 100)
    vals += [500.0, -1e9, 1e-30, -1e-30]
    for v in vals:
        v32 = float(np.float32(v))
        got = O.encode_e4m3fn_finite(v32)
        exp = _nearest_finite_code(v32, table)
        # -0.0 and tiny negatives that round to zero encode as +0 (code 0)
        if exp == 0x80:
            exp = 0
        assert got == exp, (v32, got, exp)


def test_power_of_two_ceiling_interior_and_boundaries():
    # Interior mantissas: the next power of two exactly (src/math/mxfp.rs:300-319).
    for e in range(1, 254):
        for m in (4097, 0x12345, 0x7FFFFF - 4097):
            v = fbits((e << 23) | m)
            assert bits(float(O.power_of_two_ceiling(v))) == ((e + 1) << 23)
    # Exact powers are returned unchanged.
    for e in range(1, 254):
        v = fbits(e << 23)
        assert O.power_of_two_ceiling(v) == v
    # Boundary band: the reference keeps 2^ceil(log2 v) computed in f32, which lands on one of
    # the two bracketing powers of two.
    for e in range(1, 254):
        for m in (1, 4096, 0x7FFFFF - 4096, 0x7FFFFF):
            v = fbits((e << 23) | m)
            got = float(O.power_of_two_ceiling(v))
            assert got in (math.ldexp(1.0, e - 127), math.ldexp(1.0, e - 126)), (e, m, got)


def test_e4m3_activation_simulation_kat():
    k = KATS["e4m3_activation_blocks"]
    out = O.simulate_e4m3_activation(np.array(k["input"], np.float32), k["block"])
    for i, v in k["expect_exact"].items():
        assert out[int(i)] == v
    with pytest.raises(O.OracleError):
        O.simulate_e4m3_activation(np.array([1.0, np.nan, 2.0], np.float32), 2)


def test_bf16_ties_to_even_kat():
    for value, expect in KATS["bf16_ties_to_even"]["cases"]:
        assert O.round_to_bf16(value) == expect


def test_bf16_rounding_matches_torch_on_every_high_half():
    torch = pytest.importorskip("torch")
    highs = np.arange(65536, dtype=np.uint32)
    for low in (0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF):
        b = (highs << 16) | np.uint32(low)
        v = b.view(np.float32)
        ref = torch.from_numpy(v.copy()).to(torch.bfloat16).float().numpy()
        arr = v.copy()
        finite_in = np.isfinite(v)
        finite_out = np.isfinite(ref)
        ok = finite_in & finite_out
        # Scalar oracle on every element that the reference accepts.
        got = np.array([O.round_to_bf16(float(x)) for x in v[ok][::97]], np.float32)
        assert np.array_equal(got.view(np.uint32), ref[ok][::97].view(np.uint32))
        # In-place form: rounding all accepted values gives torch's bits.
        acc = np.ascontiguousarray(v[ok])
        assert O.round_to_bf16_in_place(acc) == O.OK
        assert np.array_equal(acc.view(np.uint32), ref[ok].view(np.uint32))
        del arr


def test_bf16_rounding_rejects_nonfinite_and_overflow_and_keeps_prefix():
    for inv in KATS["bf16_rounding_rejects"]["invalid_bits"]:
        with pytest.raises(O.OracleError):
            O.round_to_bf16(fbits(inv))
        for pos in (0, 5, 33):
            vals = np.full(36, 1.003, np.float32)
            vals[pos + 1] = fbits(inv)
            before = vals.copy()
            st = O.round_to_bf16_in_place(vals[1:35].copy())
            assert st == O.NONFINITE
            work = vals.copy()
            sub = work[1:35]
            sub_c = np.ascontiguousarray(sub)
            O.round_to_bf16_in_place(sub_c)
            # elements before the failure are rounded, the failing one and the rest untouched
            assert np.all(sub_c[:pos] == np.float32(1.0)) or pos == 0
            assert np.array_equal(sub_c[pos:].view(np.uint32), before[1 + pos:35].view(np.uint32))


def test_silu_closed_form():
    for v in (-5.0, -1.0, 0.0, 0.5, 3.0):
        assert abs(float(O.silu(v)) - v / (1 + math.exp(-v))) < 1e-6
