"""GPU parity tests: the HIP path through the C ABI against the CPU oracle on the same seeded
inputs.  Bars: dequantised weights bit-exact; top-k ids identical except near-ties (< 1e-6);
layer outputs within 1e-3 relative L2."""

import math
import os
from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from urbilateria_amd import configs as C
from urbilateria_amd import native as N
from urbilateria_amd import synth

from .gpu_helpers import REL_L2_BAR, ids_match, noaux_scores, rel_l2, sqrt_softplus_scores

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu(require_gpu):
    from urbilateria_amd import moe  # noqa: F401  (fails loudly without liburb_moe.so)
    torch.cuda.set_device(0)
    yield


def moe_mod():
    from urbilateria_amd import moe
    return moe


def _oracle(host: C.HostLayer, x: np.ndarray, threads: int = 4, token_ids=None):
    return O.moe_forward(host.spec, host.experts, host.router_weight, x, host.correction_bias,
                         host.shared, threads=threads,
                         shared_expert_gate=host.shared_expert_gate, token_ids=token_ids,
                         hash_experts=host.hash_experts)


def _scores(spec, res, bias):
    if spec.router == C.ROUTER_SOFTMAX_TOPK:
        return res.logits
    if spec.router == C.ROUTER_SQRT_SOFTPLUS:
        return sqrt_softplus_scores(res.logits, bias)
    return noaux_scores(res.logits, bias)


# ------------------------------------------------------------------------------- dequant
def test_mxfp4_dequant_bit_exact_every_code_and_scale():
    rows, cols = 255, 32
    nib = np.tile(np.arange(16, dtype=np.uint8), 2)
    packed = np.tile((nib[0::2] | (nib[1::2] << 4)).astype(np.uint8), (rows, 1))
    scales = np.arange(255, dtype=np.uint8).reshape(rows, 1)
    got = moe_mod().dequant_rows(C.FMT_MXFP4, torch.from_numpy(packed).cuda(),
                                 torch.from_numpy(scales).cuda(), rows, cols).cpu().numpy()
    ref = np.stack([O.row(O.FMT_MXFP4, packed, scales, rows, cols, r) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_mxfp8_dequant_bit_exact_every_code_and_scale():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)  # 254 finite codes
    cols = 256
    row = np.zeros(cols, np.uint8)
    row[:len(codes)] = codes
    rows = 255
    data = np.tile(row, (rows, 1))
    scales = np.repeat(np.arange(255, dtype=np.uint8).reshape(rows, 1), cols // 32, axis=1)
    got = moe_mod().dequant_rows(C.FMT_MXFP8, torch.from_numpy(data).cuda(),
                                 torch.from_numpy(np.ascontiguousarray(scales)).cuda(), rows,
                                 cols).cpu().numpy()
    ref = np.stack([O.row(O.FMT_MXFP8, data, scales, rows, cols, r) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_bf16_dequant_bit_exact_every_finite_encoding():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7F80) != 0x7F80
    data = bits[finite]
    data = data[: len(data) // 64 * 64].reshape(-1, 64)
    got = moe_mod().dequant_rows(C.FMT_BF16, torch.from_numpy(data.view(np.int16)).cuda(), None,
                                 data.shape[0], 64).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), data.astype(np.uint32) << 16)


def test_device_generator_matches_host_generator():
    spec = C.small_spec(C.WORKLOADS["c4_mxfp8"].spec, hidden=128, n_experts=4, intermediate=64)
    dev = moe_mod().DeviceLayer.synthesize(spec).to_host()
    host = C.make_host_layer(spec)
    assert np.array_equal(dev.router_weight, host.router_weight)
    for e in range(spec.n_experts):
        for m in range(3):
            assert np.array_equal(dev.experts[e][m][0].ravel(), host.experts[e][m][0].ravel())
            assert np.array_equal(dev.experts[e][m][1].ravel(), host.experts[e][m][1].ravel())
    spec4 = C.small_spec(C.WORKLOADS["c3_mxfp4_decode"].spec, hidden=128, n_experts=4,
                         intermediate=64)
    dev4 = moe_mod().DeviceLayer.synthesize(spec4).to_host()
    host4 = C.make_host_layer(spec4)
    for e in range(spec4.n_experts):
        for m in range(3):
            assert np.array_equal(dev4.experts[e][m][0].ravel(), host4.experts[e][m][0].ravel())
    for m in range(3):
        assert np.array_equal(dev4.shared[m][0].ravel(), host4.shared[m][0].view(np.uint8).ravel())
    x = moe_mod().synth_activations(3, 128).cpu().numpy()
    assert np.array_equal(x, synth.activations("x", 3, 128))


# ------------------------------------------------------------------------------- CDNA4 builtins
def test_mfma_16x16x32_bf16_lane_layout():
    # The GEMM kernels assume: A lane l = row l%16, k 8*(l/16)+[0,8); B lane l = column l%16,
    # same k; C lane l = column l%16, rows 4*(l/16)+[0,4).  Small integers are exact in BF16.
    rng = np.random.default_rng(1)
    A = rng.integers(-3, 4, (16, 32)).astype(np.float32)
    B = rng.integers(-3, 4, (32, 16)).astype(np.float32)
    a, b = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    c = torch.zeros((16, 16), device="cuda")
    N.check(N.synth_lib().urb_probe_mfma_16x16x32(a.data_ptr(), b.data_ptr(), c.data_ptr(), None))
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), A @ B)


@pytest.mark.parametrize("fmt", [C.FMT_MXFP4, C.FMT_MXFP8])
def test_mfma_scale_16x16x128_operands(fmt):
    # One scaled-MFMA step of the MX-activation kernels, operands built by their own helpers:
    # A = row-major E4M3 codes with E8M0 block scales, B = one weight panel step as the panel
    # lanes load it.  Codes of magnitude 0.5 .. 3.75 (E2M1: 0 .. 6) and scales 2^-1 .. 2^1 make
    # every product a multiple of 2^-10 below 2^6, so every partial sum is exact in f32 and C
    # must equal A.B^T exactly in any summation order.
    rng = np.random.default_rng(7)
    fin8 = np.array([c for c in range(256) if 48 <= (c & 0x7F) <= 71], np.uint8)
    dec8 = np.array([O.decode_e4m3fn(c) for c in range(256)], np.float64)
    A = rng.choice(fin8, (16, 128)).astype(np.uint8)
    sa = rng.integers(126, 129, (16, 4)).astype(np.uint8)
    sb = rng.integers(126, 129, (16, 4)).astype(np.uint8)
    Av = dec8[A] * np.exp2(np.repeat(sa.astype(np.float64) - 127, 32, axis=1))
    if fmt == C.FMT_MXFP8:
        Bc = rng.choice(fin8, (16, 128)).astype(np.uint8)
        Bv = dec8[Bc]
        Bbytes = Bc
    else:
        Bc = rng.integers(0, 16, (16, 128)).astype(np.uint8)
        Bv = np.array([O.decode_e2m1(int(c)) for c in Bc.ravel()], np.float64).reshape(16, 128)
        Bbytes = (Bc[:, 0::2] | (Bc[:, 1::2] << 4)).astype(np.uint8)
    Bv = Bv * np.exp2(np.repeat(sb.astype(np.float64) - 127, 32, axis=1))
    dev = [torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in (A, sa, Bbytes, sb)]
    c = torch.zeros((16, 16), device="cuda")
    N.check(N.synth_lib().urb_probe_mfma_scale_16x16x128(
        fmt, *(d.data_ptr() for d in dev), c.data_ptr(), None))
    torch.cuda.synchronize()
    got = c.cpu().numpy().astype(np.float64)
    ref = Av @ Bv.T
    assert np.array_equal(got, ref), float(np.abs(got - ref).max())


@pytest.mark.parametrize("fmt", [C.FMT_MXFP4, C.FMT_MXFP8])
def test_mfma_scale_16x16x128_accumulates_below_f32_accuracy(fmt):
    # Why the MX-activation compositions run on the BF16 MFMA instead of
    # v_mfma_scale_f32_16x16x128_f8f6f4: on full-range operands (every finite E4M3 code, E2M1 or
    # E4M3 weights, E8M0 scales 2^-10 .. 2^10) its 128-term dot products miss the exact sum by
    # more than any f32 summation order can (a sequential f32 sum of 128 exact products is off
    # by at most 127 * 2^-24 of the sum of their magnitudes).  200 random steps; the error is
    # |C - exact| / sum_k |a_k b_k| per output.
    rng = np.random.default_rng(11)
    fin8 = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    dec8 = np.array([O.decode_e4m3fn(c) for c in range(256)], np.float64)
    dec4 = np.array([O.decode_e2m1(c) for c in range(16)], np.float64)
    worst, errs = 0.0, []
    for _ in range(200):
        A = rng.choice(fin8, (16, 128)).astype(np.uint8)
        sa = rng.integers(117, 138, (16, 4)).astype(np.uint8)
        sb = rng.integers(117, 138, (16, 4)).astype(np.uint8)
        if fmt == C.FMT_MXFP8:
            Bc = rng.choice(fin8, (16, 128)).astype(np.uint8)
            Bv, Bbytes = dec8[Bc], Bc
        else:
            Bc = rng.integers(0, 16, (16, 128)).astype(np.uint8)
            Bv = dec4[Bc]
            Bbytes = (Bc[:, 0::2] | (Bc[:, 1::2] << 4)).astype(np.uint8)
        Av = dec8[A] * np.exp2(np.repeat(sa.astype(np.float64) - 127, 32, axis=1))
        Bv = Bv * np.exp2(np.repeat(sb.astype(np.float64) - 127, 32, axis=1))
        dev = [torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in (A, sa, Bbytes, sb)]
        c = torch.zeros((16, 16), device="cuda")
        N.check(N.synth_lib().urb_probe_mfma_scale_16x16x128(
            fmt, *(d.data_ptr() for d in dev), c.data_ptr(), None))
        torch.cuda.synchronize()
        got = c.cpu().numpy().astype(np.float64)
        mag = np.abs(Av) @ np.abs(Bv).T
        e = np.abs(got - Av @ Bv.T) / np.where(mag > 0, mag, 1.0)
        errs.append(float(e.max()))
    worst = max(errs)
    f32_bound = 127 * 2.0 ** -24
    print(f"\nscaled MFMA 16x16x128 ({'E4M3 x E2M1' if fmt == C.FMT_MXFP4 else 'E4M3 x E4M3'}): "
          f"max error {worst:.3g}, median of step maxima {np.median(errs):.3g} of sum|a b|; "
          f"f32 sequential-sum bound {f32_bound:.3g}")
    assert worst > f32_bound
    assert worst < 1e-3


def _bf16_rne_bits(x):
    """Round-to-nearest-even BF16 bits of finite float32 values (the textbook bit formula)."""
    b = x.view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_activation_split_is_round_to_nearest_even_hi_and_lo():
    # The grouped GEMM stages f32 activations as hi = bf16(x), lo = bf16(x - hi) through the
    # hardware pack conversion.  Exact against the RNE bit formula for normal values of every
    # magnitude, halfway ties, f32 denormals, signed zeros and the overflow to infinity.
    rng = np.random.default_rng(7)
    parts = [
        (rng.standard_normal(20000) * np.exp2(rng.integers(-126, 127, 20000))).astype(np.float32),
        # ties: bf16 value plus exactly half an ulp (even and odd lower neighbours)
        ((rng.integers(0, 1 << 16, 4000, dtype=np.uint32) << 16) | 0x8000).view(np.float32),
        rng.integers(1, 1 << 23, 4000, dtype=np.uint32).view(np.float32),       # denormals
        (rng.integers(1, 1 << 23, 4000, dtype=np.uint32) | (1 << 31)).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, np.finfo(np.float32).max, -np.finfo(np.float32).max,
                  np.finfo(np.float32).tiny, 3.0e38, 1e-45, -1e-45], np.float32),
    ]
    x = np.concatenate(parts)
    x = x[np.isfinite(x)]
    x = x[: x.size // 2 * 2]
    hi_ref = _bf16_rne_bits(x)
    with np.errstate(invalid="ignore", over="ignore"):
        rest = (x - (hi_ref.astype(np.uint32) << 16).view(np.float32)).astype(np.float32)
    lo_ref = _bf16_rne_bits(rest)
    xd = torch.from_numpy(x).cuda()
    hi = torch.empty(x.size, dtype=torch.int16, device="cuda")
    lo = torch.empty(x.size, dtype=torch.int16, device="cuda")
    N.check(N.synth_lib().urb_probe_split_bf16(xd.data_ptr(), x.size, hi.data_ptr(),
                                               lo.data_ptr(), None))
    torch.cuda.synchronize()
    assert np.array_equal(hi.cpu().numpy().view(np.uint16), hi_ref)
    assert np.array_equal(lo.cpu().numpy().view(np.uint16), lo_ref)


def _probe_cvt(fmt, codes, scales):
    out = torch.empty(codes.size, dtype=torch.int16, device="cuda")
    c_dev = torch.from_numpy(codes).cuda()   # held: a dropped temporary's block can be reused
    s_dev = torch.from_numpy(scales).cuda()
    N.check(N.synth_lib().urb_probe_cvt_bf16(fmt, c_dev.data_ptr(), s_dev.data_ptr(),
                                             codes.size, out.data_ptr(), None))
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("fmt", [C.FMT_MXFP4, C.FMT_MXFP8])
def test_scaled_bf16_conversion_matches_dequantised_weights(fmt):
    # The GEMM B path converts code * 2^(s-127) straight to BF16.  Wherever the reference's f32
    # weight is finite and a BF16 value, the conversion must give exactly it (up to the sign of
    # zero, which no dot product can observe).
    ncode = 16 if fmt == C.FMT_MXFP4 else 256
    codes = np.repeat(np.arange(ncode, dtype=np.uint8), 255)
    scales = np.tile(np.arange(255, dtype=np.uint8), ncode)
    keep = np.ones(codes.size, bool) if fmt == C.FMT_MXFP4 else (codes & 0x7F) != 0x7F
    codes, scales = codes[keep], scales[keep]
    got = _probe_cvt(fmt, codes, scales)
    dec = O.decode_e2m1 if fmt == C.FMT_MXFP4 else O.decode_e4m3fn
    ref = np.array([np.float32(dec(int(c)) * np.float32(O.decode_e8m0(int(s))))
                    for c, s in zip(codes, scales)], np.float32)
    rb = ref.view(np.uint32)
    exact = np.isfinite(ref) & ((rb & 0xFFFF) == 0)
    g32 = (got.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(g32[exact], ref[exact]), np.nonzero(g32[exact] != ref[exact])
    # inexact (BF16-subnormal underflow of E4M3 subnormals at tiny scales): nearest neighbours
    sub = np.isfinite(ref) & ~exact
    if sub.any():
        assert np.all(np.abs(g32[sub] - ref[sub]) <= np.abs(ref[sub]))
    ovf = ~np.isfinite(ref)
    print(f"fmt {fmt}: {exact.sum()} exact, {sub.sum()} below BF16 subnormal range, "
          f"{ovf.sum()} overflow -> {np.unique(got[ovf])[:8]}")


# ------------------------------------------------------------------------------- layers
SMALL = [(name, T) for name in C.WORKLOADS for T in (1, 3, 40)]


def _small_layer(name, hidden=256, n_experts=16, intermediate=128):
    w = C.workload(name)
    spec = C.small_spec(w.spec, hidden=hidden, n_experts=n_experts, intermediate=intermediate)
    bias = C.zipf_bias(spec.n_experts, w.zipf_s, 0.05) if w.zipf_s else None
    return C.make_host_layer(spec, bias=bias)


@pytest.mark.parametrize("name,T", SMALL)
def test_small_layer_matches_oracle(name, T):
    host = _small_layer(name)
    spec = host.spec
    x = synth.activations(f"x.{T}", T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, w = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    layer.close()


# top_k at its extremes (plain, MX-activation and gated-shared-expert compositions): one
# expert; 16, the most the fused one-token down + combine takes (one wave per slot); 32, the
# header's limit (per-slot down projections, then the combine kernel).  At T = 1 (the one-token
# launches) and T = 40 (the grouped GEMMs).
TOPK = [(name, k, T) for name in ("c1_bf16_decode", "c3_mxfp4_decode", "c4_mxfp8",
                                  "c4_mxfp8_mx_activation", "c5_mxfp4_dsv41", "qwen36_release")
        for k in (1, 16, 32) for T in (1, 40)]


@pytest.mark.parametrize("name,k,T", TOPK)
def test_top_k_extremes_match_oracle(name, k, T):
    w = C.workload(name)
    spec = C.small_spec(w.spec, hidden=256, n_experts=64, intermediate=128, top_k=k)
    bias = C.zipf_bias(spec.n_experts, w.zipf_s, 0.05) if w.zipf_s else None
    host = C.make_host_layer(spec, bias=bias)
    x = synth.activations(f"x.topk.{k}.{T}", T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, wts = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    assert np.allclose(wts.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    layer.close()


# The header's largest geometry, one dimension at a time: 512 experts (the routing's lane
# slots, group-limited for c3), hidden 12288 (the one-token kernels stage 48 KiB of input
# pieces per workgroup), intermediate 12288 (past the fused down + combine's 96 KiB of SwiGLU
# rows: per-slot down projections, then the combine kernel).
LARGEST = [(name, dims, T) for name in ("c1_bf16_decode", "c3_mxfp4_decode", "c4_mxfp8")
           for dims in ((512, 256, 128), (16, 12288, 128), (16, 256, 12288)) for T in (1, 3)]


@pytest.mark.parametrize("name,dims,T", LARGEST,
                         ids=[f"{n}-E{d[0]}-H{d[1]}-I{d[2]}-T{t}" for n, d, t in LARGEST])
def test_largest_geometry_matches_oracle(name, dims, T):
    E, H, I = dims
    w = C.workload(name)
    spec = C.small_spec(w.spec, hidden=H, n_experts=E, intermediate=I)
    bias = C.zipf_bias(spec.n_experts, w.zipf_s, 0.05) if w.zipf_s else None
    host = C.make_host_layer(spec, bias=bias)
    x = synth.activations(f"x.largest.{E}.{H}.{I}.{T}", T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, wts = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    assert np.allclose(wts.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    layer.close()


@pytest.mark.parametrize("name", list(C.WORKLOADS))
def test_router_logits_match_oracle(name):
    host = _small_layer(name, hidden=512, n_experts=64)
    spec = host.spec
    x = synth.activations("x.router", 17, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=17)
    logits, ids, w = layer.route(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    logits = logits.cpu().numpy()
    if spec.composition == C.COMPOSE_QWEN36:
        # the 8-lane FP32 tree is reproduced exactly, BF16 logits are bit-identical
        assert np.array_equal(logits.view(np.uint32), ref.logits.view(np.uint32))
    else:
        # f64 accumulation in another order (GEMV, < 16 tokens) or f32 MFMA partials of 32
        # products folded into f64 (GEMM): the error stays far inside the 1e-6 near-tie gap
        # that top-k parity allows.
        err = np.abs(logits.astype(np.float64) - ref.logits.astype(np.float64))
        assert err.max() <= 2e-7 + 2 * np.spacing(np.abs(ref.logits)).max()
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    layer.close()


@pytest.mark.parametrize("E,groups,topk_group", [(64, 32, 5), (64, 16, 3), (64, 8, 4),
                                                 (128, 8, 3), (256, 8, 4), (256, 4, 2),
                                                 (160, 8, 4), (384, 4, 2)])
def test_group_limited_routing_matches_oracle(E, groups, topk_group):
    # groups of 2 .. 64 experts are scored by a lane butterfly, groups of 20 and 96 by a scan
    # over the scores in LDS; one token and a batch of nine take the same per-token routine
    spec = replace(C.small_spec(C.workload("c3_mxfp4_decode").spec, hidden=256, n_experts=E,
                                intermediate=128), n_group=groups, topk_group=topk_group)
    host = C.make_host_layer(spec, bias=C.zipf_bias(E, 1.1, 0.05))
    for T in (1, 9):
        x = synth.activations(f"x.groups.{E}.{groups}.{T}", T, spec.hidden)
        layer = moe_mod().MoeLayer(host, max_tokens=T)
        _, ids, w = layer.route(torch.from_numpy(x).cuda())
        ref = _oracle(host, x)
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
        assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
        layer.close()


@pytest.mark.parametrize("name,T", [(n, T) for n in ("c3_mxfp4_decode", "c4_mxfp8")
                                     for T in (1, 5, 40)])
def test_sqrt_softplus_router_layer_matches_oracle(name, T):
    w = C.WORKLOADS[name]
    spec = replace(C.small_spec(w.spec, hidden=256, n_experts=64, intermediate=128, top_k=6),
                   router=C.ROUTER_SQRT_SOFTPLUS, routed_scaling_factor=1.5, n_group=1,
                   topk_group=1)
    host = C.make_host_layer(spec, bias=C.zipf_bias(64, 1.1, 0.05))
    x = synth.activations(f"x.ssp.{T}", T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, wt = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    assert rel_l2(y.cpu().numpy(), ref.output) < REL_L2_BAR
    assert np.allclose(wt.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    layer.close()


# ------------------------------------------------------------------------------- MX activations
def _quantizer_cases():
    rng = np.random.default_rng(12)
    rows = [rng.standard_normal(256) * s for s in (1e-6, 1e-3, 0.3, 1.0, 7.0, 300.0, 1e5, 1e30)]
    # block maxima just above / below powers of two times 448 (the power_of_two_ceiling band
    # near exact powers, where the reference keeps its log2/ceil/powf formula)
    edge = []
    for e in range(-20, 20):
        for m in (0, 1, 2, 3, 4096, 4097, 0x7FFFFF - 4097, 0x7FFFFF - 4096, 0x7FFFFF - 1, 5000):
            v = np.float32(np.uint32(((127 + e) << 23) | m).view(np.float32)) * np.float32(448.0)
            edge.append(v)
    edge = np.array(edge, np.float32)
    blocks = []
    for v in edge:
        b = rng.standard_normal(32).astype(np.float32) * v / 4
        b[rng.integers(32)] = v * (1 if rng.integers(2) else -1)
        blocks.append(b)
    rows.append(np.concatenate(blocks)[: (len(blocks) * 32 // 256) * 256])
    # zeros, values below the 1e-4 floor, E4M3 subnormals and ties
    rows.append(np.concatenate([np.zeros(32), np.full(32, 3e-5), rng.standard_normal(32) * 1e-4,
                                np.arange(-16, 16) * 2.0 ** -9 * 7, np.arange(-16, 16) * 0.5625,
                                np.full(32, 448.0), np.full(32, -1e38), np.arange(32) - 15.5]))
    return [np.asarray(r, np.float32) for r in rows]


def test_quantize_e4m3_matches_simulate_e4m3_activation_bit_exact():
    dec8 = np.array([O.decode_e4m3fn(c) for c in range(256)], np.float32)
    for r in _quantizer_cases():
        x = r.reshape(1, -1)
        codes, scales = moe_mod().quantize_e4m3(torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        c = codes.cpu().numpy().ravel()
        s = scales.cpu().numpy().ravel().astype(np.int64)
        got = dec8[c] * np.exp2(np.repeat(s - 127, 32)).astype(np.float32)
        ref = O.simulate_e4m3_activation(x.ravel(), 32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            np.nonzero(got.view(np.uint32) != ref.view(np.uint32))[0][:8]
        assert not np.any((c & 0x7F) == 0x7F)  # never a NaN code


def test_quantize_e4m3_128_value_blocks_bit_exact():
    # DeepSeek V4's prepare_mx_activation: simulate_e4m3_activation(x, 128)
    dec8 = np.array([O.decode_e4m3fn(c) for c in range(256)], np.float32)
    for r in _quantizer_cases():
        x = np.ascontiguousarray(r[: r.size // 128 * 128].reshape(1, -1))
        if x.size == 0:
            continue
        codes, scales = moe_mod().quantize_e4m3(torch.from_numpy(x).cuda(), block=128)
        torch.cuda.synchronize()
        c = codes.cpu().numpy().ravel()
        s = scales.cpu().numpy().ravel().astype(np.int64)
        got = dec8[c] * np.exp2(np.repeat(s - 127, 128)).astype(np.float32)
        ref = O.simulate_e4m3_activation(x.ravel(), 128)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # blocks of 32 whose magnitudes alternate by 2^16: the 128-value scale differs from the
    # 32-value one and puts the small blocks on E4M3's subnormal grid
    x = synth.activations("x.q128", 2, 512)
    x = np.ascontiguousarray(x * np.repeat(np.exp2(16.0 * (np.arange(16) % 2)), 32),
                             dtype=np.float32)
    c128, s128 = moe_mod().quantize_e4m3(torch.from_numpy(x).cuda(), block=128)
    torch.cuda.synchronize()
    got = dec8[c128.cpu().numpy()] * np.exp2(
        np.repeat(s128.cpu().numpy().astype(np.int64) - 127, 128, axis=1)).astype(np.float32)
    ref = np.stack([O.simulate_e4m3_activation(row, 128) for row in x])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert not np.array_equal(ref, np.stack([O.simulate_e4m3_activation(row, 32) for row in x]))


MX_LAYERS = [(comp, fmt, T) for comp in (C.COMPOSE_HY4, C.COMPOSE_DSV41, C.COMPOSE_DSV4)
             for fmt in (C.FMT_MXFP4, C.FMT_MXFP8) for T in (1, 5, 40)]


def _hy4_layer(fmt, hidden=256, n_experts=32, intermediate=128, top_k=6,
               composition=C.COMPOSE_HY4):
    # Hy4: grouped sigmoid router; DeepSeek V4.1: its sqrt-softplus router
    router = C.ROUTER_SIGMOID_NOAUX_TC if composition == C.COMPOSE_HY4 else C.ROUTER_SQRT_SOFTPLUS
    spec = C.LayerSpec(hidden=hidden, n_experts=n_experts, top_k=top_k, intermediate=intermediate,
                       shared_intermediate=intermediate, expert_format=fmt, shared_format=fmt,
                       router=router, composition=composition, n_group=4,
                       topk_group=2, normalize=True, routed_scaling_factor=2.5, swiglu_limit=7.0)
    return C.make_host_layer(spec, bias=C.zipf_bias(n_experts, 1.1, 0.05))


@pytest.mark.parametrize("comp,fmt,T", MX_LAYERS)
def test_mx_activation_layer_matches_oracle(comp, fmt, T):
    host = _hy4_layer(fmt, composition=comp)
    spec = host.spec
    x = synth.activations(f"x.hy4.{T}", T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, w = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    # BF16 outputs: every element is a BF16 value
    assert np.all((y.cpu().numpy().view(np.uint32) & 0xFFFF) == 0)
    layer.close()


def test_dsv41_router_logits_are_the_fp32_tree_bit_for_bit():
    # DeepSeek V4.1's router.matvec_fp32_accum is the 8-lane FP32 tree without a BF16 step
    host = _hy4_layer(C.FMT_MXFP4, hidden=512, n_experts=64, composition=C.COMPOSE_DSV41)
    x = synth.activations("x.dsv.router", 9, 512)
    layer = moe_mod().MoeLayer(host, max_tokens=9)
    logits, ids, w = layer.route(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    logits = logits.cpu().numpy()
    assert np.array_equal(logits.view(np.uint32), ref.logits.view(np.uint32))
    assert np.any((logits.view(np.uint32) & 0xFFFF) != 0)  # not BF16-rounded
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(host.spec, ref, host.correction_bias))
    layer.close()


def _dsv4_hash_layer(fmt=C.FMT_MXFP4, vocab=50, n_experts=32, top_k=6):
    spec = C.LayerSpec(hidden=256, n_experts=n_experts, top_k=top_k, intermediate=128,
                       shared_intermediate=128, expert_format=fmt, shared_format=fmt,
                       router=C.ROUTER_SQRT_SOFTPLUS, composition=C.COMPOSE_DSV4,
                       routed_scaling_factor=1.5, swiglu_limit=10.0)
    return C.make_host_layer(spec, hash_vocab=vocab)


@pytest.mark.parametrize("fmt,T", [(C.FMT_MXFP4, 1), (C.FMT_MXFP4, 7), (C.FMT_MXFP8, 40),
                                   (C.FMT_MXFP4, 300)])
def test_dsv4_hash_layer_matches_oracle(fmt, T):
    # DeepSeek V4's hash layers: the token's tid2eid row gives the experts in table order, the
    # weights s / sum(s) * 1.5 over that row (deepseek_v4/math.rs:451-516, runtime.rs:2664-2681)
    host = _dsv4_hash_layer(fmt)
    x = synth.activations(f"x.dsv4.hash.{T}", T, host.spec.hidden)
    tokens = (synth.splitmix64(synth.stream_seed(f"tok.{T}"), 0, T) % 50).astype(np.uint32)
    tokens[T // 2:] = tokens[: T - T // 2]  # repeated tokens
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    tok = torch.from_numpy(tokens.view(np.int32)).cuda()
    y, ids, w = layer.forward(torch.from_numpy(x).cuda(), token_ids=tok)
    ref = _oracle(host, x, token_ids=tokens)
    ids = ids.cpu().numpy()
    assert np.array_equal(ids, ref.ids)
    assert np.array_equal(ids, host.hash_experts[tokens].astype(np.int32))
    assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    logits, rids, rw = layer.route(torch.from_numpy(x).cuda(), token_ids=tok)
    assert np.array_equal(rids.cpu().numpy(), ref.ids)
    assert np.allclose(logits.cpu().numpy(), ref.logits, rtol=2e-6, atol=1e-7)
    layer.close()


def test_dsv4_hash_errors():
    host = _dsv4_hash_layer()
    x = torch.from_numpy(synth.activations("x.dsv4.err", 3, host.spec.hidden)).cuda()
    layer = moe_mod().MoeLayer(host, max_tokens=3)
    with pytest.raises(N.UrbError) as e:  # hash routing needs the token ids
        layer.forward(x)
    assert e.value.status == N.ERR_ARGUMENT
    with pytest.raises(N.UrbError) as e:  # token id outside the table (load_i64_matrix_row)
        layer.forward(x, token_ids=torch.tensor([3, 50, 1], dtype=torch.int32, device="cuda"))
    assert e.value.status == N.ERR_SHAPE
    y, ids, _ = layer.forward(x, token_ids=torch.tensor([3, 49, 1], dtype=torch.int32,
                                                        device="cuda"))
    assert np.array_equal(ids.cpu().numpy(), host.hash_experts[[3, 49, 1]])
    layer.close()
    bad = host.hash_experts.copy()
    bad[7, 2] = host.spec.n_experts  # "hash expert IDs must be in range"
    dup = host.hash_experts.copy()
    dup[9, 1] = dup[9, 0]
    for table, spec, status in ((bad, host.spec, N.ERR_INVALID_GEOMETRY),
                                (dup, host.spec, N.ERR_ARGUMENT),
                                (host.hash_experts,
                                 replace(host.spec, router=C.ROUTER_SIGMOID_NOAUX_TC),
                                 N.ERR_ARGUMENT)):
        h = replace(host, spec=spec, hash_experts=table)
        with pytest.raises(N.UrbError) as e:
            moe_mod().MoeLayer(h, max_tokens=1)
        assert e.value.status == status


def test_hy4_errors():
    host = _hy4_layer(C.FMT_MXFP8)
    for bad, status in ((dict(swiglu_limit=0.0), N.ERR_INVALID_GEOMETRY),
                        (dict(swiglu_limit=float("inf")), N.ERR_NONFINITE),
                        (dict(expert_format=C.FMT_BF16), N.ERR_ARGUMENT),
                        (dict(shared_format=C.FMT_BF16), N.ERR_ARGUMENT)):
        h = C.HostLayer(replace(host.spec, **bad), host.router_weight, host.experts, host.shared,
                        host.correction_bias)
        with pytest.raises(N.UrbError) as e:
            moe_mod().MoeLayer(h, max_tokens=1)
        assert e.value.status == status
    layer = moe_mod().MoeLayer(host, max_tokens=2)
    x = torch.from_numpy(synth.activations("x.hy4.nan", 2, host.spec.hidden)).cuda()
    x[1, 5] = float("nan")
    with pytest.raises(N.UrbError) as e:
        layer.forward(x)
    assert e.value.status == N.ERR_NONFINITE
    layer.close()


@pytest.mark.parametrize("comp,T,E", [(C.COMPOSE_QWEN36, 40, 40), (C.COMPOSE_QWEN36, 600, 40),
                                      (C.COMPOSE_QWEN36, 600, 248), (C.COMPOSE_DSV41, 777, 40),
                                      (C.COMPOSE_QWEN36, 64, 40), (C.COMPOSE_QWEN36, 300, 248),
                                      (C.COMPOSE_DSV41, 512, 72)])
def test_batched_lane8_router_is_bit_identical(comp, T, E):
    # From 64 tokens the tiled 8-lane router runs (one token per workgroup up to 512 tokens,
    # then 16 or 8 tokens per workgroup); its logits must equal the reference tree bit for bit,
    # for partial token tiles and expert counts that are not multiples of 32 as well.
    if comp == C.COMPOSE_QWEN36:
        spec = C.small_spec(C.WORKLOADS["c1_bf16_decode"].spec, hidden=640, n_experts=E,
                            intermediate=128)
        host = C.make_host_layer(spec)
    else:
        host = _hy4_layer(C.FMT_MXFP4, hidden=640, n_experts=E, composition=C.COMPOSE_DSV41)
    x = synth.activations(f"x.tiled.{T}", T, host.spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    logits, ids, w = layer.route(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), ref.logits.view(np.uint32))
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(host.spec, ref, host.correction_bias))
    layer.close()


def test_forward_is_deterministic_and_chunked_calls_equal_tokenwise():
    host = _small_layer("c5_mxfp4_zipf_prefill", hidden=128, n_experts=16, intermediate=128)
    T = 1100  # > one 1024-token internal chunk
    x = torch.from_numpy(synth.activations("x.chunk", T, 128)).cuda()
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y1, i1, _ = layer.forward(x)
    y2, i2, _ = layer.forward(x)
    assert torch.equal(y1, y2) and torch.equal(i1, i2)
    single = moe_mod().MoeLayer(host, max_tokens=1)
    for t in (0, 1023, 1024, 1099):
        ys, _, _ = single.forward(x[t:t + 1].contiguous())
        # the single token takes the GEMV path (f32 products of BF16 pieces, ~1e-6 of the
        # oracle); the batch the MFMA GEMMs, whose MX down projection multiplies the SwiGLU rows
        # rounded to f16 after a per-row power-of-two scale (2^-11 relative per element): the
        # two agree within the layer's 1e-3 bar, not to f32 rounding
        assert rel_l2(ys.cpu().numpy(), y1[t:t + 1].cpu().numpy()) < 1e-3
    layer.close()
    single.close()


# ------------------------------------------------------------------------------- panel layout
def _panel_pack_np(fmt, data, scales):
    """Restates the panel layout on the host: slab t of a 16-row panel, 16-byte unit
    l = ln + 16 lq <- row ln's bytes at 64 t + 16 lq (BF16, MXFP4) or
    128 (t // 2) + 32 lq + 16 (t % 2) (MXFP8); scale slab s, byte l <- row ln, block 4 s + lq."""
    raw = np.ascontiguousarray(data).view(np.uint8)
    rows = raw.shape[0]
    rb = raw.size // rows
    units = raw.reshape(rows // 16, 16, rb // 16, 16)          # [panel, row, unit, byte]
    out = np.empty((rows // 16, rb // 64, 64, 16), np.uint8)  # [panel, slab, lane, byte]
    for t in range(rb // 64):
        for lq in range(4):
            off = (t // 2) * 128 + 32 * lq + 16 * (t % 2) if fmt == C.FMT_MXFP8 else 64 * t + 16 * lq
            out[:, t, 16 * lq:16 * lq + 16, :] = units[:, :, off // 16, :]
    packed_scales = None
    if scales is not None:
        sc = np.ascontiguousarray(scales).reshape(rows // 16, 16, -1)  # [panel, row, block]
        nb = sc.shape[2]
        ps = np.empty((rows // 16, nb // 4, 64), np.uint8)
        for lq in range(4):
            ps[:, :, 16 * lq:16 * lq + 16] = sc[:, :, lq::4].transpose(0, 2, 1)
        packed_scales = ps.ravel()
    return out.ravel(), packed_scales


@pytest.mark.parametrize("fmt", [C.FMT_BF16, C.FMT_MXFP4, C.FMT_MXFP8])
def test_pack_matrix_matches_host_restatement(fmt):
    spec = C.small_spec(C.WORKLOADS["c4_mxfp8"].spec, hidden=256, n_experts=2, intermediate=384)
    from dataclasses import replace
    spec = replace(spec, expert_format=fmt)
    host = C.make_host_layer(spec)
    for m, (rows, cols) in enumerate(((384, 256), (384, 256), (256, 384))):
        d, s = host.experts[1][m]
        dd = torch.from_numpy(np.ascontiguousarray(d).view(np.uint8).copy()).cuda()
        ss = None if s is None else torch.from_numpy(np.ascontiguousarray(s).copy()).cuda()
        pd, ps = moe_mod().pack_matrix(fmt, dd, ss, rows, cols)
        torch.cuda.synchronize()
        want_d, want_s = _panel_pack_np(fmt, d, s)
        assert np.array_equal(pd.cpu().numpy().view(np.uint8).ravel(), want_d)
        if s is not None:
            assert np.array_equal(ps.cpu().numpy().ravel(), want_s)


def test_borrowed_panel_layer_equals_copied_layer():
    for name in ("c2_bf16_prefill", "c3_mxfp4_decode", "c4_mxfp8"):
        host = _small_layer(name)
        dev = moe_mod().DeviceLayer.from_host(host)
        x = torch.from_numpy(synth.activations("x.borrow", 5, host.spec.hidden)).cuda()
        copied = moe_mod().MoeLayer(dev, max_tokens=5)
        borrowed = moe_mod().MoeLayer(moe_mod().packed_layer(dev), max_tokens=5,
                                      source=N.SOURCE_DEVICE_BORROW)
        for T in (1, 5):
            y1, i1, w1 = copied.forward(x[:T].contiguous())
            y2, i2, w2 = borrowed.forward(x[:T].contiguous())
            assert torch.equal(y1, y2) and torch.equal(i1, i2) and torch.equal(w1, w2)
        assert borrowed.memory()[0] == 0
        copied.close()
        borrowed.close()


def _consolidate(dev):
    """Stacks a layer's per-expert matrices into the consolidated checkpoint tensors:
    gate_up [E, 2I, ...] (gate rows, then up rows), down [E, H, ...], scale sidecars alike."""
    spec = dev.spec
    E, H, I = spec.n_experts, spec.hidden, spec.intermediate
    rows = lambda t, r: t.contiguous().view(torch.uint8).reshape(r, -1)
    gu = torch.stack([torch.cat([rows(dev.experts[e][0][0], I), rows(dev.experts[e][1][0], I)])
                      for e in range(E)]).contiguous()
    dn = torch.stack([rows(dev.experts[e][2][0], H) for e in range(E)]).contiguous()
    gus = dns = None
    if dev.experts[0][0][1] is not None:
        gus = torch.stack([torch.cat([rows(dev.experts[e][0][1], I), rows(dev.experts[e][1][1], I)])
                           for e in range(E)]).contiguous()
        dns = torch.stack([rows(dev.experts[e][2][1], H) for e in range(E)]).contiguous()
    return gu, gus, dn, dns


def test_consolidated_checkpoint_layer_equals_per_expert_layer():
    # Qwen3.6 packed BF16 gate_up_proj / down_proj and Hy4 consolidated E4M3 + U8 scales,
    # used through per-expert views, give the per-expert layer's results bit for bit.
    for name in ("c2_bf16_prefill", "c3_mxfp4_decode", "c4_mxfp8_mx_activation"):
        host = _small_layer(name)
        dev = moe_mod().DeviceLayer.from_host(host)
        gu, gus, dn, dns = _consolidate(dev)
        cons = moe_mod().DeviceLayer.from_consolidated(dev.spec, dev.router_weight, gu, gus, dn,
                                                       dns, dev.shared, dev.correction_bias)
        x = torch.from_numpy(synth.activations("x.consolidated", 5, host.spec.hidden)).cuda()
        a = moe_mod().MoeLayer(dev, max_tokens=5)
        b = moe_mod().MoeLayer(cons, max_tokens=5)
        for T in (1, 5):
            y1, i1, w1 = a.forward(x[:T].contiguous())
            y2, i2, w2 = b.forward(x[:T].contiguous())
            assert torch.equal(y1, y2) and torch.equal(i1, i2) and torch.equal(w1, w2)
            # and the consolidated layer against the oracle on the same host weights
            ref = _oracle(host, x[:T].cpu().numpy())
            assert ids_match(i2.cpu().numpy(), ref.ids,
                             _scores(host.spec, ref, host.correction_bias))
            assert rel_l2(y2.cpu().numpy(), ref.output) < REL_L2_BAR
        a.close()
        b.close()


# ------------------------------------------------ Qwen3.6 with its sigmoid-gated shared expert
def _qwen_shared_layer(hidden=256, n_experts=16, intermediate=128):
    spec = replace(C.small_spec(C.WORKLOADS["c2_bf16_prefill"].spec, hidden=hidden,
                                n_experts=n_experts, intermediate=intermediate),
                   shared_intermediate=intermediate, shared_format=C.FMT_BF16)
    return C.make_host_layer(spec)


@pytest.mark.parametrize("comp,T,bf16_x", [(C.COMPOSE_GLM, 256, True), (C.COMPOSE_GLM, 300, True),
                                           (C.COMPOSE_GLM, 520, True), (C.COMPOSE_GLM, 520, False),
                                           (C.COMPOSE_QWEN36, 300, True)])
def test_dense_shared_batch_matches_oracle(comp, T, bf16_x):
    # f32-activation batches of 256+ tokens run the BF16 shared expert in line: the gate/up on
    # the split-K dense kernel (256-token tiles; 300 and 520 end in a partial tile; f32 token
    # rows take the lo-half MFMAs, BF16-valued ones skip them); GLM's down on the dense f16
    # kernel (128-token tiles, 300 and 520 again partial), Qwen3.6's on dense 32-token tiles of
    # four panels per wave
    if comp == C.COMPOSE_GLM:
        spec = C.LayerSpec(hidden=512, n_experts=16, top_k=4, intermediate=256,
                           shared_intermediate=256, expert_format=C.FMT_MXFP4,
                           shared_format=C.FMT_BF16, router=C.ROUTER_SIGMOID_NOAUX_TC,
                           composition=C.COMPOSE_GLM, n_group=4, topk_group=2, normalize=True,
                           routed_scaling_factor=2.5)
        host = C.make_host_layer(spec, bias=C.zipf_bias(16, 1.1, 0.05))
    else:
        host = _qwen_shared_layer()
        spec = host.spec
    x = synth.activations(f"x.dense.{comp}.{T}", T, spec.hidden)
    if not bf16_x:
        x = synth.normals(synth.stream_seed(f"x.dense.f32.{T}"), T * spec.hidden).reshape(
            T, spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, w = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    layer.close()


def test_dense_shared_down_f16_range_matches_oracle():
    # GLM batches of 256+ tokens with a BF16 shared expert run its down projection on f16 MFMAs
    # over an f16 copy of the matrix when every non-zero value is exactly an f16 after one power
    # of two (exponents within 32 binades); one weight 2^-67 among values near 2^-4 leaves that
    # range, so the context keeps no copy (its weight bytes show it) and the BF16 hi/lo path runs
    spec = C.LayerSpec(hidden=512, n_experts=16, top_k=4, intermediate=256,
                       shared_intermediate=256, expert_format=C.FMT_MXFP4,
                       shared_format=C.FMT_BF16, router=C.ROUTER_SIGMOID_NOAUX_TC,
                       composition=C.COMPOSE_GLM, n_group=4, topk_group=2, normalize=True,
                       routed_scaling_factor=2.5)
    host = C.make_host_layer(spec, bias=C.zipf_bias(16, 1.1, 0.05))
    down, scales = host.shared[2]
    wide = down.copy()
    wide.reshape(-1)[7] = (60 << 7) | 0x25  # BF16 exponent field 60: ~2^-67
    wide_host = replace(host, shared=[host.shared[0], host.shared[1], (wide, scales)])
    x = synth.activations("x.dense.f16range", 300, spec.hidden)
    sizes = []
    for h in (host, wide_host):
        layer = moe_mod().MoeLayer(h, max_tokens=300)
        y, ids, w = layer.forward(torch.from_numpy(x).cuda())
        ref = _oracle(h, x)
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, h.correction_bias))
        err = rel_l2(y.cpu().numpy(), ref.output)
        assert err < REL_L2_BAR, err
        sizes.append(layer.memory()[0])
        layer.close()
    # the f16 copy: the down matrix's 512 x 256 values at 2 bytes
    assert sizes[0] - sizes[1] == 512 * 256 * 2


def _lo_layer(comp):
    if comp == "glm":
        spec = C.LayerSpec(hidden=512, n_experts=16, top_k=4, intermediate=256,
                           expert_format=C.FMT_BF16, router=C.ROUTER_SIGMOID_NOAUX_TC,
                           composition=C.COMPOSE_GLM, n_group=4, topk_group=2, normalize=True,
                           routed_scaling_factor=2.5)
        return C.make_host_layer(spec, bias=C.zipf_bias(16, 1.1, 0.05))
    return _small_layer("c2_bf16_prefill", hidden=512, n_experts=16, intermediate=256)


@pytest.mark.parametrize("comp,T", [("glm", 40), ("qwen", 40), ("qwen", 100), ("qwen", 600)])
def test_token_inputs_keep_their_lo_halves_when_the_router_sees_them(comp, T):
    # The grouped GEMMs drop the lo halves of BF16-valued token rows; the router (the batched
    # MFMA router for GLM, the 8-lane routers for Qwen at each batch-size path) reports a value
    # off the BF16 grid in the call's input -- one token suffices -- and the GEMMs then keep
    # them.  Dropping them moves the output by ~2e-3: the GPU output must sit nearer the oracle
    # on the input than on its BF16 rounding.
    host = _lo_layer(comp)
    spec = host.spec
    x_bf = synth.activations(f"x.lo.bf16.{T}", T, spec.hidden)
    x_f32 = synth.normals(synth.stream_seed(f"x.lo.f32.{T}"), T * spec.hidden).reshape(
        T, spec.hidden).astype(np.float32)
    x_mix = x_bf.copy()
    x_mix[T - 3] = x_f32[T - 3]
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    for x in (x_f32, x_bf, x_mix, x_bf):
        y, ids, _ = layer.forward(torch.from_numpy(x).cuda())
        y = y.cpu().numpy()
        ref = _oracle(host, x)
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
        assert rel_l2(y, ref.output) < REL_L2_BAR
        if x is not x_bf:
            rounded = _oracle(host, torch.from_numpy(x).bfloat16().float().numpy())
            t = T - 3
            assert rel_l2(y[t], ref.output[t]) < 0.5 * rel_l2(y[t], rounded.output[t])
    layer.close()


@pytest.mark.parametrize("fmt,shared_fmt,hidden,inter",
                         [(f, g, 256, 128) for f in (C.FMT_BF16, C.FMT_MXFP4, C.FMT_MXFP8)
                          for g in (C.FMT_BF16, C.FMT_MXFP4, C.FMT_MXFP8)]
                         + [(C.FMT_MXFP4, C.FMT_BF16, 2048, 1024),
                            (C.FMT_MXFP8, C.FMT_MXFP4, 2048, 1024)])
def test_one_token_shared_expert_launches_match_oracle(fmt, shared_fmt, hidden, inter):
    # One token with a shared expert: the routing runs beside the shared gate+up and the shared
    # down beside the routed gate+up, for every pair of weight formats; H 2048 splits K in both
    spec = C.LayerSpec(hidden=hidden, n_experts=64, top_k=8, intermediate=inter,
                       shared_intermediate=inter, expert_format=fmt, shared_format=shared_fmt,
                       router=C.ROUTER_SIGMOID_NOAUX_TC, composition=C.COMPOSE_GLM, n_group=8,
                       topk_group=4, normalize=True, routed_scaling_factor=2.5)
    host = C.make_host_layer(spec, bias=C.zipf_bias(64, 1.1, 0.05))
    x = synth.activations(f"x.one.{fmt}.{shared_fmt}.{hidden}", 1, hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=1)
    for _ in range(2):  # a second call reuses the workspace
        y, ids, w = layer.forward(torch.from_numpy(x).cuda())
        ref = _oracle(host, x)
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
        assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
        err = rel_l2(y.cpu().numpy(), ref.output)
        assert err < REL_L2_BAR, err
    layer.close()


@pytest.mark.parametrize("T", [1, 5, 40])
def test_qwen_gated_shared_expert_matches_oracle(T):
    # T = 1 takes the fused down+combine kernel, T > 1 the grouped GEMMs and combine kernel;
    # the gate logit is the router's 8-lane tree, so routes and gates agree exactly
    host = _qwen_shared_layer()
    x = synth.activations(f"x.qsh.{T}", T, host.spec.hidden)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    y, ids, w = layer.forward(torch.from_numpy(x).cuda())
    ref = _oracle(host, x)
    assert np.array_equal(ids.cpu().numpy(), ref.ids)
    assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    err = rel_l2(y.cpu().numpy(), ref.output)
    assert err < REL_L2_BAR, err
    # the FFN block over the same layer
    h, nw = _block_inputs(T, host.spec.hidden, 21 + T)
    out, bids, _ = layer.forward_block(torch.from_numpy(h).cuda(), torch.from_numpy(nw).cuda(),
                                       1e-6)
    bref = _oracle(host, O.zc_rms_norm(h, nw, 1e-6))
    assert np.array_equal(bids.cpu().numpy(), bref.ids)
    want = O.add_residual_bf16(h, bref.output)
    assert rel_l2(out.cpu().numpy() - h, want - h) < REL_L2_BAR
    layer.close()


def test_qwen_shared_expert_needs_its_gate_and_bf16():
    host = _qwen_shared_layer()
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(replace(host, shared_expert_gate=None), max_tokens=2)
    assert e.value.status == N.ERR_ARGUMENT
    spec = replace(host.spec, shared_format=C.FMT_MXFP4)
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(C.make_host_layer(spec), max_tokens=2)
    assert e.value.status == N.ERR_ARGUMENT
    bad = host.shared_expert_gate.copy()
    bad[3] = 0x7F80  # +inf
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(replace(host, shared_expert_gate=bad), max_tokens=2)
    assert e.value.status == N.ERR_NONFINITE


# ------------------------------------------------------ experts streamed through HBM slots
@pytest.mark.parametrize("name", ["c2_bf16_prefill", "c3_mxfp4_decode", "c4_mxfp8"])
def test_streamed_residency_layer_equals_resident_layer(name):
    # 16 experts in host memory, 10 HBM slots placed by the residency policy: every call gives
    # the fully resident layer's results on the same token runs, bit for bit, and the policy's
    # telemetry is the serial LRU replay of the calls' access sequences
    from urbilateria_amd import residency as R
    host = _small_layer(name)
    spec = host.spec
    streamed = R.StreamedMoeLayer(host, slots=10, max_tokens=6)
    resident = moe_mod().MoeLayer(host, max_tokens=6)
    replay, rt = R.LayerLruCache(1, 10), R.Telemetry()
    for call, T in enumerate((1, 3, 6, 2, 6)):
        x = torch.from_numpy(synth.activations(f"x.stream.{call}", T, spec.hidden)).cuda()
        y, ids, w = streamed.forward(x)
        parts = [resident.forward(x[a:b].contiguous()) for a, b in streamed.last_runs]
        assert torch.equal(y, torch.cat([p[0] for p in parts]))
        assert torch.equal(ids, torch.cat([p[1] for p in parts]))
        assert torch.equal(w, torch.cat([p[2] for p in parts]))
        # the streamed layer against the oracle on the host weights it streams from
        ref = _oracle(host, x.cpu().numpy())
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
        assert rel_l2(y.cpu().numpy(), ref.output) < REL_L2_BAR
        assert np.allclose(w.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
        for t in range(T):
            for key in sorted(ids[t].tolist()):
                replay.access(rt, 0, key, lambda key=key: (key, 1, 1))
    got, want = streamed.telemetry, rt
    assert (got.hits, got.misses, got.evictions) == (want.hits, want.misses, want.evictions)
    assert got.misses > 10 and got.evictions > 0  # the slots did turn over
    streamed.close()
    resident.close()


def test_streamed_layer_survives_a_failed_load():
    # A host expert with an E8M0 NaN scale fails its load after the LRU evicted a victim and
    # after its bytes were packed into a slot.  The call raises; once the expert is repaired,
    # every later call equals the resident layer bit for bit -- no resident expert's slot was
    # reused by the failed load or handed out twice afterwards.
    from urbilateria_amd import residency as R
    host = _small_layer("c3_mxfp4_decode")
    spec = host.spec
    resident = moe_mod().MoeLayer(host, max_tokens=6)
    xs = [torch.from_numpy(synth.activations(f"x.stream.fail.{c}", 6, spec.hidden)).cuda()
          for c in range(6)]
    warm = xs[0][:1].contiguous()  # one token: 8 of the 10 slots
    _, ids0, _ = resident.forward(warm)
    _, ids1, _ = resident.forward(xs[1])
    warm_set = set(ids0.ravel().tolist())
    cands = [e for e in ids1.ravel().tolist() if e not in warm_set]
    if not cands:
        pytest.skip("every expert of the second call is routed by the warm-up token")
    bad_expert = cands[0]
    good = host.experts[bad_expert][0]
    broken = good[1].copy()
    broken[3] = 0xFF
    experts = [list(e) for e in host.experts]
    experts[bad_expert][0] = (good[0], broken)
    streamed = R.StreamedMoeLayer(replace(host, experts=experts), slots=10, max_tokens=6)
    streamed.forward(warm)
    assert not streamed.cache.contains(0, bad_expert)
    with pytest.raises(R.LoadError):
        streamed.forward(xs[1])
    experts[bad_expert][0] = good  # repaired in the host store the layer streams from
    for x in xs[1:] + xs[:1]:
        y, ids, w = streamed.forward(x)
        parts = [resident.forward(x[a:b].contiguous()) for a, b in streamed.last_runs]
        assert torch.equal(y, torch.cat([p[0] for p in parts]))
        assert torch.equal(ids, torch.cat([p[1] for p in parts]))
        assert torch.equal(w, torch.cat([p[2] for p in parts]))
        slots = [e.value for e in streamed.cache.entries(0)]
        assert len(slots) == len(set(slots)) and all(0 <= s < 10 for s in slots)
    streamed.close()
    resident.close()


def test_streamed_layer_refuses_a_cache_of_another_capacity():
    from urbilateria_amd import residency as R
    host = _small_layer("c3_mxfp4_decode")
    with pytest.raises(ValueError):
        R.StreamedMoeLayer(host, slots=10, max_tokens=2, cache=R.LayerLruCache(1, 12))
    cache = R.LayerLruCache(2, 10)
    streamed = R.StreamedMoeLayer(host, slots=10, max_tokens=2, layer_index=1, cache=cache)
    cache.lend_unused_capacity(1, 16)  # the other layer's 10 unused slots are lent here
    x = torch.from_numpy(synth.activations("x.stream.lend", 2, host.spec.hidden)).cuda()
    with pytest.raises(ValueError):
        streamed.forward(x)
    streamed.close()


def test_streamed_hash_routed_layer_equals_resident_layer():
    # A DeepSeek-V4 hash layer streamed through 10 HBM slots: the token ids reach the routing of
    # every run, and each run equals the resident layer's call bit for bit
    from urbilateria_amd import residency as R
    host = _dsv4_hash_layer(n_experts=16, vocab=30)
    streamed = R.StreamedMoeLayer(host, slots=10, max_tokens=6)
    resident = moe_mod().MoeLayer(host, max_tokens=6)
    for call, T in enumerate((1, 4, 6)):
        x = torch.from_numpy(synth.activations(f"x.stream.hash.{call}", T,
                                               host.spec.hidden)).cuda()
        tok = torch.tensor([(7 * call + 5 * t) % 30 for t in range(T)], dtype=torch.int32,
                           device="cuda")
        y, ids, w = streamed.forward(x, token_ids=tok)
        assert np.array_equal(ids.cpu().numpy(), host.hash_experts[tok.cpu().numpy()])
        parts = [resident.forward(x[a:b].contiguous(), token_ids=tok[a:b])
                 for a, b in streamed.last_runs]
        assert torch.equal(y, torch.cat([p[0] for p in parts]))
        assert torch.equal(w, torch.cat([p[2] for p in parts]))
    streamed.close()
    resident.close()


def test_set_expert_validates_and_needs_a_borrowed_context():
    host = _small_layer("c3_mxfp4_decode")
    dev = moe_mod().DeviceLayer.from_host(host)
    layer = moe_mod().MoeLayer(dev, max_tokens=2)  # a copied context
    lib = N.moe_lib()
    mats = (N.Matrix * 3)(*[N.Matrix(d.data_ptr(), s.data_ptr()) for d, s in dev.experts[0]])
    import ctypes
    assert lib.urb_moe_set_expert(layer._ctx, 0, ctypes.addressof(mats), None) == N.ERR_ARGUMENT
    layer.close()
    packed = moe_mod().packed_layer(dev)
    borrowed = moe_mod().MoeLayer(packed, max_tokens=2, source=N.SOURCE_DEVICE_BORROW)
    bad_scales = packed.experts[1][0][1].clone()
    bad_scales[5] = 0xFF  # an E8M0 NaN scale
    mats = (N.Matrix * 3)(N.Matrix(packed.experts[1][0][0].data_ptr(), bad_scales.data_ptr()),
                          *[N.Matrix(d.data_ptr(), s.data_ptr()) for d, s in packed.experts[1][1:]])
    assert lib.urb_moe_set_expert(borrowed._ctx, 1, ctypes.addressof(mats), None) == \
        N.ERR_INVALID_SCALE
    assert lib.urb_moe_set_expert(borrowed._ctx, 16, ctypes.addressof(mats), None) == \
        N.ERR_ARGUMENT
    borrowed.close()


# ------------------------------------------------- the Qwen3.6 FFN block around the MoE call
def _block_inputs(T, H, seed):
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((T, H)) * np.exp2(rng.integers(-3, 4, (T, 1)))).astype(np.float32)
    h = np.array([O.round_to_bf16(v) for v in h.ravel()], np.float32).reshape(T, H)
    w = (rng.standard_normal(H) * 0.1).astype(np.float32)
    return h, w


@pytest.mark.parametrize("T,H", [(1, 128), (37, 2048), (3, 7168)])
def test_zc_rms_norm_hook_is_bit_exact(T, H):
    # the sequential f32 mean square of the reference, the 1 + weight scale and the BF16 cast
    h, w = _block_inputs(T, H, 11 + H)
    if T > 2:
        h[1] = 1.0
        h[1, 0] = 4096.0  # x0^2 absorbs every later square in a left-to-right f32 sum
    got = moe_mod().zc_rms_norm_bf16(torch.from_numpy(h).cuda(), torch.from_numpy(w).cuda(),
                                     1e-6).cpu().numpy()
    ref = O.zc_rms_norm(h, w, 1e-6)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T", [1, 5, 40])
def test_forward_block_matches_oracle(T):
    # out = bf16(h + moe(bf16(zero_centered_rms_norm(h)))): the normalized input is exact, so
    # the router sees the reference's inputs and the routes agree exactly
    host = _small_layer("c2_bf16_prefill")
    spec = host.spec
    h, w = _block_inputs(T, spec.hidden, 5 + T)
    layer = moe_mod().MoeLayer(host, max_tokens=T)
    hd, wd = torch.from_numpy(h).cuda(), torch.from_numpy(w).cuda()
    out, ids, rw = layer.forward_block(hd, wd, 1e-6)
    n = O.zc_rms_norm(h, w, 1e-6)
    ref = _oracle(host, n)
    want = O.add_residual_bf16(h, ref.output)
    assert np.array_equal(ids.cpu().numpy(), ref.ids)
    assert np.allclose(rw.cpu().numpy(), ref.weights, rtol=1e-5, atol=1e-7)
    err = rel_l2(out.cpu().numpy() - h, want - h)
    assert err < REL_L2_BAR, err
    # the block equals the plain call on the normalized input plus the BF16 residual step
    y, _, _ = layer.forward(torch.from_numpy(n).cuda())
    resid = O.add_residual_bf16(h, y.cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), resid)
    # out may alias h
    lib = N.moe_lib()
    N.check(lib.urb_moe_forward_block(layer._ctx, hd.data_ptr(), wd.data_ptr(), 1e-6, T,
                                      hd.data_ptr(), None, None, None))
    layer.sync()
    assert torch.equal(hd, out)
    layer.close()


def test_forward_block_errors():
    host = _small_layer("c2_bf16_prefill")
    layer = moe_mod().MoeLayer(host, max_tokens=4)
    h, w = _block_inputs(4, host.spec.hidden, 9)
    hd, wd = torch.from_numpy(h).cuda(), torch.from_numpy(w).cuda()
    for eps in (0.0, -1.0, float("nan")):
        with pytest.raises(N.UrbError) as e:
            layer.forward_block(hd, wd, eps)
        assert e.value.status == N.ERR_INVALID_GEOMETRY
    bad = hd.clone()
    bad[2, 3] = float("inf")
    with pytest.raises(N.UrbError) as e:
        layer.forward_block(bad, wd, 1e-6)
    assert e.value.status == N.ERR_NONFINITE
    wbad = wd.clone()
    wbad[0] = float("nan")
    with pytest.raises(N.UrbError) as e:
        layer.forward_block(hd, wbad, 1e-6)
    assert e.value.status == N.ERR_NONFINITE
    out, _, _ = layer.forward_block(hd, wd, 1e-6)  # the latched error was cleared
    assert torch.isfinite(out).all()
    layer.close()
    glm = moe_mod().MoeLayer(_small_layer("c3_mxfp4_decode"), max_tokens=4)
    with pytest.raises(N.UrbError) as e:
        glm.forward_block(hd, wd, 1e-6)
    assert e.value.status == N.ERR_ARGUMENT
    glm.close()


# ------------------------------------------------------------------------------- errors
def test_nonfinite_input_is_reported():
    for name in ("c1_bf16_decode", "c3_mxfp4_decode"):
        host = _small_layer(name)
        layer = moe_mod().MoeLayer(host, max_tokens=2)
        x = torch.from_numpy(synth.activations("x", 2, host.spec.hidden)).cuda()
        x[1, 7] = float("inf")
        with pytest.raises(N.UrbError) as e:
            layer.forward(x)
        assert e.value.status == N.ERR_NONFINITE
        x[1, 7] = 0.5
        layer.forward(x)  # the latched error was cleared; a good call succeeds
        layer.close()


# GLM batches with MX experts run the down projection on f16 MFMAs when every down matrix's
# E8M0 codes keep its weights exact in f16 (MXFP4 104..140, MXFP8 112..134), and on the BF16
# hi + lo pair otherwise.  Both must meet the bar: scales at the edges of the f16 range, and
# scales outside it (one block of one expert) that switch the layer to the BF16 path.
@pytest.mark.parametrize("name,codes", [("c3_mxfp4_decode", (104, 140)),
                                        ("c3_mxfp4_decode", (103, 125)),
                                        ("c3_mxfp4_decode", (119, 160)),
                                        ("c4_mxfp8", (112, 134)),
                                        ("c4_mxfp8", (111, 125))])
def test_down_projection_scale_range_matches_oracle(name, codes):
    host = _small_layer(name)
    spec = host.spec
    rng = np.random.default_rng(codes[0] * 1000 + codes[1])
    for e in range(spec.n_experts):
        data, scales = host.experts[e][2]
        s = scales.copy()
        s[:] = rng.integers(119, 126, s.shape, dtype=np.uint8)
        # the range's two ends, in blocks of every expert's down matrix
        s[0, 0], s[-1, -1] = codes
        host.experts[e][2] = (data, s)
    for T in (5, 40):
        x = synth.activations(f"x.f16range.{T}", T, spec.hidden)
        layer = moe_mod().MoeLayer(host, max_tokens=T)
        y, ids, _ = layer.forward(torch.from_numpy(x).cuda())
        layer.sync()
        ref = _oracle(host, x)
        assert ids_match(ids.cpu().numpy(), ref.ids, _scores(spec, ref, host.correction_bias))
        err = rel_l2(y.cpu().numpy(), ref.output)
        print(f"{name} codes {codes} T={T}: rel L2 {err:.3e}")
        assert err < REL_L2_BAR, err
        layer.close()


def test_invalid_payloads_rejected_at_create():
    host = _small_layer("c3_mxfp4_decode")
    host.experts[3][1][1][2, 1] = 0xFF
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(host, max_tokens=1)
    assert e.value.status == N.ERR_INVALID_SCALE
    host = _small_layer("c4_mxfp8")
    host.experts[2][2][0][5, 9] = 0x7F
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(host, max_tokens=1)
    assert e.value.status == N.ERR_NONFINITE
    host = _small_layer("c1_bf16_decode")
    host.experts[0][0][0][0, 0] = 0x7F80
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(host, max_tokens=1)
    assert e.value.status == N.ERR_NONFINITE
    host = _small_layer("c5_mxfp4_zipf_prefill")
    host.correction_bias[4] = np.nan
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(host, max_tokens=1)
    assert e.value.status == N.ERR_INVALID_GEOMETRY


def test_shape_and_geometry_errors():
    import dataclasses
    host = _small_layer("c3_mxfp4_decode")
    bad = dataclasses.replace(host.spec, n_group=3)
    h2 = C.HostLayer(bad, host.router_weight, host.experts, host.shared)
    with pytest.raises(N.UrbError) as e:
        moe_mod().MoeLayer(h2, max_tokens=1)
    assert e.value.status == N.ERR_INVALID_GEOMETRY
    for dims in ({"hidden": 192}, {"intermediate": 96}, {"hidden": 12288 + 128}):
        bad = dataclasses.replace(host.spec, **dims)
        h3 = C.HostLayer(bad, host.router_weight, host.experts, host.shared)
        with pytest.raises(N.UrbError) as e:
            moe_mod().MoeLayer(h3, max_tokens=1)
        assert e.value.status == N.ERR_SHAPE
    # route_sqrt_softplus: validate_positive(scale) -> invalid, non-finite bias -> NonFinite
    # (deepseek_v4/math.rs:468-475); the router belongs to the GLM composition only.
    ssp = dataclasses.replace(host.spec, router=C.ROUTER_SQRT_SOFTPLUS)
    nan_bias = np.zeros(ssp.n_experts, np.float32)
    nan_bias[3] = np.nan
    for spec, bias, status in (
            (dataclasses.replace(ssp, routed_scaling_factor=0.0), None, N.ERR_INVALID_GEOMETRY),
            (ssp, nan_bias, N.ERR_NONFINITE),
            (dataclasses.replace(ssp, composition=C.COMPOSE_QWEN36), None, N.ERR_ARGUMENT)):
        h4 = C.HostLayer(spec, host.router_weight, host.experts, host.shared, bias)
        with pytest.raises(N.UrbError) as e:
            moe_mod().MoeLayer(h4, max_tokens=1)
        assert e.value.status == status
    layer = moe_mod().MoeLayer(host, max_tokens=2)
    x = torch.zeros((3, host.spec.hidden), device="cuda")
    with pytest.raises(N.UrbError) as e:
        layer.forward(x)  # more tokens than max_tokens
    assert e.value.status == N.ERR_SHAPE
    # an empty batch (valid buffers, 0 tokens): a shape error, nothing enqueued
    y = torch.empty((1, host.spec.hidden), device="cuda")
    assert N.moe_lib().urb_moe_forward(layer._ctx, x.data_ptr(), 0, y.data_ptr(), None, None,
                                       None) == N.ERR_SHAPE
    layer.close()


# ------------------------------------------------------------------------------- full size
# The five configurations at their benchmark sizes, the c5 layer with its two single-beta Zipf
# biases ("flat", "hot"), the MX-activation compositions, the Qwen3.6 release layer with its
# gated shared expert and DeepSeek-V4 Flash (score- and hash-routed), each with the benchmark's
# own bias: every token's ids, route weights and outputs against the oracle.
FULL = [("c1_bf16_decode", 1), ("c2_bf16_prefill", 128), ("c3_mxfp4_decode", 1),
        ("c3_mxfp4_decode", 32), ("c4_mxfp8", 1), ("c4_mxfp8", 512),
        ("c5_mxfp4_zipf_prefill", 1024), ("c5_mxfp4_zipf_flat", 1024),
        ("c5_mxfp4_zipf_hot", 1024),
        ("c4_mxfp8_mx_activation", 1), ("c4_mxfp8_mx_activation", 512),
        ("c5_mxfp4_mx_activation", 1024), ("c5_mxfp4_dsv41", 1),
        ("c5_mxfp4_dsv41", 1024), ("qwen36_release", 1), ("qwen36_release", 128),
        ("dsv4_flash", 1), ("dsv4_flash", 1024), ("dsv4_flash_hash", 1),
        ("dsv4_flash_hash", 1024)]

ORACLE_THREADS = max(1, min(16, os.cpu_count() or 1))


def _full_layer(name, T):
    w = C.workload(name)
    spec = w.spec
    _, bias = C.workload_bias(w)
    dev = moe_mod().DeviceLayer.synthesize(spec, correction_bias=bias)
    tok = None
    if w.hash_vocab:
        dev.hash_experts = torch.from_numpy(C.hash_table(w.hash_vocab, spec.n_experts,
                                                         spec.top_k)).cuda()
        ids_tok = synth.splitmix64(synth.stream_seed("bench.tokens"), 0, T) % np.uint64(
            w.hash_vocab)
        tok = torch.from_numpy(ids_tok.astype(np.int32)).cuda()
    x = moe_mod().synth_activations(T, spec.hidden)
    layer = moe_mod().MoeLayer(dev, max_tokens=T)
    y, ids, wts = layer.forward(x, token_ids=tok)
    layer.sync()
    return (spec, bias, dev, x, tok, layer, y.cpu().numpy(), ids.cpu().numpy(),
            wts.cpu().numpy())


def _route_weights_match(ids, wts, ref_ids, ref_w):
    """Route weights of every token whose ids equal the oracle's (a near-tie swap changes the
    selected set, and with it the normaliser); returns the tokens compared."""
    same = np.all(ids == ref_ids, axis=1)
    assert np.allclose(wts[same], ref_w[same], rtol=1e-5, atol=1e-7)
    return int(same.sum())


@pytest.mark.parametrize("name,T", FULL)
def test_full_size_workload_matches_oracle_on_every_token(name, T):
    spec, bias, dev, x, tok, layer, y, ids, wts = _full_layer(name, T)
    print(f"{name} T={T}: {len(np.unique(ids))} experts, hottest routed by "
          f"{np.bincount(ids.ravel()).max()} tokens", flush=True)
    host = dev.to_host(experts=sorted(set(ids.ravel().tolist())))
    ts = None if tok is None else tok.cpu().numpy()
    ref = _oracle(host, x.cpu().numpy(), threads=ORACLE_THREADS, token_ids=ts)
    assert ids_match(ids, ref.ids, _scores(spec, ref, bias))
    same = _route_weights_match(ids, wts, ref.ids, ref.weights)
    assert same >= T - max(1, T // 100), f"only {same} of {T} tokens with the oracle's ids"
    err = rel_l2(y, ref.output)
    worst = max(rel_l2(y[t], ref.output[t]) for t in range(T))
    print(f"{name} T={T}: rel L2 {err:.3e} over all tokens, worst token {worst:.3e}, route "
          f"weights equal on {same} tokens")
    assert err < REL_L2_BAR
    layer.close()
