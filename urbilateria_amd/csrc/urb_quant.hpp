// urb_quant.hpp -- simulate_e4m3_activation on the device: the quantizer's lane routine, shared
// by the quantize kernel (urb_hy4.hip) and the routers, which quantize a token's input as a
// side job of their launch (urb_route.hip).
#pragma once

#include "urb_device.hpp"
#include "urb_panel.hpp"

namespace urb {

// ------------------------------------------------------------------------------------------
// simulate_e4m3_activation as (code, scale) pairs.
// ------------------------------------------------------------------------------------------

// power_of_two_ceiling (src/math/mxfp.rs:300-319) for a positive finite normal value: the
// exponent increment, except near powers of two (mantissa <= 4096 or >= 2^23 - 1 - 4096), where
// the reference keeps 2^ceil(log2(v)) with an f32 logarithm.  log2 here is the f64 logarithm
// rounded to f32 (correctly rounded there: no mantissa in that band puts log2(v) near an f32
// rounding boundary).
__device__ __forceinline__ float pow2_ceiling(float v) {
  const uint32_t bits = f2u(v);
  const uint32_t exponent = bits & 0x7f800000u, mantissa = bits & 0x007fffffu;
  if (mantissa == 0) return v;
  if (exponent == 0 || mantissa <= 4096u || mantissa >= 0x007fffffu - 4096u) {
    const float l = (float)log2((double)v);
    return ldexpf(1.0f, (int)ceilf(l));
  }
  return u2f(exponent + 0x00800000u);
}

// encode_e4m3fn_finite (src/math/mxfp.rs:246-275): clamp to +-448, round to nearest even on the
// E4M3 grid (subnormals below 2^-6 on the 2^-9 grid), saturate at code 0x7E; -0 encodes as 0.
__device__ __forceinline__ uint32_t encode_e4m3(float value) {
  value = fminf(fmaxf(value, -448.0f), 448.0f);
  const float mag = fabsf(value);
  if (mag == 0.0f) return 0;
  uint32_t code;
  if (mag < 0.015625f) {
    code = (uint32_t)rintf(mag * 512.0f);
  } else {
    const uint32_t b = f2u(mag);
    const uint32_t r = (b + 0x7ffffu + ((b >> 20) & 1u)) & ~0xfffffu;
    const uint32_t e = (r >> 23) & 0xffu;
    const uint32_t ex = e > 120u ? e - 120u : 0u;
    code = min((ex << 3) | ((r >> 20) & 7u), 0x7eu);
  }
  return (value < 0.0f && code != 0) ? (code | 0x80u) : code;
}

// One 32-lane half wavefront per block of 32 * VPT values of a row-major [rows, cols] f32
// matrix (cols % (32 * VPT) == 0), VPT consecutive values per lane: 32-value blocks (Hy4,
// DeepSeek V4.1) with VPT 1, DeepSeek V4's 128-value blocks with VPT 4.  Outputs (each
// optional): the simulated values decode(code) * scale (`values` may alias x: every lane reads
// its elements before any lane writes), the codes [rows, cols] and the scales
// [rows, cols / (32 * VPT)] (the E8M0 byte is the biased exponent of the power-of-two scale).
// Non-finite input -> status (mxfp.rs:93-99).
template <int VPT>
__device__ __forceinline__ void quantize_lanes(const float* x, size_t nblocks, int cols,
                                               float* values, uint8_t* __restrict__ codes,
                                               uint8_t* __restrict__ scales, int* status,
                                               int round_first, const float* __restrict__ row_w,
                                               const int32_t* __restrict__ row_slot,
                                               uint16_t* __restrict__ pieces, size_t gid) {
  const size_t blk = gid >> 5;
  const size_t e0 = gid * VPT;  // first element of this lane
  const bool live = blk < nblocks;
  float v[VPT];
  if constexpr (VPT == 4) {
    const float4 q = live ? *reinterpret_cast<const float4*>(x + e0)
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    v[0] = live ? x[e0] : 0.0f;
  }
  if (round_first && live) {
    // the lane's values lie in one row (cols is a multiple of the block)
    const float rw = row_w ? row_w[row_slot ? row_slot[e0 / (size_t)cols] : e0 / (size_t)cols]
                           : 1.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      float r;
      const float p = row_w ? v[j] * rw : v[j];
      if (!rne_bf16(p, &r) && status) flag(status, kStatusNonFinite);
      else v[j] = r;
    }
  }
  float a = fabsf(v[0]);
#pragma unroll
  for (int j = 1; j < VPT; ++j) a = fmaxf(a, fabsf(v[j]));
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  if (!live) return;
  bool fin = true;
#pragma unroll
  for (int j = 0; j < VPT; ++j) fin = fin && finite(v[j]);
  if (!fin && status) flag(status, kStatusNonFinite);
  a = fmaxf(a, 1.0e-4f);  // fold(1.0e-4, f32::max) over |x| (mxfp.rs:104-107)
  const float scale = pow2_ceiling(a / 448.0f);
  uint32_t code[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) code[j] = encode_e4m3(v[j] / scale);
  if (values || pieces) {
    // E4M3 code -> value via the conversion instruction (exact), times the power of two
    float d[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      d[j] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code[j], 1.0f, false)[0] * scale;
    if (values) {
      if constexpr (VPT == 4)
        *reinterpret_cast<float4*>(values + e0) = make_float4(d[0], d[1], d[2], d[3]);
      else
        values[e0] = d[0];
    }
    if (pieces) {
      const size_t row = e0 / (size_t)cols;
      const int col = (int)(e0 - row * (size_t)cols);
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        store_piece_value(pieces + row * (size_t)(cols / 8) * kPieceUnit, col + j, d[j]);
    }
  }
  if (codes)
#pragma unroll
    for (int j = 0; j < VPT; ++j) codes[e0 + j] = (uint8_t)code[j];
  if (scales && (gid & 31) == 0) scales[blk] = (uint8_t)(f2u(scale) >> 23);
}

}  // namespace urb
