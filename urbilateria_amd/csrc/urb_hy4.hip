// urb_hy4.hip -- the MX-activation mode (Hy4 composition): the activation quantizer and the
// combine.  The projections run on the BF16 MFMA kernels (urb_gemm.hip, urb_decode.hip): a
// simulated E4M3 activation is an E4M3 code times a power of two, exactly a BF16 value, so
// the A operand needs no low half and every product is exact; the f32 accumulation of those
// kernels then stays within f32 rounding of the reference's sums.
//
// (CDNA4's v_mfma_scale_f32_16x16x128_f8f6f4 takes the codes and E8M0 scales as they are, but
// its sum of 128 products is not accurate to f32: measured on MI355X, its error reaches
// ~2e-4 of the sum of |products| for full-range E4M3/E2M1 operands.  The BF16 rounding and
// E4M3 re-quantization between Hy4's projections amplify that past the layer's parity bar, so
// the scaled MFMA is not used here; tests/test_gpu_parity.py pins its operand layout.)
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

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
__global__ __launch_bounds__(256) void quantize_kernel(const float* x, size_t nblocks, int cols,
                                                       float* values,
                                                       uint8_t* __restrict__ codes,
                                                       uint8_t* __restrict__ scales, int* status,
                                                       int round_first,
                                                       const float* __restrict__ row_w,
                                                       const int32_t* __restrict__ row_slot,
                                                       uint16_t* __restrict__ pieces) {
  const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
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

void launch_quantize(const float* x, size_t rows, size_t cols, float* values, uint8_t* codes,
                     uint8_t* scales, int* status, hipStream_t s, int round_first,
                     const float* row_w, const int32_t* row_slot, int block, uint16_t* pieces) {
  const size_t nblocks = rows * cols / block;
  const size_t threads = nblocks * 32;
  const unsigned grid = (unsigned)((threads + 255) / 256);
  if (block == 128)
    quantize_kernel<4><<<grid, 256, 0, s>>>(x, nblocks, (int)cols, values, codes, scales, status,
                                            round_first, row_w, row_slot, pieces);
  else
    quantize_kernel<1><<<grid, 256, 0, s>>>(x, nblocks, (int)cols, values, codes, scales, status,
                                            round_first, row_w, row_slot, pieces);
}

// ------------------------------------------------------------------------------------------
// Combine (Hy4 MoeWeights::forward, src/models/hy4/runtime.rs:1387-1445): out = 0; for the
// routes in ascending expert id, out += w * y (f32 multiply, f32 add); out += shared; BF16.
// Without weights (DeepSeek V4.1, deepseek_v41/runtime.rs:1995-2017) out += y (1 * y is y).
// ------------------------------------------------------------------------------------------
template <int KMAX>
__global__ __launch_bounds__(256) void combine_hy4_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ pos,
                                                          const float* __restrict__ w,
                                                          const int32_t* __restrict__ asc,
                                                          const float* __restrict__ shared,
                                                          int T, int K, int H,
                                                          float* __restrict__ out,
                                                          int* status) {
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (h4 * 4 >= H) return;
  int rk[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) rk[j] = j < K ? asc[(size_t)t * K + j] : 0;
  float wt[KMAX];
  float4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      wt[j] = w ? w[(size_t)t * K + rk[j]] : 1.0f;
      const int p = pos ? pos[(size_t)t * K + rk[j]] : rk[j];
      v[j] = reinterpret_cast<const float4*>(y + (size_t)p * H)[h4];
    }
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      acc[0] = acc[0] + wt[j] * v[j].x;
      acc[1] = acc[1] + wt[j] * v[j].y;
      acc[2] = acc[2] + wt[j] * v[j].z;
      acc[3] = acc[3] + wt[j] * v[j].w;
    }
  }
  if (shared) {
    const float4 sh = reinterpret_cast<const float4*>(shared + (size_t)t * H)[h4];
    acc[0] = acc[0] + sh.x;
    acc[1] = acc[1] + sh.y;
    acc[2] = acc[2] + sh.z;
    acc[3] = acc[3] + sh.w;
  }
  bool bad = false;
  float r[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (!rne_bf16(acc[u], &r[u])) {
      bad = true;
      r[u] = acc[u];
    }
  if (bad) flag(status, kStatusNonFinite);
  reinterpret_cast<float4*>(out + (size_t)t * H)[h4] = make_float4(r[0], r[1], r[2], r[3]);
}

void launch_combine_hy4(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                        const int32_t* asc, const float* shared, int T, int K, int H,
                        float* out, int* status, hipStream_t s) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_hy4_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, shared, T, K,
                                                H, out, status);
  else
    combine_hy4_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, shared, T,
                                                 K, H, out, status);
}

}  // namespace urb
