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
#include "urb_quant.hpp"

#include <algorithm>

namespace urb {

// The quantizer over a whole [rows, cols] matrix: quantize_lanes (urb_quant.hpp), one lane per
// thread.
template <int VPT>
__global__ __launch_bounds__(256) void quantize_kernel(const float* x, size_t nblocks, int cols,
                                                       float* values,
                                                       uint8_t* __restrict__ codes,
                                                       uint8_t* __restrict__ scales, int* status,
                                                       int round_first,
                                                       const float* __restrict__ row_w,
                                                       const int32_t* __restrict__ row_slot,
                                                       uint16_t* __restrict__ pieces) {
  quantize_lanes<VPT>(x, nblocks, cols, values, codes, scales, status, round_first, row_w,
                      row_slot, pieces, blockIdx.x * (size_t)blockDim.x + threadIdx.x);
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
      v[j] = u2f4(ldg16_stream(y + (size_t)p * H + 4 * h4));
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
    const float4 sh = u2f4(ldg16_stream(shared + (size_t)t * H + 4 * h4));
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
  stg16_stream(out + (size_t)t * H + 4 * h4, make_float4(r[0], r[1], r[2], r[3]));
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
