// urb_block.hip -- the decoder layer's steps either side of the MoE call (Qwen3.6).
//
// The post-attention zero-centred RMSNorm with its BF16 cast feeds the router and the experts
// (src/models/qwen3_6/runtime.rs:1053-1057); the residual add after the combine
// (runtime.rs:1060) is fused into the combine kernels (urb_combine.hip, and the one-token
// down + combine kernel in urb_decode.hip).
//
// zero_centered_rms_norm (src/models/qwen3_8/norm.rs:38-52, 176-186): the mean square is the
// reference's left-to-right f32 sum of x*x divided by H, so one lane adds the products in index
// order (a tree sum would differ in the last bits and move router inputs across BF16 rounding
// boundaries); the products, the square root, the reciprocal and the scaling run in parallel.
// One token per 256-thread workgroup: the serial sum costs ~4 cycles per element, so H = 2048
// adds ~4 us, paid once per call for any token count.
#include "urb_device.hpp"
#include "urb_kernels.hpp"

namespace urb {

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ h,
                                                       const float* __restrict__ weight, int H,
                                                       float eps, float* __restrict__ out,
                                                       int* status) {
  extern __shared__ float4 sq[];  // [H / 4] squares
  __shared__ float inv_s;
  const int t = blockIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(h + (size_t)t * H);
  const float4* w4 = reinterpret_cast<const float4*>(weight);
  float4* o4 = reinterpret_cast<float4*>(out + (size_t)t * H);
  const int n4 = H / 4;
  bool bad = false;
  for (int i = threadIdx.x; i < n4; i += blockDim.x) {
    const float4 v = x4[i];
    bad |= !finite(v.x) || !finite(v.y) || !finite(v.z) || !finite(v.w);
    sq[i] = make_float4(__fmul_rn(v.x, v.x), __fmul_rn(v.y, v.y), __fmul_rn(v.z, v.z),
                        __fmul_rn(v.w, v.w));
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // 128 squares per batch: the batch's LDS reads are issued together, then added in order
    constexpr int B = 32;
    float sum = 0.0f;
    auto add = [&](const float4& q) {
      sum = __fadd_rn(sum, q.x);
      sum = __fadd_rn(sum, q.y);
      sum = __fadd_rn(sum, q.z);
      sum = __fadd_rn(sum, q.w);
    };
    int i = 0;
    for (; i + B <= n4; i += B) {
      float4 q[B];
#pragma unroll
      for (int u = 0; u < B; ++u) q[u] = sq[i + u];
#pragma unroll
      for (int u = 0; u < B; ++u) add(q[u]);
    }
    for (; i < n4; ++i) add(sq[i]);
    const float mean_square = __fdiv_rn(sum, (float)H);
    // sqrtf and / are correctly rounded here (HIP's __fsqrt_rn is the 1-ulp native root)
    inv_s = 1.0f / sqrtf(__fadd_rn(mean_square, eps));
  }
  __syncthreads();
  const float inv = inv_s;
  bad |= !finite(inv);
  for (int i = threadIdx.x; i < n4; i += blockDim.x) {
    const float4 v = x4[i], w = w4[i];
    const float vv[4] = {v.x, v.y, v.z, v.w}, ww[4] = {w.x, w.y, w.z, w.w};
    float r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      bad |= !finite(ww[u]);
      const float o = __fmul_rn(__fmul_rn(vv[u], inv), __fadd_rn(1.0f, ww[u]));
      if (!rne_bf16(o, &r[u])) {
        bad = true;
        r[u] = o;
      }
    }
    o4[i] = make_float4(r[0], r[1], r[2], r[3]);
  }
  if (bad && status) flag(status, kStatusNonFinite);
}

void launch_rms_norm(const float* h, const float* weight, int T, int H, float eps, float* out,
                     int* status, hipStream_t s) {
  rms_norm_kernel<<<T, 256, (size_t)H * sizeof(float), s>>>(h, weight, H, eps, out, status);
}

}  // namespace urb
