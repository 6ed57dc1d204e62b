// urb_combine.hip -- the weighted combines, payload validation and the dequantisation hook.
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {

// ------------------------------------------------------------------------------------------
// Combines.
// Qwen (src/models/qwen3_6/runtime.rs:1398-1415): routes in ascending expert id,
//   c = bf16(w * y), acc = bf16(acc + c), acc from +0.0.
// GLM (src/models/glm/runtime/moe.rs:162-171): acc = f64(shared) (or 0), then in ranking
//   order acc += f64(w) * f64(y); out = f32(acc).
// Every input row is read once and the output is not read back by this call, so both go
// through non-temporal loads and stores (GLM, 1024 tokens x 8 routes x 7168: 54 -> 50 us).
// ------------------------------------------------------------------------------------------
template <int KMAX>
__global__ __launch_bounds__(256) void combine_qwen_kernel(const float* __restrict__ y,
                                                           const int32_t* __restrict__ pos,
                                                           const float* __restrict__ w,
                                                           const int32_t* __restrict__ asc,
                                                           int T, int K, int H,
                                                           const float* __restrict__ res,
                                                           const float* __restrict__ shared,
                                                           const float* __restrict__ gate,
                                                           float* __restrict__ out,
                                                           int* status) {
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (h4 * 4 >= H) return;
  // all route metadata first, then every expert row: two dependent round trips in total
  int rk[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) rk[j] = j < K ? asc[(size_t)t * K + j] : 0;
  float wt[KMAX];
  float4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      wt[j] = w[(size_t)t * K + rk[j]];
      const int p = pos ? pos[(size_t)t * K + rk[j]] : rk[j];
      v[j] = u2f4(ldg16_stream(y + (size_t)p * H + 4 * h4));
    }
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool bad = false;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      const float vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float c;
        if (!rne_bf16(wt[j] * vv[u], &c)) { bad = true; c = wt[j] * vv[u]; }
        const float s = acc[u] + c;
        if (!rne_bf16(s, &acc[u])) { bad = true; acc[u] = s; }
      }
    }
  }
  if (shared) {
    // the gated shared expert, added last (src/models/qwen3_6/runtime.rs:1449-1461):
    // c = bf16(scale * s), acc = bf16(acc + c)
    const float sc = qwen_shared_scale(gate[t], bad);
    const float4 s4 = u2f4(ldg16_stream(shared + (size_t)t * H + 4 * h4));
    const float ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float c;
      if (!rne_bf16(sc * ss[u], &c)) { bad = true; c = sc * ss[u]; }
      const float a = acc[u] + c;
      if (!rne_bf16(a, &acc[u])) { bad = true; acc[u] = a; }
    }
  }
  if (res) {
    // add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494)
    const float4 r4 = u2f4(ldg16_stream(res + (size_t)t * H + 4 * h4));
    const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float s = rr[u] + acc[u];
      if (!rne_bf16(s, &acc[u])) { bad = true; acc[u] = s; }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
  stg16_stream(out + (size_t)t * H + 4 * h4, make_float4(acc[0], acc[1], acc[2], acc[3]));
}

template <int KMAX>
__global__ __launch_bounds__(256) void combine_glm_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ pos,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ shared,
                                                          int T, int K, int H,
                                                          float* __restrict__ out) {
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (h4 * 4 >= H) return;
  float wt[KMAX];
  float4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      wt[j] = w[(size_t)t * K + j];
      const int p = pos ? pos[(size_t)t * K + j] : j;
      v[j] = u2f4(ldg16_stream(y + (size_t)p * H + 4 * h4));
    }
  }
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  if (shared) {
    const float4 s = u2f4(ldg16_stream(shared + (size_t)t * H + 4 * h4));
    acc[0] = s.x; acc[1] = s.y; acc[2] = s.z; acc[3] = s.w;
  }
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      const double wd = (double)wt[j];
      acc[0] += wd * (double)v[j].x;
      acc[1] += wd * (double)v[j].y;
      acc[2] += wd * (double)v[j].z;
      acc[3] += wd * (double)v[j].w;
    }
  }
  stg16_stream(out + (size_t)t * H + 4 * h4,
               make_float4((float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]));
}

void launch_combine_qwen(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                         const int32_t* asc, int T, int K, int H, float* out, int* status,
                         hipStream_t s, const float* residual, const float* shared,
                         const float* gate) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_qwen_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H,
                                                residual, shared, gate, out, status);
  else
    combine_qwen_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H,
                                                 residual, shared, gate, out, status);
}

void launch_combine_glm(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                        const float* shared, int T, int K, int H, float* out, hipStream_t s) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_glm_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, shared, T, K, H, out);
  else
    combine_glm_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, shared, T, K, H,
                                                out);
}

// ------------------------------------------------------------------------------------------
// Payload validation (one pass at create):
//   BF16  any element with an all-ones exponent (src/model/bf16.rs:743-773)     -> bit 1
//   MXFP8 any E4M3 code with magnitude 0x7F (src/math/mxfp.rs:880-888)          -> bit 1
//   MX    any E8M0 scale 0xFF (src/math/mxfp.rs:890-898, 1431-1435)             -> bit 2
// ------------------------------------------------------------------------------------------
__global__ void validate_kernel(int fmt, const uint8_t* __restrict__ data, size_t nbytes,
                                const uint8_t* __restrict__ scales, size_t sbytes, int* flags,
                                int f16_lo, int f16_hi) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t tid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  int f = 0;
  if (fmt != kFmtMXFP4) {
    const size_t n4 = nbytes / 4;
    const uint32_t* d4 = reinterpret_cast<const uint32_t*>(data);
    for (size_t i = tid; i < n4; i += stride) {
      uint32_t v = d4[i];
      if (fmt == kFmtBF16) {
        if ((v & 0x7f80u) == 0x7f80u || ((v >> 16) & 0x7f80u) == 0x7f80u) f |= 1;
      } else {
        for (int b = 0; b < 4; ++b)
          if (((v >> (8 * b)) & 0x7fu) == 0x7fu) f |= 1;
      }
    }
    for (size_t i = n4 * 4 + tid; i < nbytes; i += stride) {
      if (fmt == kFmtBF16) {
        // a dangling half of a BF16 element cannot occur (nbytes is even and 4-aligned rows)
      } else if ((data[i] & 0x7fu) == 0x7fu) {
        f |= 1;
      }
    }
  }
  for (size_t i = tid; i < sbytes; i += stride) {
    const int v = scales[i];
    if (v == 0xff) f |= 2;
    if (f16_lo <= f16_hi && (v < f16_lo || v > f16_hi)) f |= 4;
  }
  if (f) atomicOr(flags, f);
}

void launch_validate(int fmt, const uint8_t* data, size_t data_bytes, const uint8_t* scales,
                     size_t scale_bytes, int* flags, hipStream_t s, bool f16_range) {
  size_t work = std::max(data_bytes / 4, scale_bytes);
  int blocks = (int)std::min<size_t>(std::max<size_t>((work + 255) / 256, 1), 4096);
  const int lo = f16_range ? kF16ScaleLo[fmt] : 1, hi = f16_range ? kF16ScaleHi[fmt] : 0;
  validate_kernel<<<blocks, 256, 0, s>>>(fmt, data, data_bytes, scales, scale_bytes, flags, lo,
                                         hi);
}

// Dequantised rows, value = decode(code) * scale in f32 (bit-exact parity hook).
__global__ void dequant_kernel(int fmt, const uint8_t* __restrict__ data,
                               const uint8_t* __restrict__ scales, int cols, int row0, int count,
                               float* __restrict__ out) {
  const size_t n = (size_t)count * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = row0 + i / cols;
    const int c = (int)(i % cols);
    float v;
    if (fmt == kFmtBF16) {
      const uint16_t* d = reinterpret_cast<const uint16_t*>(data);
      v = u2f((uint32_t)d[r * cols + c] << 16);
    } else if (fmt == kFmtMXFP4) {
      uint32_t byte = data[r * (cols / 2) + c / 2];
      f32x2 pair = fp4x2<0>(byte);
      // The conversion yields -0.0 for code 8; the reference table holds +0.0 there
      // (src/math/mxfp.rs:73-79).  Adding +0.0 maps -0.0 to +0.0 and leaves the rest exact.
      v = (pair[c & 1] + 0.0f) * e8m0_to_f32(scales[r * (cols / 32) + c / 32]);
    } else {
      uint32_t byte = data[r * cols + c];
      f32x2 pair = fp8x2<false>(byte);
      v = pair[0] * e8m0_to_f32(scales[r * (cols / 32) + c / 32]);
    }
    out[i] = v;
  }
}

void launch_dequant(int fmt, const uint8_t* data, const uint8_t* scales, int rows, int cols,
                    int row0, int count, float* out, hipStream_t s) {
  (void)rows;
  size_t n = (size_t)count * cols;
  int blocks = (int)std::min<size_t>((n + 255) / 256, 16384);
  dequant_kernel<<<std::max(blocks, 1), 256, 0, s>>>(fmt, data, scales, cols, row0, count, out);
}

__global__ void fill_i32_kernel(int32_t* p, int32_t v, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

void launch_fill_i32(int32_t* p, int32_t v, size_t n, hipStream_t s) {
  int blocks = (int)std::min<size_t>(std::max<size_t>((n + 255) / 256, 1), 1024);
  fill_i32_kernel<<<blocks, 256, 0, s>>>(p, v, n);
}

__global__ void check_finite_kernel(const float* __restrict__ x, size_t n, int* status) {
  bool bad = false;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    bad |= !finite(x[i]);
  if (bad) flag(status, kStatusNonFinite);
}

void launch_check_finite(const float* x, size_t n, int* status, hipStream_t s) {
  int blocks = (int)std::min<size_t>(std::max<size_t>((n + 255) / 256, 1), 1024);
  check_finite_kernel<<<blocks, 256, 0, s>>>(x, n, status);
}

}  // namespace urb
