// urb_synth.hip -- device-side generator for the seeded synthetic workloads.
//
// Bit-for-bit the same definition as urbilateria_amd/synth.py: SplitMix64 (the reference's
// src/generation.rs:419-440) indexed by draw number, Box-Muller normals on draws 2i and 2i+1,
// RNE BF16, E2M1 nibbles from the low 4 bits of each draw, E8M0 = 119 + draw % 7, E4M3 = the
// nearest-even finite encoding of clamp(N(0,1), +-448).  Used to build full-size layers
// directly in HBM; these entry points are workload tooling, not part of the MoE ABI.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "urb_panel.hpp"

namespace urb {

// ---- operands of v_mfma_scale_f32_16x16x128_f8f6f4 (one 128-k step), for the layout probe ----
// Lane l = ln + 16 c of a wavefront feeds row ln of a 16-row block.  Measured operand layout:
//   E4M3: bytes 0..15 = k 16 c + [0, 16), bytes 16..31 = k 64 + 16 c + [0, 16);
//   E2M1: nibbles 0..31 (low nibble first) = k 32 c + [0, 32), bytes 16..31 unused;
// and the E8M0 scale a lane supplies covers k 32 c + [0, 32) of its row, i.e. MX block
// 4 step + c: one byte per lane, as the panel scale slabs hold them.
typedef int i32x8 __attribute__((ext_vector_type(8)));

// An MXFP4 panel slab's unit (block 4 step + c of row ln) is the E2M1 operand as it stands.
__device__ __forceinline__ i32x8 mx_operand(const BRaw<kFmtMXFP4>& r) {
  return i32x8{(int)r.q.x, (int)r.q.y, (int)r.q.z, (int)r.q.w, 0, 0, 0, 0};
}

// MXFP8 slabs 2 step and 2 step + 1 give lane group c the halves P_c, Q_c of block
// 4 step + c; the E4M3 operand wants (P_{c/2} | P_{2+c/2}) for even c and (Q_{c/2} | Q_{2+c/2})
// for odd c.  permlane16_swap(P, Q) = ([P0 Q0 P2 Q2], [P1 Q1 P3 Q3]) (rows of 16 lanes), then
// permlane32_swap of those = ([P0 Q0 P1 Q1], [P2 Q2 P3 Q3]).
__device__ __forceinline__ i32x8 mx_operand(const BRaw<kFmtMXFP8>& r) {
  const uint32_t p[4] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[0].w};
  const uint32_t q[4] = {r.q[1].x, r.q[1].y, r.q[1].z, r.q[1].w};
  i32x8 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto a = __builtin_amdgcn_permlane16_swap(p[i], q[i], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(a[0], a[1], false, false);
    o[i] = (int)b[0];
    o[4 + i] = (int)b[1];
  }
  return o;
}

// Quantized activations staged in LDS: one 128-byte step of a row at pitch kQLd (the 16-byte
// pad makes the 16 rows of a lane group hit distinct banks).
constexpr int kQLd = kKS + 16;
__device__ __forceinline__ i32x8 lds_qfrag(const uint8_t* base, int m, int c) {
  const uint4 lo = *reinterpret_cast<const uint4*>(base + m * kQLd + 16 * c);
  const uint4 hi = *reinterpret_cast<const uint4*>(base + m * kQLd + 64 + 16 * c);
  return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

template <int FMT>
__device__ __forceinline__ f32x4 mfma_mx(const i32x8& a, int sa, const i32x8& b, int sb,
                                         f32x4 c) {
  // A: E4M3 (format 0); B: E2M1 (format 4) or E4M3.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, FMT == kFmtMXFP4 ? 4 : 0,
                                                          0, sa, 0, sb);
}

}  // namespace urb

namespace {

__device__ __forceinline__ uint64_t splitmix(uint64_t seed, uint64_t n) {
  uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ double unit(uint64_t u) {
  return (double)(u >> 11) * (1.0 / 9007199254740992.0);
}
__device__ __forceinline__ float normal(uint64_t seed, uint64_t i, double mean, double std) {
  double u0 = unit(splitmix(seed, 2 * i)), u1 = unit(splitmix(seed, 2 * i + 1));
  double z = sqrt(-2.0 * log(1.0 - u0)) * cos(6.283185307179586 * u1);
  return (float)(mean + std * z);
}
__device__ __forceinline__ uint16_t bf16_bits(float v) {
  uint32_t b = __float_as_uint(v);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ uint8_t e4m3_encode(float value) {
  value = fminf(fmaxf(value, -448.0f), 448.0f);
  float mag = fabsf(value);
  if (mag == 0.0f) return 0;
  uint32_t code;
  if (mag < 0.015625f) {
    code = (uint32_t)rintf(mag * 512.0f);
  } else {
    uint32_t bits = __float_as_uint(mag);
    uint32_t rounded = (bits + ((1u << 19) - 1) + ((bits >> 20) & 1u)) & 0xfff00000u;
    uint32_t e = (rounded >> 23) & 0xffu;
    e = e > 120 ? e - 120 : 0;
    code = min((e << 3) | ((rounded >> 20) & 7u), 0x7eu);
  }
  if (signbit(value) && code != 0) code |= 0x80u;
  return (uint8_t)code;
}

__global__ void bf16_kernel(uint64_t seed, size_t n, double mean, double std, uint16_t* out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = bf16_bits(normal(seed, i, mean, std));
}
__global__ void act_kernel(uint64_t seed, size_t n, float* out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = __uint_as_float((uint32_t)bf16_bits(normal(seed, i, 0.0, 1.0)) << 16);
}
__global__ void fp4_kernel(uint64_t seed, size_t nbytes, uint8_t* out) {
  for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nbytes;
       b += (size_t)gridDim.x * blockDim.x) {
    uint32_t lo = (uint32_t)(splitmix(seed, 2 * b) & 0xf);
    uint32_t hi = (uint32_t)(splitmix(seed, 2 * b + 1) & 0xf);
    out[b] = (uint8_t)(lo | (hi << 4));
  }
}
__global__ void fp8_kernel(uint64_t seed, size_t n, uint8_t* out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = e4m3_encode(normal(seed, i, 0.0, 1.0));
}
__global__ void e8m0_kernel(uint64_t seed, size_t n, uint8_t* out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = (uint8_t)(119 + splitmix(seed, i) % 7);
}

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// One v_mfma_f32_16x16x32_bf16 with operands placed by the lane layout the GEMM kernels
// assume: A lane l holds row l%16, k = 8*(l/16) + [0,8); B lane l holds column l%16, the same
// k range; C lane l holds column l%16, rows 4*(l/16) + [0,4).
__global__ void mfma_layout_kernel(const float* A, const float* B, float* C) {
  const int l = threadIdx.x;
  bf16x8_t a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)A[(l % 16) * 32 + 8 * (l / 16) + i];
    b[i] = (__bf16)B[(8 * (l / 16) + i) * 16 + (l % 16)];
  }
  f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  for (int i = 0; i < 4; ++i) C[(4 * (l / 16) + i) * 16 + (l % 16)] = c[i];
}

// Scaled conversions to BF16 as the GEMM B-operand path uses them: element i of `codes`
// (E2M1 nibble in the low 4 bits for fmt 1, E4M3 byte for fmt 2) times E8M0 scale `scales[i]`.
__global__ void cvt_bf16_kernel(int fmt, const uint8_t* codes, const uint8_t* scales, int n,
                                uint16_t* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t sb = (uint32_t)scales[i] << 23;
  float scale = __uint_as_float(sb ? sb : 0x00400000u);
  bf16x2_t v;
  if (fmt == 1) v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((uint32_t)codes[i] & 0xf, scale, 0);
  else v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)codes[i], scale, false);
  out[i] = __builtin_bit_cast(uint16_t, v[0]);
}

// hi/lo BF16 split of the GEMM activation staging, for n / 2 float pairs.
__global__ void split_bf16_kernel(const float* x, int pairs, uint32_t* hi, uint32_t* lo) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  uint32_t h, l;
  urb::split_bf16(x[2 * i], x[2 * i + 1], h, l);
  hi[i] = h;
  lo[i] = l;
}

// One v_mfma_scale_f32_16x16x128_f8f6f4 step built by the operand helpers above: A = a row-major [16][128] E4M3 matrix with [16][4] E8M0 scales,
// staged in LDS and read as lds_qfrag does; B = 16 weight rows as one panel's 128-column step
// (MXFP4 packed [16][64] or MXFP8 [16][128], scales [16][4]) loaded into the panel lanes
// (unit ln + 16 c = row ln, block c; MXFP8 as the two half-block slabs) and turned into the
// operand by mx_operand.  C[16][16] = A . B^T in the C layout of the BF16 MFMA.
template <int FMT>
__global__ void mfma_scale_layout_kernel(const uint8_t* A, const uint8_t* sa, const uint8_t* B,
                                         const uint8_t* sb, float* C) {
  using namespace urb;
  __shared__ __attribute__((aligned(16))) uint8_t aq[16 * kQLd];
  const int l = threadIdx.x, r = l % 16, c = l / 16;
  for (int i = l; i < 16 * 128; i += 64) aq[(i / 128) * kQLd + i % 128] = A[i];
  __syncthreads();
  const i32x8 a = lds_qfrag(aq, r, c);
  BRaw<FMT> raw;
  if constexpr (FMT == kFmtMXFP4) {
    raw.q = *reinterpret_cast<const uint4*>(B + r * 64 + 16 * c);
  } else {
    raw.q[0] = *reinterpret_cast<const uint4*>(B + r * 128 + 32 * c);
    raw.q[1] = *reinterpret_cast<const uint4*>(B + r * 128 + 32 * c + 16);
  }
  raw.s = sb[r * 4 + c];
  const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4_t acc = mfma_mx<FMT>(a, sa[r * 4 + c], mx_operand(raw), (int)raw.s, z);
  for (int i = 0; i < 4; ++i) C[(4 * c + i) * 16 + r] = acc[i];
}

int grid_for(size_t n) {
  size_t b = (n + 255) / 256;
  return (int)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

}  // namespace

extern "C" {

// BF16 N(mean, std) matrix, `n` elements of u16 bits.
int urb_synth_bf16(uint64_t seed, size_t n, double mean, double std, void* out, void* stream) {
  bf16_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, n, mean, std, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// N(0, 1) activations rounded to BF16, as f32.
int urb_synth_activations(uint64_t seed, size_t n, float* out, void* stream) {
  act_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, n, out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// E2M1 nibbles, `nbytes` packed bytes (two codes per byte, low nibble first).
int urb_synth_fp4(uint64_t seed, size_t nbytes, void* out, void* stream) {
  fp4_kernel<<<grid_for(nbytes), 256, 0, (hipStream_t)stream>>>(seed, nbytes, (uint8_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// E4M3FN codes of clamp(N(0,1), +-448).
int urb_synth_fp8(uint64_t seed, size_t n, void* out, void* stream) {
  fp8_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, n, (uint8_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// E8M0 scales 119 + draw % 7.
int urb_synth_e8m0(uint64_t seed, size_t n, void* out, void* stream) {
  e8m0_kernel<<<grid_for(n), 256, 0, (hipStream_t)stream>>>(seed, n, (uint8_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// Diagnostics: C[16,16] = A[16,32] . B[32,16] through one MFMA (device f32 arrays).
int urb_probe_mfma_16x16x32(const float* A, const float* B, float* C, void* stream) {
  mfma_layout_kernel<<<1, 64, 0, (hipStream_t)stream>>>(A, B, C);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// Diagnostics: C[16,16] = (A * sa)[16,128] . (B * sb)[16,128]^T through one scaled MFMA step
// of the MX-activation kernels.
// fmt_b: 1 = MXFP4 weights, 2 = MXFP8 weights.
int urb_probe_mfma_scale_16x16x128(int fmt_b, const void* A, const void* sa, const void* B,
                                   const void* sb, float* C, void* stream) {
  const uint8_t *a = (const uint8_t*)A, *as = (const uint8_t*)sa, *b = (const uint8_t*)B,
                *bs = (const uint8_t*)sb;
  if (fmt_b == 1)
    mfma_scale_layout_kernel<urb::kFmtMXFP4><<<1, 64, 0, (hipStream_t)stream>>>(a, as, b, bs, C);
  else if (fmt_b == 2)
    mfma_scale_layout_kernel<urb::kFmtMXFP8><<<1, 64, 0, (hipStream_t)stream>>>(a, as, b, bs, C);
  else
    return 7;
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
// Diagnostics: BF16 bits of code[i] * E8M0 scale[i] via the scaled conversion instructions.
int urb_probe_cvt_bf16(int fmt, const void* codes, const void* scales, int n, void* out,
                       void* stream) {
  cvt_bf16_kernel<<<(n + 255) / 256, 256, 0, (hipStream_t)stream>>>(
      fmt, (const uint8_t*)codes, (const uint8_t*)scales, n, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

// Diagnostics: the activation hi/lo BF16 split (hi = bf16(x), lo = bf16(x - hi)) of n floats
// (n even); hi and lo receive n BF16 values each.
int urb_probe_split_bf16(const float* x, int n, void* hi, void* lo, void* stream) {
  if (n <= 0 || n % 2) return 7;
  const int pairs = n / 2;
  split_bf16_kernel<<<(pairs + 255) / 256, 256, 0, (hipStream_t)stream>>>(
      x, pairs, (uint32_t*)hi, (uint32_t*)lo);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // extern "C"
