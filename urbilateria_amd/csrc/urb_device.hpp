// urb_device.hpp -- device helpers shared by the MoE kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace urb {

constexpr int kWave = 64;

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Loads through pointers that were themselves read from memory (the per-expert matrix table)
// are generic (flat) to the compiler; flat loads also count against the LDS wait counter, so a
// wait for an LDS read would drain every weight load in flight.  These name the global address
// space explicitly.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16(const void* p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
// Non-temporal form for data read once (streamed expert weights): the load does not keep its
// lines in the caches, so they do not evict what is reused.
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
  const u32x4_t v =
      __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 u2f4(uint4 u) {
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                     __uint_as_float(u.w));
}
// Non-temporal store of 16 bytes (outputs no kernel of the same call reads back soon).
__device__ __forceinline__ void stg16_stream(void* p, float4 v) {
  const u32x4_t u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                     __float_as_uint(v.w)};
  __builtin_nontemporal_store(u, (__attribute__((address_space(1))) u32x4_t*)p);
}
__device__ __forceinline__ uint32_t ldg_u8(const void* p) {
  return *(const __attribute__((address_space(1))) uint8_t*)p;
}
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// BF16 (little-endian u16) -> f32: the high half of the f32 bit pattern
// (src/model/bf16.rs:478-482).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return u2f(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return u2f(pair & 0xffff0000u); }

// E8M0 -> f32: the byte is the biased f32 exponent; code 0 is 2^-127 (subnormal 0x00400000)
// (src/math/mxfp.rs:53-57).
__device__ __forceinline__ float e8m0_to_f32(uint32_t code) {
  uint32_t b = code << 23;
  return u2f(b ? b : 0x00400000u);
}

// Round-to-nearest-even to BF16, false on non-finite input or output
// (src/models/qwen3_8/math.rs:66-78).
__device__ __forceinline__ bool rne_bf16(float v, float* out) {
  uint32_t b = f2u(v);
  if ((b & 0x7f800000u) == 0x7f800000u) return false;
  uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
  if ((r & 0x7f800000u) == 0x7f800000u) return false;
  *out = u2f(r);
  return true;
}

__device__ __forceinline__ bool finite(float v) { return (f2u(v) & 0x7f800000u) != 0x7f800000u; }

// f32::total_cmp ordering key.
__device__ __forceinline__ int32_t total_key(float v) {
  int32_t b = (int32_t)f2u(v);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// exp in f32 evaluated through the f64 exponential, so the f32 result is the correctly rounded
// value except in vanishingly rare double-rounding cases.
__device__ __forceinline__ float exp_f32(float x) { return (float)exp((double)x); }

// silu(v) = v / (1 + exp(-v)) (src/math/ops.rs:36-38).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + exp_f32(-v)); }

__device__ __forceinline__ void flag(int* status, int bits) { atomicOr(status, bits); }

// Qwen3.6's shared-expert scale (finish_ordered_moe, src/models/qwen3_6/runtime.rs:1436-1448):
// sigmoid of the gate logit in the two-branch form, rounded to BF16; `bad` on a non-finite gate
// or scale.
__device__ __forceinline__ float qwen_shared_scale(float g, bool& bad) {
  if (!finite(g)) {
    bad = true;
    return 0.0f;
  }
  float s;
  if (g >= 0.0f) {
    s = 1.0f / (1.0f + exp_f32(-g));
  } else {
    const float e = exp_f32(g);
    s = e / (1.0f + e);
  }
  float r;
  if (!rne_bf16(s, &r)) {
    bad = true;
    return s;
  }
  return r;
}

// Wave64 reductions through cross-lane shuffles.
__device__ __forceinline__ float wave_sum_f32(float v, int width = kWave) {
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v, int width = kWave) {
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
  return v;
}

// --- packed-format decoders (CDNA4 conversion instructions, scale argument 1.0) ---
// E2M1: byte `sel` of `w` holds two codes, low nibble first (src/math/mxfp.rs:1861-1866).
template <int SEL>
__device__ __forceinline__ f32x2 fp4x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, SEL);
}
// E4M3FN: 16-bit half `HI` of `w` holds two codes, low byte first.
template <bool HI>
__device__ __forceinline__ f32x2 fp8x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, HI);
}

// Decodes 8 E2M1 codes of one 32-bit word into v[0..7] (element order = column order).
__device__ __forceinline__ void decode_fp4x8(uint32_t w, float* v) {
  f32x2 a = fp4x2<0>(w), b = fp4x2<1>(w), c = fp4x2<2>(w), d = fp4x2<3>(w);
  v[0] = a[0]; v[1] = a[1]; v[2] = b[0]; v[3] = b[1];
  v[4] = c[0]; v[5] = c[1]; v[6] = d[0]; v[7] = d[1];
}
// Decodes 4 E4M3FN codes of one 32-bit word into v[0..3].
__device__ __forceinline__ void decode_fp8x4(uint32_t w, float* v) {
  f32x2 a = fp8x2<false>(w), b = fp8x2<true>(w);
  v[0] = a[0]; v[1] = a[1]; v[2] = b[0]; v[3] = b[1];
}

}  // namespace urb
