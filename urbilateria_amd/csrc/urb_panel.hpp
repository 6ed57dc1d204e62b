// urb_panel.hpp -- device-side access to panel-layout weights (layout in urb_kernels.hpp).
#pragma once

#include "urb_device.hpp"
#include "urb_kernels.hpp"

namespace urb {

enum { kFmtBF16 = 0, kFmtMXFP4 = 1, kFmtMXFP8 = 2 };

template <int FMT>
__host__ __device__ constexpr size_t panel_row_bytes(size_t K) {
  return FMT == kFmtBF16 ? K * 2 : (FMT == kFmtMXFP4 ? K / 2 : K);
}

// Raw B operands of one lane for one K step.
template <int FMT>
struct BRaw;
template <>
struct BRaw<kFmtBF16> { uint4 q[4]; };
template <>
struct BRaw<kFmtMXFP4> { uint4 q; uint32_t s; };
template <>
struct BRaw<kFmtMXFP8> { uint4 q[2]; uint32_t s; };

// pd = panel data + 16 * lane, ps = panel scales + lane (see the layout in urb_kernels.hpp).
template <int FMT>
__device__ __forceinline__ void load_b(BRaw<FMT>& r, const uint8_t* __restrict__ pd,
                                       const uint8_t* __restrict__ ps, int step) {
  if constexpr (FMT == kFmtBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r.q[j] = ldg16(pd + (size_t)(4 * step + j) * 1024);
  } else if constexpr (FMT == kFmtMXFP4) {
    r.q = ldg16(pd + (size_t)step * 1024);
    r.s = ldg_u8(ps + (size_t)step * 64);
  } else {
    r.q[0] = ldg16(pd + (size_t)(2 * step) * 1024);
    r.q[1] = ldg16(pd + (size_t)(2 * step + 1) * 1024);
    r.s = ldg_u8(ps + (size_t)step * 64);
  }
}

typedef unsigned short u16;

__device__ __forceinline__ u16 bf16_rne_bits(float v) {
  uint32_t b = f2u(v);
  return (u16)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// k offset (within the K step) of MFMA j's operands for lane group lq.
template <int FMT>
__device__ __forceinline__ int frag_k(int j, int lq) {
  return FMT == kFmtBF16 ? 32 * j + 8 * lq : 32 * lq + 8 * j;
}

__device__ __forceinline__ bf16x8 pack8(bf16x2 a, bf16x2 b, bf16x2 c, bf16x2 d) {
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// MFMA j's B operand from the raw step data (j is a compile-time constant after unrolling).
template <int FMT>
__device__ __forceinline__ bf16x8 decode_b(const BRaw<FMT>& r, int j) {
  if constexpr (FMT == kFmtBF16) {
    return __builtin_bit_cast(bf16x8, r.q[j]);
  } else if constexpr (FMT == kFmtMXFP4) {
    const float sc = e8m0_to_f32(r.s);
    const uint32_t w = j == 0 ? r.q.x : j == 1 ? r.q.y : j == 2 ? r.q.z : r.q.w;
    return pack8(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
  } else {
    const float sc = e8m0_to_f32(r.s);
    const uint4 q = r.q[j >> 1];
    const uint32_t w0 = (j & 1) ? q.z : q.x, w1 = (j & 1) ? q.w : q.y;
    return pack8(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, false),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sc, true),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, false),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sc, true));
  }
}

}  // namespace urb
