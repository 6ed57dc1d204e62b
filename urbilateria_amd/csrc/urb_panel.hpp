// urb_panel.hpp -- device-side access to panel-layout weights (layout in urb_kernels.hpp).
#pragma once

#include "urb_device.hpp"
#include "urb_kernels.hpp"

#include <type_traits>

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
// STREAM: non-temporal weight loads, for weights this launch reads only once.  (A compile-time
// choice: with a runtime one the compiler merges both loads into one and drops the hint.)
template <int FMT, bool STREAM = false>
__device__ __forceinline__ void load_b(BRaw<FMT>& r, const uint8_t* __restrict__ pd,
                                       const uint8_t* __restrict__ ps, int step) {
  auto ld = [](const void* p) { return STREAM ? ldg16_stream(p) : ldg16(p); };
  if constexpr (FMT == kFmtBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r.q[j] = ld(pd + (size_t)(4 * step + j) * 1024);
  } else if constexpr (FMT == kFmtMXFP4) {
    r.q = ld(pd + (size_t)step * 1024);
    r.s = ldg_u8(ps + (size_t)step * 64);
  } else {
    r.q[0] = ld(pd + (size_t)(2 * step) * 1024);
    r.q[1] = ld(pd + (size_t)(2 * step + 1) * 1024);
    r.s = ldg_u8(ps + (size_t)step * 64);
  }
}

// The same from a wavefront-uniform panel base (held in SGPRs) plus 32-bit per-lane offsets
// (doff = 16 * lane, soff = lane): the loads take the scalar-base form of global_load, with no
// 64-bit address arithmetic per lane.
template <int FMT, bool STREAM = false>
__device__ __forceinline__ void load_b(BRaw<FMT>& r, const uint8_t* __restrict__ pbase,
                                       uint32_t doff, const uint8_t* __restrict__ sbase,
                                       uint32_t soff, int step) {
  auto ld = [&](uint32_t o) {
    const uint8_t* p = pbase + o;
    return STREAM ? ldg16_stream(p) : ldg16(p);
  };
  const uint32_t st = (uint32_t)step;
  if constexpr (FMT == kFmtBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r.q[j] = ld(doff + (4 * st + j) * 1024u);
  } else if constexpr (FMT == kFmtMXFP4) {
    r.q = ld(doff + st * 1024u);
    r.s = ldg_u8(sbase + (soff + st * 64u));
  } else {
    r.q[0] = ld(doff + 2 * st * 1024u);
    r.q[1] = ld(doff + (2 * st + 1) * 1024u);
    r.s = ldg_u8(sbase + (soff + st * 64u));
  }
}

typedef unsigned short u16;

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

// MFMA j's B operand as f16 for the MX formats (exact for E8M0 codes within
// [kF16ScaleLo, kF16ScaleHi] of the format; urb_moe_create checks the down projections).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
template <int FMT>
__device__ __forceinline__ f16x8 decode_b16(const BRaw<FMT>& r, int j) {
  static_assert(FMT != kFmtBF16, "BF16 matrices take f16 MFMAs only on the dense kernel");
  {
    const float sc = e8m0_to_f32(r.s);
    uint32_t p[4];
    if constexpr (FMT == kFmtMXFP4) {
      const uint32_t w = j == 0 ? r.q.x : j == 1 ? r.q.y : j == 2 ? r.q.z : r.q.w;
      p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 0));
      p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 1));
      p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 2));
      p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 3));
    } else {
      const uint4 q = r.q[j >> 1];
      const uint32_t w0 = (j & 1) ? q.z : q.x, w1 = (j & 1) ? q.w : q.y;
      p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, sc, false));
      p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, sc, true));
      p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, sc, false));
      p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, sc, true));
    }
    return __builtin_bit_cast(f16x8, make_uint4(p[0], p[1], p[2], p[3]));
  }
}

// ---- projection epilogues (kinds in urb_kernels.hpp) ----
// Gate/up pair -> activation; `bad` is set on a failure the reference reports.
__device__ __forceinline__ float epi_gate_up(const Epi& e, float g0, float u0, bool& bad) {
  if (e.kind == kEpiGated) {
    const float a = silu(g0) * u0;  // a non-finite value fails the down projection's input check
    if (!finite(a)) bad = true;
    return a;
  }
  float g = g0, u = u0;
  bool ok = rne_bf16(g0, &g) && rne_bf16(u0, &u);
  float a;
  if (e.kind == kEpiHy4) {
    const float gl = fminf(g, e.limit);
    const float ul = fminf(fmaxf(u, -e.limit), e.limit);
    a = gl / (1.0f + exp_f32(-gl)) * ul;
  } else {
    float sg = silu(g);
    if (e.kind == kEpiQwen) ok = ok && rne_bf16(sg, &sg);
    const float v = sg * u;
    a = v;
    ok = ok && rne_bf16(v, &a);
    if (!ok) a = v;
  }
  if (!ok) bad = true;
  return a;
}

// Down projection output.
template <int FMT>
__device__ __forceinline__ float epi_down(const Epi& e, float y, bool& bad) {
  if (e.kind == kEpiGated) {
    // MxFp8Matrix::matvec_rows rejects non-finite outputs (src/math/mxfp.rs:779-781)
    if (FMT == kFmtMXFP8 && !finite(y)) bad = true;
    return y;
  }
  float r;
  if (!rne_bf16(y, &r)) {
    bad = true;
    return y;
  }
  return r;
}

// ---- activation staging for the MFMA kernels (A operand through LDS) ----
constexpr int kMT = kGemmMTile;   // 32 tokens: two 16-row MFMA blocks
constexpr int kNT = kGemmNTile;   // 64 weight rows: one 16-row panel per wave
constexpr int kKS = kGemmKStep;   // 128 k per step
constexpr int kALd = kKS;         // bf16 values per staged row: 16 chunks of 8

// LDS layout of MT staged rows: chunk c (8 bf16 at k = 8c, 16 B) of row m sits in the 128 B block
// c * MT/8 + m/8, at position (m ^ h(c)) & 7 of the block, where h swaps bits 1 and 2 of c.
// Measured on MI355X (SQ_LDS_BANK_CONFLICT over 35 lane patterns): 64 banks of 4 B; a 16-byte
// read is served in four passes of 16 lanes, a pass being the lanes with equal lane bit 5 and
// equal parity of lane bits 2-4, and is conflict-free when each pass hits 16 distinct 16 B bank
// slots; a 16-byte store is conflict-free when each 8 consecutive lanes hit 8 distinct positions
// mod 8.  MFMA fragment reads (row m = 16 mb + lane % 16 at chunk 4 (lane / 16) + j, or
// 4 j + lane / 16 for BF16 weights) and staging stores (one row's chunks 0..7 or 8..15 per 8
// lanes) then cost no extra cycles; row-major rows at any padding cost 4 per read.
template <int MT>
__device__ __forceinline__ int a_chunk(int m, int c) {
  const int h = (c & 1) | ((c >> 1) & 2) | ((c << 1) & 4);
  return 8 * ((c * (MT / 8) + (m >> 3)) * 8 + ((m ^ h) & 7));
}

// A staging: thread t covers row t/8 and the k chunks t%8 and 8 + t%8 of the K step (8 values
// each: the eight threads of a row read its first 256 B, then its second).
struct AStage { float4 v[4]; };

__device__ __forceinline__ void load_a(AStage& a, const float* __restrict__ src, bool valid,
                                       int k0) {
  const int c = threadIdx.x & 7;
  if (valid) {
    const float4* p = reinterpret_cast<const float4*>(src + k0);
    a.v[0] = p[2 * c]; a.v[1] = p[2 * c + 1]; a.v[2] = p[16 + 2 * c]; a.v[3] = p[17 + 2 * c];
  } else {
    a.v[0] = a.v[1] = a.v[2] = a.v[3] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Two floats to packed BF16, round to nearest even (v_cvt_pk_bf16_f32; denormals kept).
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2v));
}

// hi/lo BF16 split of two floats: hi = bf16(v), lo = bf16(v - hi) (v - hi is exact), packed
// (element 0 in the low half).
__device__ __forceinline__ void split_bf16(float v0, float v1, uint32_t& hi, uint32_t& lo) {
  hi = pk_bf16(v0, v1);
  lo = pk_bf16(v0 - u2f(hi << 16), v1 - u2f(hi & 0xffff0000u));
}

// Writes hi/lo BF16 halves of the staged values into LDS row m of MT (default: this thread's
// staging row); returns whether any lo half is non-zero.
template <int MT = kMT>
__device__ __forceinline__ bool store_a(const AStage& a, u16* hi, u16* lo,
                                        int m = (int)(threadIdx.x >> 3)) {
  const int c = threadIdx.x & 7;
  const float* v = reinterpret_cast<const float*>(a.v);
  uint32_t h[8], l[8], lor = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    split_bf16(v[2 * i], v[2 * i + 1], h[i], l[i]);
    lor |= l[i];
  }
  const int o0 = a_chunk<MT>(m, c), o1 = a_chunk<MT>(m, 8 + c);
  *reinterpret_cast<uint4*>(hi + o0) = make_uint4(h[0], h[1], h[2], h[3]);
  *reinterpret_cast<uint4*>(hi + o1) = make_uint4(h[4], h[5], h[6], h[7]);
  *reinterpret_cast<uint4*>(lo + o0) = make_uint4(l[0], l[1], l[2], l[3]);
  *reinterpret_cast<uint4*>(lo + o1) = make_uint4(l[4], l[5], l[6], l[7]);
  return (lor & 0x7fff7fffu) != 0;
}

// Writes the BF16 (round to nearest even) of the staged values into LDS row m: the hi halves
// alone, for rows whose values are BF16 already.
template <int MT = kMT>
__device__ __forceinline__ void store_a_hi(const AStage& a, u16* hi,
                                           int m = (int)(threadIdx.x >> 3)) {
  const int c = threadIdx.x & 7;
  const float* v = reinterpret_cast<const float*>(a.v);
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = pk_bf16(v[2 * i], v[2 * i + 1]);
  *reinterpret_cast<uint4*>(hi + a_chunk<MT>(m, c)) = make_uint4(h[0], h[1], h[2], h[3]);
  *reinterpret_cast<uint4*>(hi + a_chunk<MT>(m, 8 + c)) = make_uint4(h[4], h[5], h[6], h[7]);
}

// f16 activation rows (the f16 down projection's input, written by the gate/up epilogue at the
// scale of each row's panel group): thread c of row m loads chunks c and 8 + c of the K step at
// k0, and the exponent field `e` of the group they belong to (`gex` = the row's groups, `gw` =
// columns per group).
struct AStage16 { uint4 v[2]; int e; };
__device__ __forceinline__ void load_a16(AStage16& a, const u16* __restrict__ src,
                                         const int* __restrict__ gex, int gw, int k0) {
  const int c = threadIdx.x & 7;
  a.v[0] = ldg16(src + k0 + 8 * c);
  a.v[1] = ldg16(src + k0 + 64 + 8 * c);
  a.e = gex[k0 / gw];
}
// Stages them at the row's scale: times 2^(e - emax) (<= 1; exact unless the result is
// subnormal in f16, i.e. below 2^-29 of the row's largest value).
template <int MT = kMT>
__device__ __forceinline__ void store_a16g(const AStage16& a, u16* dst, int emax,
                                           int m = (int)(threadIdx.x >> 3)) {
  typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
  const int c = threadIdx.x & 7, d = a.e - emax;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(a.v);
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f16x2v v = __builtin_bit_cast(f16x2v, w[i]);
    v[0] = __builtin_amdgcn_ldexph(v[0], d);
    v[1] = __builtin_amdgcn_ldexph(v[1], d);
    h[i] = __builtin_bit_cast(uint32_t, v);
  }
  *reinterpret_cast<uint4*>(dst + a_chunk<MT>(m, c)) = make_uint4(h[0], h[1], h[2], h[3]);
  *reinterpret_cast<uint4*>(dst + a_chunk<MT>(m, 8 + c)) = make_uint4(h[4], h[5], h[6], h[7]);
}

// BF16 activation rows (Epi::xb): thread c of row m loads chunks c and 8 + c of the K step at
// k0 and stages them as they are -- the BF16-valued rows' hi halves, with no conversion.
__device__ __forceinline__ void load_ab(AStage16& a, const u16* __restrict__ src, int k0) {
  const int c = threadIdx.x & 7;
  a.v[0] = ldg16(src + k0 + 8 * c);
  a.v[1] = ldg16(src + k0 + 64 + 8 * c);
}
template <int MT = kMT>
__device__ __forceinline__ void store_ab(const AStage16& a, u16* dst,
                                         int m = (int)(threadIdx.x >> 3)) {
  const int c = threadIdx.x & 7;
  *reinterpret_cast<uint4*>(dst + a_chunk<MT>(m, c)) = a.v[0];
  *reinterpret_cast<uint4*>(dst + a_chunk<MT>(m, 8 + c)) = a.v[1];
}

// A workgroup barrier that also ORs a per-thread flag over the four waves of a 256-thread
// workgroup, with one s_barrier: each wave's lane 0 writes the wave's OR into its slot before
// the barrier and every wave reads the four slots after it.  (HIP's __syncthreads_or reduces
// through one LDS word with an atomic, three barriers.)  `slots` (4 ints, 16-byte aligned) must
// not be rewritten before the next barrier: double-buffer them with the data they describe.
__device__ __forceinline__ bool barrier_or4(bool pred, int* slots) {
  const bool any = __ballot(pred) != 0;
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = any;
  __syncthreads();
  const int4 v = *reinterpret_cast<const int4*>(slots);
  return (v.x | v.y | v.z | v.w) != 0;
}

// The 8 staged values of row m (of MT) at k (a multiple of 8).
template <int MT = kMT>
__device__ __forceinline__ bf16x8 lds_frag(const u16* base, int m, int k) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + a_chunk<MT>(m, k >> 3)));
}

template <int N>
using Int = std::integral_constant<int, N>;

// ---- BF16 pieces of f32 vectors: the A operand of the decode MFMA GEMVs ----
// An f32 value v is carried as two BF16 values: hi = bf16(v) and lo = bf16(v - hi) (round to
// nearest even; v - hi is exact in f32), so hi + lo keeps 16 significant bits of v, like the
// hi/lo split of the grouped GEMMs' activations.  A vector of K values (K % 8 == 0) is stored
// as K / 8 units of 32 B: unit u = hi and lo of values 8 u .. 8 u + 7, 8 BF16 each.  Lane
// (ln, lq) of an MFMA reads 16 B, piece ln % 2 of one unit, so A row r holds piece r % 2 and C
// rows 0 and 1 are the two pieces' partial sums (rows 2..15 repeat them).

// The two pieces of two values, packed in pairs (value a in the low halves).
__device__ __forceinline__ void split2_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - u2f(hi << 16), b - u2f(hi & 0xffff0000u));
}

// The unit of values v[0..8): 2 x 16 B, pieces in order.
__device__ __forceinline__ void store_piece_unit(const float* v, uint16_t* unit) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split2_pair(v[2 * i], v[2 * i + 1], h[i], l[i]);
  uint4* d = reinterpret_cast<uint4*>(unit);
  d[0] = make_uint4(h[0], h[1], h[2], h[3]);
  d[1] = make_uint4(l[0], l[1], l[2], l[3]);
}

// One value k of a piece vector (scattered 2-byte stores; for epilogues that own one value).
__device__ __forceinline__ void store_piece_value(uint16_t* vec, int k, float v) {
  uint32_t h, l;
  split2_pair(v, 0.0f, h, l);
  uint16_t* u = vec + (size_t)(k >> 3) * kPieceUnit + (k & 7);
  u[0] = (uint16_t)h;
  u[8] = (uint16_t)l;
}

// Units [first, units) step `stride` of the piece vector of x[0..8 units) (f32).
__device__ __forceinline__ void split_vector(const float* __restrict__ x, int units,
                                             uint16_t* __restrict__ out, int first, int stride) {
  for (int u = first; u < units; u += stride) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * u];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * u + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    store_piece_unit(v, out + (size_t)u * kPieceUnit);
  }
}

}  // namespace urb
