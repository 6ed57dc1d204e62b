// urb_decode.hpp -- the one-token MFMA GEMV (decode projections) as a device routine, with its
// launch geometry, shared by the decode kernels (urb_decode.hip) and the launch that runs the
// shared expert's gate+up beside the routing (urb_route.hip).
#pragma once

#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {

// The A fragment lane (ln, lq) feeds MFMA j of step s: piece ln % 2 of the unit holding
// k = 128 s + frag_k(j, lq) .. + 8, from a piece vector staged in LDS (16 B per piece).
template <int FMT>
__device__ __forceinline__ bf16x8 lds_piece(const uint4* xs, int s, int j, int lq, int piece) {
  const int u = (kGemmKStep * s + frag_k<FMT>(j, lq)) >> 3;
  return __builtin_bit_cast(bf16x8, xs[2 * u + piece]);
}

// Copies `units` piece units (32 B each) from global memory to LDS, all threads.
__device__ __forceinline__ void stage_pieces(const uint16_t* __restrict__ src, uint4* dst,
                                             int units) {
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  for (int i = threadIdx.x; i < 2 * units; i += blockDim.x) dst[i] = s4[i];
}

// Slot a -> (expert, permuted position) of a one-token call: the ranked ids (perm.direct) or
// the dense expert (the shared expert, table entry 0).
__device__ __forceinline__ bool decode_slot(const Perm& perm, int a, int& expert, int& pos) {
  if (perm.dense_tokens > 0) {
    if (a != 0) return false;
    expert = 0;
    pos = 0;
    return true;
  }
  if (a >= perm.direct_k) return false;
  expert = perm.direct[a];
  pos = a;
  return true;
}

constexpr int kDecodeMaxWaves = 16;

// A workgroup of W waves (blockDim.x / 64) is W / KSPLIT groups of NP consecutive 16-row panels
// times KSPLIT parts of K, for one slot (`by`), workgroup `bx` of the slot's panel
// groups.  xs (LDS): the slot's input pieces, cols / 8 units of 32 B.
// HALF (gate+up, one panel): a group is half a panel pair -- 8 gate rows and the same 8 up rows
// in one 16-column MFMA operand (lanes ln < 8 read the gate panel, ln >= 8 the up panel) -- so
// a matrix of R rows offers R / 8 groups instead of R / 16: twice the workgroups for a dense
// matrix whose R / 16 workgroups would leave half the CUs idle.
template <int FMT, bool PAIR, int NP, int DW, int WMAX, bool HALF = false>
__device__ __forceinline__ void gemv_mfma_body(
    const ExpertMats* __restrict__ mats, const Perm& perm, int rows, int cols, int ksplit,
    const uint16_t* __restrict__ xp, float* __restrict__ out, uint16_t* __restrict__ out_xp,
    Epi epi, int* status, uint4* xs, int bx, int by) {
  static_assert(!HALF || (PAIR && NP == 1), "half panel pairs: gate+up, one panel per wave");
  __shared__ float red[WMAX][NP][16][2];
  int expert, pos;
  if (!decode_slot(perm, by, expert, pos)) return;
  const ExpertMats m = mats[expert];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lq = lane >> 4, piece = ln & 1;
  const int part = wave % ksplit;
  const int groups = (int)(blockDim.x >> 6) / ksplit;  // panel groups per workgroup
  const int group = bx * groups + wave / ksplit;
  const int panel0 = HALF ? group >> 1 : group * NP;
  const int half = HALF ? group & 1 : 0;
  const bool valid = panel0 < rows / kPanelRows;
  const int steps = cols / kGemmKStep;
  const int s_begin = steps * part / ksplit, n = steps * (part + 1) / ksplit - s_begin;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(cols);
  const size_t pscales = (size_t)kPanelRows * (cols / 32);
  const int pv = valid ? panel0 : 0;
  const uint8_t* pd0 = m.data[PAIR ? 0 : 2] + pv * pbytes;
  const uint8_t* ps0 = FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + pv * pscales;
  const uint8_t* pd1 = PAIR ? m.data[1] + pv * pbytes : nullptr;
  const uint8_t* ps1 = (PAIR && FMT != kFmtBF16) ? m.scales[1] + pv * pscales : nullptr;
  // HALF: lane (ln, lq) takes the panel lane holding row 8 half + ln % 8 at k-quad lq, from the
  // gate panel (ln < 8) or the up panel (ln >= 8)
  const int src = HALF ? lq * 16 + half * 8 + (ln & 7) : lane;
  const uint32_t doff = 16u * src, soff = src;
  const uint8_t* pdh = HALF && ln >= 8 ? pd1 : pd0;
  const uint8_t* psh = HALF && ln >= 8 ? ps1 : ps0;

  constexpr int R = DW + 1;
  BRaw<FMT> r0[R][NP], r1[R][NP];
  auto fetch = [&](int slot, int s) {
    if constexpr (HALF) {
      load_b<FMT, true>(r0[slot][0], pdh, doff, psh, soff, s);
      return;
    }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      load_b<FMT, true>(r0[slot][q], pd0 + q * pbytes, doff, ps0 + q * pscales, soff, s);
      if constexpr (PAIR)
        load_b<FMT, true>(r1[slot][q], pd1 + q * pbytes, doff, ps1 + q * pscales, soff, s);
    }
  };
  // the first weight steps go out before the input is staged, so the two latencies overlap;
  // gate/up read the token's input (row 0), down the slot's activation row
  if (valid) {
#pragma unroll
    for (int d = 0; d < DW; ++d)
      if (d < n) fetch(d, s_begin + d);
  }
  stage_pieces(xp + (size_t)(PAIR ? 0 : pos) * (cols / 8) * kPieceUnit, xs, cols / 8);
  __syncthreads();

  f32x4 acc0[NP], acc1[NP];
#pragma unroll
  for (int q = 0; q < NP; ++q) acc0[q] = acc1[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (valid) {
    for (int i0 = 0; i0 < n; i0 += R) {
#pragma unroll
      for (int d = 0; d < R; ++d) {
        const int i = i0 + d;
        if (i >= n) break;
        if (i + DW < n) fetch((d + DW) % R, s_begin + i + DW);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8 a = lds_piece<FMT>(xs, s_begin + i, j, lq, piece);
#pragma unroll
          for (int q = 0; q < NP; ++q) {
            acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, decode_b<FMT>(r0[d][q], j),
                                                              acc0[q], 0, 0, 0);
            if constexpr (PAIR && !HALF)
              acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, decode_b<FMT>(r1[d][q], j),
                                                                acc1[q], 0, 0, 0);
          }
        }
      }
    }
  }
  // lane (ln, 0): rows 0 and 1 are the hi and lo partial sums of weight row ln
  float v0[NP], v1[NP];
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    v0[q] = acc0[q][0] + acc0[q][1];
    v1[q] = acc1[q][0] + acc1[q][1];
  }
  if (ksplit > 1) {
    if (lq == 0)
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        red[wave][q][ln][0] = v0[q];
        red[wave][q][ln][1] = v1[q];
      }
    __syncthreads();
    if (part == 0 && lq == 0)
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        v0[q] = 0.0f;
        v1[q] = 0.0f;
        for (int z = 0; z < ksplit; ++z) {  // K parts in order
          v0[q] += red[wave + z][q][ln][0];
          v1[q] += red[wave + z][q][ln][1];
        }
      }
  }
  if constexpr (HALF) {
    // column ln < 8: gate row 8 half + ln; its up row is column ln + 8
    const float up = __shfl_xor(v0[0], 8);
    if (!valid || part != 0 || lq != 0 || ln >= 8) return;
    bool bad = false;
    const int r = panel0 * kPanelRows + half * 8 + ln;
    const float v = epi_gate_up(epi, v0[0], up, bad);
    if (out) out[(size_t)pos * rows + r] = v;
    if (out_xp) store_piece_value(out_xp + (size_t)pos * (rows / 8) * kPieceUnit, r, v);
    if (bad) flag(status, kStatusNonFinite);
    return;
  }
  if (!valid || part != 0 || lq != 0) return;
  bool bad = false;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int r = (panel0 + q) * kPanelRows + ln;
    const float v = PAIR ? epi_gate_up(epi, v0[q], v1[q], bad) : epi_down<FMT>(epi, v0[q], bad);
    if (out) out[(size_t)pos * rows + r] = v;
    if (out_xp) store_piece_value(out_xp + (size_t)pos * (rows / 8) * kPieceUnit, r, v);
  }
  if (bad) flag(status, kStatusNonFinite);
}

// Weight steps in flight per wave, panels per wave and the largest workgroup (waves).  Measured
// on MI355X (one token, every weight from HBM): two steps in flight beat one, four, six and
// eight; with the input in LDS, a deeper ring only costs occupancy.
template <int FMT, bool PAIR>
constexpr int decode_depth() { return 2; }
template <int FMT, bool PAIR>
constexpr int decode_panels() { return 1; }
template <int FMT, bool PAIR>
constexpr int decode_max_waves() { return PAIR ? 8 : kDecodeMaxWaves; }

// Launch geometry of gemv_mfma_body: K is split until the launch has ~8192 waves, keeping at
// least two steps a part; a workgroup holds max(4, ksplit) waves; grid = (panel-group
// workgroups, slots); LDS = the input pieces.
struct GemvShape {
  int ksplit, waves;
  dim3 grid;
  size_t lds;
};
template <int FMT, bool PAIR>
inline GemvShape gemv_mfma_shape(int rows, int cols, int max_active) {
  constexpr int NP = decode_panels<FMT, PAIR>();
  constexpr int WMAX = decode_max_waves<FMT, PAIR>();
  const int panels = rows / kPanelRows, steps = cols / kGemmKStep;
  int ksplit = 1;
  while (ksplit < WMAX && (long)panels / NP * max_active * ksplit < 8192 &&
         steps / (2 * ksplit) >= 1)
    ksplit *= 2;
  const int waves = std::max(4, ksplit);
  const int per_wg = waves / ksplit * NP;
  return {ksplit, waves, dim3((panels + per_wg - 1) / per_wg, max_active), (size_t)cols / 8 * 32};
}

}  // namespace urb
