// urb_gemm.hip -- grouped expert GEMMs on CDNA4 MFMA (prefill and batched decode).
//
// For each tile of up to kGemmMTile tokens routed to one expert (the permutation's row tiles)
// and each group of four 16-row weight panels of that expert's matrix, a 256-thread workgroup
// computes C[tokens, rows] = A[tokens, K] . W[rows, K]^T with v_mfma_f32_16x16x32_bf16:
//
//  * B (weights) streams from HBM straight into registers in the panel layout
//    (urb_kernels.hpp): wave w sweeps panel 4 x + w front to back, one 1 KiB slab per load
//    instruction, DEPTH K steps ahead of the MFMAs.  Lane l = ln + 16 lq holds row ln; for
//    BF16 its 16 B are MFMA j's operand directly (k = 32 j + 8 lq), for the MX formats they
//    are one whole 32-column block (k = 32 lq + [0, 32)), decoded in registers with the scaled
//    CDNA4 conversions (v_cvt_scalef32_pk_bf16_fp4/fp8, exact: E2M1 or E4M3 times 2^k is a
//    BF16 value) into the operands of four MFMAs (MFMA j takes k = 32 lq + 8 j + [0, 8)).
//  * A (activations, f32) is gathered through the permutation, split into hi + lo BF16 halves
//    (hi = bf16(a), lo = bf16(a - hi): the product keeps 16 significant bits of a) and staged
//    in LDS one K step ahead; the lo MFMAs are skipped for a K step whose lo half is all zero
//    (BF16-valued activations), and the second 16-token MFMA block for tiles of <= 16 tokens.
//  * Accumulation is f32 in the MFMA; the epilogue is the same as the decode kernels'.
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {


// Activation staging of one workgroup in LDS: hi and lo BF16 halves of MT token rows, double
// buffered, plus the per-wave lo-half flags of each buffer.
template <int MT>
struct GemmLds {
  u16 a_hi[2][MT * kALd];
  u16 a_lo[2][MT * kALd];
  int lo_flag[2][4];
  int rexp[MT];  // row exponents: the f16 down's scales, the gate/up's row maxima
};

// One workgroup's tile: `w` (a row tile of the permutation, or dense tile w) times panel group
// `group` of the weight rows.  NP panels per wave (the workgroup covers 4 NP panels = 64 NP
// weight rows): every staged activation fragment feeds NP (x2 for gate+up) MFMAs.  MT tokens per
// tile: 32 in every launch.  (The template also builds 64-token tiles, each weight byte feeding
// twice the MFMAs before it is re-read; with the panels per wave halved to fit the registers they
// measured slower, on dense batches and on the hot experts of a Zipf-routed 1024-token batch
// alike.)  F16 (the down projection of a batch with epi.rowexp): the rows are staged in
// f16 with their power-of-two scales and the MFMAs take f16 operands (see Epi).
template <int FMT, bool PAIR, int DEPTH, int NP, int MT, int AD, bool F16 = false>
__device__ __forceinline__ void gemm_tile(const ExpertMats* __restrict__ mats, const Perm& perm,
                                          int w, int group, int rows, int K,
                                          const float* __restrict__ in, float* __restrict__ out,
                                          const Epi& epi, int* status, GemmLds<MT>& lds) {
  constexpr int RG = MT / 32;       // staging rows per thread
  constexpr int MBMAX = MT / 16;    // 16-token MFMA blocks per tile
  auto& a_hi = lds.a_hi;
  auto& a_lo = lds.a_lo;
  auto& lo_flag = lds.lo_flag;
  int expert, base, count, m0;
  if (perm.dense_tokens > 0) {
    expert = 0;
    base = 0;
    count = perm.dense_tokens;
    m0 = w * MT;
  } else {
    expert = perm.tiles[2 * w];
    m0 = perm.tiles[2 * w + 1];
    base = perm.offsets[expert];
    count = perm.counts[expert];
  }
  const int mrows = min(MT, count - m0);
  // An expert whose tokens fit one tile has its weights read by this tile only: stream them
  // (non-temporal loads).  A hot expert's tiles instead share its lines through the caches.
  const bool stream = count <= MT;
  const ExpertMats m = mats[expert];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lq = lane >> 4;
  const int panel0 = (group * 4 + wave) * NP;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(K);
  const size_t pscales = (size_t)kPanelRows * (K / 32);

  // wavefront-uniform panel bases; the lane's unit is at 16 lane (data), lane (scales)
  const uint8_t* pd0 = m.data[PAIR ? 0 : 2] + panel0 * pbytes;
  const uint8_t* ps0 = FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + panel0 * pscales;
  const uint8_t* pd1 = PAIR ? m.data[1] + panel0 * pbytes : nullptr;
  const uint8_t* ps1 = (PAIR && FMT != kFmtBF16) ? m.scales[1] + panel0 * pscales : nullptr;
  const uint32_t doff = 16u * lane, soff = lane;

  // ---- A source rows of this thread's staging slots: rows am + 32 g.  A slot past the tile's
  // last row stages the tile's first row instead: its products land in accumulator rows the
  // epilogue never stores, and the loads need no mask.
  const int am = threadIdx.x >> 3;
  const float* a_src[RG];
  const u16* a16[RG];  // F16: the rows as f16 (the gate/up epilogue's output)
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int r = am + 32 * g < mrows ? am + 32 * g : 0;
    const int p = base + m0 + r;
    const int src_row = PAIR ? (perm.dense_tokens > 0 ? p : perm.perm_token[p]) : p;
    a_src[g] = in + (size_t)src_row * K;
    // F16: the f16 rows; gate/up: the router's BF16 copy of the token rows (Epi::xb)
    const u16* abase = F16 ? reinterpret_cast<const u16*>(in) : epi.xb;
    a16[g] = abase ? abase + (size_t)src_row * K : nullptr;
  }
  // F16: each staged row's largest exponent field over the gate/up panel groups (rowexp); the
  // row is staged times 2^(141 - that), which takes its largest |value| into [2^14, 2^15).  Its
  // f16 values are stored at the scale of their own group (e of the group instead).
  int a_emax[RG];
  const int* a_gex[RG];
  const int gw = F16 ? K / epi.groups : 1;  // columns per panel group
  if constexpr (F16) {
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const int r = am + 32 * g < mrows ? am + 32 * g : 0;
      a_gex[g] = epi.rowexp + (size_t)(base + m0 + r) * epi.groups;
      int e = 0;
      for (int gg = 0; gg < epi.groups; ++gg) e = max(e, a_gex[g][gg]);
      a_emax[g] = e;
      if ((threadIdx.x & 7) == 0) lds.rexp[am + 32 * g] = 141 - e;
    }
  }

  f32x4 acc0[NP][MBMAX], acc1[NP][MBMAX];
#pragma unroll
  for (int q = 0; q < NP; ++q)
#pragma unroll
    for (int i = 0; i < MBMAX; ++i) {
      acc0[q][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc1[q][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int steps = K / kKS;
  // B registers: a ring of R = DEPTH + 1 step slots, the step loop unrolled R times so that
  // step s computes from slot s % R while slot (s + DEPTH) % R fills (no register copies).
  constexpr int R = DEPTH + 1;
  auto body = [&](auto nmb, auto streamed, auto dynamic_lo) {
    constexpr int NMB = decltype(nmb)::value;  // 16-token MFMA blocks this tile needs
    constexpr bool STREAM = decltype(streamed)::value;
    // DYNLO: the lo halves may be non-zero, checked per K step; otherwise the rows are
    // BF16-valued and only their hi halves are staged and multiplied -- XB: taken from the
    // router's BF16 copy of the rows (Epi::xb) instead of converted from the f32 rows
    constexpr int AMODE = decltype(dynamic_lo)::value;  // 0 hi of f32, 1 hi + lo, 2 BF16 copy
    constexpr bool DYNLO = AMODE == 1, XB = AMODE == 2;
    BRaw<FMT> r0[R][NP], r1[R][NP];
    auto fetch = [&](int slot, int s) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        load_b<FMT, STREAM>(r0[slot][q], pd0 + q * pbytes, doff, ps0 + q * pscales, soff, s);
        if constexpr (PAIR)
          load_b<FMT, STREAM>(r1[slot][q], pd1 + q * pbytes, doff, ps1 + q * pscales, soff, s);
      }
    };
    // Staging rows this tile's MFMA blocks read: NMB 16 of them.  The rest (a tile of <= 16
    // tokens leaves rows 16..31, waves 2 and 3, idle) neither load nor stage.
    auto staged = [&](int g) { return am + 32 * g < NMB * 16; };
    using Stage = std::conditional_t<F16 || XB, AStage16, AStage>;
    auto fill = [&](Stage& a, int g, int k0) {
      if (staged(g)) {
        if constexpr (F16) load_a16(a, a16[g], a_gex[g], gw, k0);
        else if constexpr (XB) load_ab(a, a16[g], k0);
        else load_a(a, a_src[g], true, k0);
      }
    };
    auto stage = [&](Stage (&as)[RG], int buf) {
      bool any = false;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        if (!staged(g)) continue;
        if constexpr (F16) store_a16g<MT>(as[g], a_hi[buf], a_emax[g], am + 32 * g);
        else if constexpr (XB) store_ab<MT>(as[g], a_hi[buf], am + 32 * g);
        else if constexpr (DYNLO) any |= store_a<MT>(as[g], a_hi[buf], a_lo[buf], am + 32 * g);
        else store_a_hi<MT>(as[g], a_hi[buf], am + 32 * g);
      }
      return any;
    };
    // staging then the workgroup barrier; returns whether any lo half of the step is non-zero
    auto publish = [&](Stage (&as)[RG], int buf) {
      if constexpr (DYNLO) return barrier_or4(stage(as, buf), lo_flag[buf]);
      stage(as, buf);
      __syncthreads();
      return false;
    };
    // One K step from ring slot `slot`; the lo-half MFMAs only when some lo half is non-zero.
    // (With DYNLO a uniform runtime branch around each MFMA pair: compiling both variants
    // straight-line spills the MXFP4 four-panel kernel.  Without it the step is one basic block.)
    auto mma = [&](int slot, const u16* hi, const u16* lo, bool with_lo) {
      if constexpr (F16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kf = frag_k<FMT>(j, lq);
          f16x8 ah[NMB], bh[NP];
#pragma unroll
          for (int mb = 0; mb < NMB; ++mb)
            ah[mb] = __builtin_bit_cast(f16x8, lds_frag<MT>(hi, mb * 16 + ln, kf));
#pragma unroll
          for (int q = 0; q < NP; ++q) bh[q] = decode_b16<FMT>(r0[slot][q], j);
#pragma unroll
          for (int q = 0; q < NP; ++q)
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb)
              acc0[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mb], bh[q], acc0[q][mb], 0, 0, 0);
        }
        return;
      }
      const bool LO = DYNLO && with_lo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kf = frag_k<FMT>(j, lq);
        bf16x8 ah[NMB], al[NMB];
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          ah[mb] = lds_frag<MT>(hi, mb * 16 + ln, kf);
          if (LO) al[mb] = lds_frag<MT>(lo, mb * 16 + ln, kf);
        }
        // one panel's operands decoded at a time: few registers live beside the ring
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          const bf16x8 f0 = decode_b<FMT>(r0[slot][q], j);
          bf16x8 f1;
          if constexpr (PAIR) f1 = decode_b<FMT>(r1[slot][q], j);
#pragma unroll
          for (int mb = 0; mb < NMB; ++mb) {
            acc0[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mb], f0, acc0[q][mb], 0, 0, 0);
            if constexpr (PAIR)
              acc1[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mb], f1, acc1[q][mb], 0, 0, 0);
            if (LO) {
              acc0[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[mb], f0, acc0[q][mb], 0, 0, 0);
              if constexpr (PAIR)
                acc1[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[mb], f1, acc1[q][mb], 0, 0, 0);
            }
          }
        }
      }
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (d < steps) fetch(d, d);
    // activations: step t's rows are loaded into ring slot t % AD, AD steps before they are
    // staged in LDS (at the end of step t - 1); the step loop is unrolled lcm(R, AD) times so
    // both rings are indexed by compile-time slots
    constexpr int U = (R % AD == 0) ? R : R * AD;
    Stage as[AD][RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) fill(as[0][g], g, 0);
    bool lo_any = publish(as[0], 0);
    if constexpr (AD > 1) {
#pragma unroll
      for (int e = 1; e <= AD; ++e)
        if (e < steps)
#pragma unroll
          for (int g = 0; g < RG; ++g) fill(as[e % AD][g], g, e * kKS);
    }
    for (int s0 = 0; s0 < steps; s0 += U) {
#pragma unroll
      for (int d = 0; d < U; ++d) {
        const int s = s0 + d;
        if (s >= steps) break;
        const int buf = s & 1;
        const bool more = s + 1 < steps;
        if constexpr (AD == 1) {
          if (more) {
#pragma unroll
            for (int g = 0; g < RG; ++g) fill(as[0][g], g, (s + 1) * kKS);
          }
        }
        // refill the slot step s - 1 used, DEPTH steps ahead
        if (s + DEPTH < steps) fetch((d + DEPTH) % R, s + DEPTH);
        mma(d % R, a_hi[buf], a_lo[buf], lo_any);
        if (more) lo_any = publish(as[(d + 1) % AD], buf ^ 1);
        if constexpr (AD > 1) {
          if (s + 1 + AD < steps)
#pragma unroll
            for (int g = 0; g < RG; ++g)
              fill(as[(d + 1) % AD][g], g, (s + 1 + AD) * kKS);
        }
      }
    }
  };
  using Stream = std::true_type;
  using Cached = std::false_type;
  auto run = [&](auto dyn) {
    if constexpr (MT == 64) {
      if (mrows > 32) body(Int<4>{}, Cached{}, dyn);
      else if (mrows > 16) body(Int<2>{}, Cached{}, dyn);
      else body(Int<1>{}, Cached{}, dyn);
    } else if (stream) {
      if (mrows > 16) body(Int<2>{}, Stream{}, dyn);
      else body(Int<1>{}, Stream{}, dyn);
    } else {
      if (mrows > 16) body(Int<2>{}, Cached{}, dyn);
      else body(Int<1>{}, Cached{}, dyn);
    }
  };
  // BF16-valued rows (Epi::no_lo, or no lo half seen by this call's router, Epi::lo_word),
  // from the router's BF16 copy where there is one
  if constexpr (F16) {
    run(std::false_type{});
  } else if (epi.no_lo || (epi.lo_word && *epi.lo_word != epi.lo_gen)) {
    if constexpr (PAIR) {
      if (epi.xb) run(Int<2>{});
      else run(std::false_type{});
    } else {
      run(std::false_type{});
    }
  } else {
    run(std::true_type{});
  }

  // ---- epilogue: lane holds column `row` of panel q, rows 4*lq + i of each 16-row block
  bool bad = false;
  // gate/up with rowexp (the input of an f16 down projection): the largest exponent field e of
  // each token row's activations in this panel group first, then the activations as f16 times
  // 2^(141 - e) (the group's largest |value| in [2^14, 2^15)); the down projection rescales
  // each group to its row's largest e as it stages the row
  const bool rowmax = PAIR && epi.rowexp != nullptr;
  int ex[MBMAX][4];
#pragma unroll
  for (int mb = 0; mb < MBMAX; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) ex[mb][i] = 0;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int row = (panel0 + q) * kPanelRows + ln;
#pragma unroll
    for (int mb = 0; mb < MBMAX; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mm = mb * 16 + 4 * lq + i;
        if (mm >= mrows) continue;
        const size_t p = (size_t)(base + m0 + mm);
        if constexpr (PAIR) {
          const float a = epi_gate_up(epi, acc0[q][mb][i], acc1[q][mb][i], bad);
          if (rowmax) {
            acc0[q][mb][i] = a;
            ex[mb][i] = max(ex[mb][i], (int)((__float_as_uint(a) >> 23) & 0xffu));
          } else {
            out[p * rows + row] = a;
          }
        } else {
          const float v =
              F16 ? epi_down<FMT>(epi, ldexpf(acc0[q][mb][i], -lds.rexp[mm] - epi.wshift), bad)
                  : epi_down<FMT>(epi, acc0[q][mb][i], bad);
          if (epi.stream_out) __builtin_nontemporal_store(v, &out[p * rows + row]);
          else out[p * rows + row] = v;
        }
      }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
  if (rowmax) {
    // over the 16 lanes of each k-quad (the rows ln), then the four waves through LDS
#pragma unroll
    for (int mb = 0; mb < MBMAX; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int x = 1; x < 16; x <<= 1) ex[mb][i] = max(ex[mb][i], __shfl_xor(ex[mb][i], x));
    if (threadIdx.x < MT) lds.rexp[threadIdx.x] = 0;
    __syncthreads();
    if (ln == 0) {
#pragma unroll
      for (int mb = 0; mb < MBMAX; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) atomicMax(&lds.rexp[mb * 16 + 4 * lq + i], ex[mb][i]);
    }
    __syncthreads();
    u16* out16 = reinterpret_cast<u16*>(out);
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int row = (panel0 + q) * kPanelRows + ln;
#pragma unroll
      for (int mb = 0; mb < MBMAX; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mm = mb * 16 + 4 * lq + i;
          if (mm >= mrows) continue;
          const _Float16 h = (_Float16)ldexpf(acc0[q][mb][i], 141 - lds.rexp[mm]);
          out16[(size_t)(base + m0 + mm) * rows + row] = __builtin_bit_cast(u16, h);
        }
    }
    if ((int)threadIdx.x < mrows)
      epi.rowexp[(size_t)(base + m0 + threadIdx.x) * epi.groups + group] = lds.rexp[threadIdx.x];
  }
}

// Workgroups per CU a shape is compiled for: two (up to 256 VGPRs), three (168 VGPRs) for the
// MX gate/up pairs: MXFP4 with two panels per wave, two weight steps in flight and the rows
// gathered two ahead; MXFP8 with two panels, one step, rows one ahead.
template <int FMT, bool PAIR, int DEPTH, int NP, int AD>
constexpr int gemm_blocks_per_cu() {
  if (FMT == kFmtMXFP4 && PAIR && DEPTH == 2 && NP == 2 && AD == 2) return 3;
  if (FMT == kFmtMXFP8 && PAIR && DEPTH == 1 && NP == 2 && AD == 1) return 3;
  return 2;
}

// Placement: gemm_place (urb_kernels.hpp); xsplit > 1 only for a dense batch (one expert).
template <int FMT, bool PAIR, int DEPTH, int NP, int MT, int AD = 1, bool F16 = false>
__global__ __launch_bounds__(256, (gemm_blocks_per_cu<FMT, PAIR, DEPTH, NP, AD>())) void
gemm_kernel(const ExpertMats* __restrict__ mats, Perm perm, int max_tiles, int xsplit, int rows,
            int K, const float* __restrict__ in, float* __restrict__ out, Epi epi, int* status,
            int block0) {
  __shared__ __attribute__((aligned(16))) GemmLds<MT> lds;
  const int groups = rows / (kNT * NP);
  const int ntiles = min(perm.dense_tokens > 0 ? (perm.dense_tokens + MT - 1) / MT : perm.meta[1],
                         max_tiles);
  int w, group;
  if (!gemm_place(block0 + blockIdx.x, ntiles, groups, xsplit, &w, &group)) return;
  gemm_tile<FMT, PAIR, DEPTH, NP, MT, AD, F16>(mats, perm, w, group, rows, K, in, out, epi,
                                               status, lds);
}

int gemm_xsplit(int dense_tokens, int ntiles, int groups, double wbytes, double abytes) {
  if (dense_tokens <= 0 || ntiles <= 0) return 1;
  int best = 1;
  double best_time = 0.0;
  for (int x = 1; x <= 8 && x <= groups; x *= 2) {
    const int runs = std::min(8 / x, ntiles);  // non-empty tile runs
    const double bytes = runs * wbytes + x * abytes;
    const double time = bytes / (x * runs);   // per busy XCD
    if (x == 1 || time < best_time) best = x, best_time = time;
  }
  return best;
}

template <int FMT, bool PAIR, int NP>
static int xcd_split(const Perm& perm, int max_tiles, int rows, int K) {
  const double wbytes = (PAIR ? 2.0 : 1.0) * rows * (double)panel_row_bytes<FMT>(K);
  const double abytes = (double)std::max(perm.dense_tokens, 0) * K * 4;
  return gemm_xsplit(perm.dense_tokens, max_tiles, rows / (kNT * NP), wbytes, abytes);
}

// Workgroups per XCD (32 CUs) of one launch of a dense batch: one per CU.
constexpr int kDenseBlocksPerXcd = 32;

template <int FMT, bool PAIR, int DEPTH, int NP, int MT = kMT, int AD = 1, bool F16 = false>
static void launch_shape(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                         const float* in, float* out, Epi epi, int* status, hipStream_t s,
                         bool beside) {
  const int xsplit = xcd_split<FMT, PAIR, NP>(perm, max_tiles, rows, K);
  const int per_xcd = gemm_blocks_per_xcd(max_tiles, rows / (kNT * NP), xsplit);
  // A dense batch beside the routing kernels (the shared expert on the side stream) runs as
  // launches of at most one workgroup per CU, so those kernels keep the other slots; a launch
  // of B workgroups takes placement slots block0 .. block0 + B - 1 (B a multiple of 8, so a
  // slot keeps its XCD).
  const int step = beside && perm.dense_tokens > 0 ? kDenseBlocksPerXcd : per_xcd;
  for (int b0 = 0; b0 < per_xcd; b0 += step)
    gemm_kernel<FMT, PAIR, DEPTH, NP, MT, AD, F16><<<dim3(8 * std::min(step, per_xcd - b0)), 256,
                                                     0, s>>>(mats, perm, max_tiles, xsplit, rows,
                                                             K, in, out, epi, status, 8 * b0);
}

// Weight steps in flight per wave (DEPTH) and panels per wave (NP), per format.  BF16 steps are
// 4 KiB per panel, so one panel one step deep; the MX formats stream 1-2 KiB per panel and
// step and need more panels per staged activation tile (activations are 2-4x their bytes).
// Rows are multiples of 128 (urb_moe_create), so NP = 2 always tiles them.
template <int FMT, bool PAIR>
static void launch(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                   const float* in, float* out, Epi epi, int* status, hipStream_t s, bool beside) {
  if constexpr (FMT == kFmtBF16) {
    // a dense batch (the shared expert) of more than 64 tokens: two (gate+up) or four (down)
    // panels per wave, each staged activation fragment feeding as many weight panels (a
    // 1024-token batch through a 2048 x 7168 BF16 shared expert, in isolation: gate+up 136-140
    // -> 117-121 us against 64-token tiles, down 120-125 -> 81-84 us against one panel)
    // (BF16 weights take f32 or BF16 rows here; the f16 down projection of a BF16 matrix runs
    // on urb_dense.hip's dense_down_f16_kernel)
    const int np = gemm_panels_per_wave(FMT, rows, PAIR, perm.dense_tokens);
    if constexpr (!PAIR) {
      if (np == 4) {
        launch_shape<FMT, PAIR, 1, 4>(mats, perm, max_tiles, rows, K, in, out, epi, status, s,
                                      beside);
        return;
      }
    }
    if (np == 2)
      launch_shape<FMT, PAIR, 1, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status, s, beside);
    else
      launch_shape<FMT, PAIR, 1, 1>(mats, perm, max_tiles, rows, K, in, out, epi, status, s, beside);
  }
  else if constexpr (FMT == kFmtMXFP8) {
    // down: four panels per wave where the rows allow (512 tokens over 160 experts of 6144 x
    // 2048, in isolation: 449-473 -> 443-447 us against two; four panels for gate+up were 60 %
    // slower)
    if constexpr (!PAIR) {
      if (gemm_panels_per_wave(FMT, rows, PAIR, perm.dense_tokens) == 4) {
        if (epi.rowexp)
          launch_shape<FMT, PAIR, 1, 4, kMT, 1, true>(mats, perm, max_tiles, rows, K, in, out, epi,
                                                      status, s, beside);
        else
          launch_shape<FMT, PAIR, 1, 4>(mats, perm, max_tiles, rows, K, in, out, epi, status, s,
                                        beside);
        return;
      }
    }
    // the gate/up pair runs at three workgroups per CU (512 tokens over 160 experts of 6144 x
    // 2048: 735-736 -> 689 us against two per CU, in one process).
    // activation rows gathered one step ahead: two steps ahead (as the MXFP4 gate+up) was 1 %
    // faster in isolation on f32 token rows (512 tokens over 160 experts of 6144 x 2048: 782-787
    // -> 776-777 us) but 1.5 % slower on BF16-valued rows, which skip the lo-half MFMAs
    // (774-776 -> 786-787 us in the layer call)
    if (!PAIR && epi.rowexp)
      launch_shape<FMT, PAIR, 1, 2, kMT, 1, !PAIR>(mats, perm, max_tiles, rows, K, in, out, epi,
                                                   status, s, beside);
    else
      launch_shape<FMT, PAIR, 1, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status, s,
                                    beside);
  }
  else if constexpr (PAIR) {
    // the gate/up pair: two panels per wave with two weight steps in flight and the activation
    // rows gathered two steps ahead, at three workgroups per CU (1024 tokens, top-8 over 384
    // experts of 7168 x 2048, Zipf-routed: 1,207-1,210 against 1,224 us for four panels one
    // step deep at two per CU; gathering two steps ahead took that shape 1417 -> 1253 us)
    launch_shape<FMT, PAIR, 2, 2, kMT, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status,
                                          s, beside);
  } else {
    const int np = gemm_panels_per_wave(FMT, rows, PAIR, perm.dense_tokens);
    // the down projection: four panels per wave where the rows allow, four workgroups per CU
    // on the f16 rows (127 VGPRs; 1024 tokens, top-8 over 384 experts of 7168 x 2048: 690
    // against 713-716 us for eight panels at two per CU, in one process)
    if (np == 4 && epi.rowexp)
      launch_shape<FMT, PAIR, 1, 4, kMT, 1, true>(mats, perm, max_tiles, rows, K, in, out, epi,
                                                  status, s, beside);
    else if (np == 4)
      launch_shape<FMT, PAIR, 1, 4>(mats, perm, max_tiles, rows, K, in, out, epi, status, s,
                                    beside);
    else if (epi.rowexp)
      launch_shape<FMT, PAIR, 2, 2, kMT, 1, true>(mats, perm, max_tiles, rows, K, in, out, epi,
                                                  status, s, beside);
    else
      launch_shape<FMT, PAIR, 2, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status, s,
                                    beside);
  }
}

int gemm_panels_per_wave(int fmt, int rows, bool pair, int dense_tokens) {
  if (fmt == kFmtBF16) {
    if (dense_tokens <= 64) return 1;
    return !pair && rows % (kNT * 4) == 0 ? 4 : 2;
  }
  if (fmt == kFmtMXFP8) return !pair && rows % (kNT * 4) == 0 ? 4 : 2;
  if (pair) return 2;
  return rows % (kNT * 4) == 0 ? 4 : 2;
}

int gemm_placement(int fmt, bool pair, int dense_tokens, int max_tiles, int rows, int K,
                   int32_t* tile_of_block, int32_t* group_of_block, int capacity) {
  const int np = gemm_panels_per_wave(fmt, rows, pair, dense_tokens);
  const int groups = rows / (kNT * np);
  const double rb = fmt == kFmtBF16 ? 2.0 * K : fmt == kFmtMXFP4 ? K / 2.0 : (double)K;
  const int xsplit = gemm_xsplit(dense_tokens, max_tiles, groups, (pair ? 2.0 : 1.0) * rows * rb,
                                 (double)dense_tokens * K * 4);
  const int blocks = 8 * gemm_blocks_per_xcd(max_tiles, groups, xsplit);
  for (int b = 0; b < blocks && b < capacity; ++b) {
    int t = -1, g = -1;
    if (!gemm_place(b, max_tiles, groups, xsplit, &t, &g)) t = g = -1;
    tile_of_block[b] = t;
    group_of_block[b] = g;
  }
  return blocks;
}

void launch_gemm_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                         int I, const float* x, float* act, Epi epi, int* status,
                         hipStream_t s, bool beside) {
  if (fmt == kFmtBF16)
    launch<kFmtBF16, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s, beside);
  else if (fmt == kFmtMXFP4)
    launch<kFmtMXFP4, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s, beside);
  else
    launch<kFmtMXFP8, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s, beside);
}

void launch_gemm_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                      int I, const float* act, float* y, Epi epi, int* status, hipStream_t s,
                      bool beside) {
  if (fmt == kFmtBF16)
    launch<kFmtBF16, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s, beside);
  else if (fmt == kFmtMXFP4)
    launch<kFmtMXFP4, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s, beside);
  else
    launch<kFmtMXFP8, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s, beside);
}

}  // namespace urb
