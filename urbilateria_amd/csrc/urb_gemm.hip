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


// NP panels per wave (the workgroup covers 4 NP panels = 64 NP weight rows): every staged
// activation fragment feeds NP (x2 for gate+up) MFMAs.  MT tokens per tile (32 or 64; 64 for
// large dense batches, so each weight byte feeds twice the MFMAs before it is re-read).
template <int FMT, bool PAIR, int DEPTH, int NP, int MT>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const ExpertMats* __restrict__ mats,
                                                      Perm perm, int rows, int K,
                                                      const float* __restrict__ in,
                                                      float* __restrict__ out, Epi epi,
                                                      int* status) {
  constexpr int RG = MT / 32;       // staging rows per thread
  constexpr int MBMAX = MT / 16;    // 16-token MFMA blocks per tile
  __shared__ __attribute__((aligned(16))) u16 a_hi[2][MT * kALd];
  __shared__ __attribute__((aligned(16))) u16 a_lo[2][MT * kALd];

  // ---- which tile
  const int w = blockIdx.y;
  int expert, base, count, m0;
  if (perm.dense_tokens > 0) {
    expert = 0;
    base = 0;
    count = perm.dense_tokens;
    m0 = w * MT;
    if (m0 >= count) return;
  } else {
    if (w >= perm.meta[1]) return;
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lq = lane >> 4;
  const int panel0 = (blockIdx.x * 4 + wave) * NP;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(K);
  const size_t pscales = (size_t)kPanelRows * (K / 32);

  const uint8_t* pd0 = m.data[PAIR ? 0 : 2] + panel0 * pbytes + 16 * lane;
  const uint8_t* ps0 = FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + panel0 * pscales + lane;
  const uint8_t* pd1 = PAIR ? m.data[1] + panel0 * pbytes + 16 * lane : nullptr;
  const uint8_t* ps1 = (PAIR && FMT != kFmtBF16) ? m.scales[1] + panel0 * pscales + lane : nullptr;

  // ---- A source rows of this thread's staging slots: rows am + 32 g
  const int am = threadIdx.x >> 3;
  bool a_valid[RG];
  const float* a_src[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int r = am + 32 * g;
    a_valid[g] = r < mrows;
    a_src[g] = in;
    if (a_valid[g]) {
      const int p = base + m0 + r;
      const int src_row = PAIR ? (perm.dense_tokens > 0 ? p : perm.perm_token[p]) : p;
      a_src[g] = in + (size_t)src_row * K;
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
  auto body = [&](auto nmb, auto streamed) {
    constexpr int NMB = decltype(nmb)::value;  // 16-token MFMA blocks this tile needs
    constexpr bool STREAM = decltype(streamed)::value;
    BRaw<FMT> r0[DEPTH][NP], r1[DEPTH][NP];
    auto fetch = [&](int d, int s) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        load_b<FMT, STREAM>(r0[d][q], pd0 + q * pbytes, ps0 + q * pscales, s);
        if constexpr (PAIR) load_b<FMT, STREAM>(r1[d][q], pd1 + q * pbytes, ps1 + q * pscales, s);
      }
    };
    auto stage = [&](AStage (&as)[RG], int buf) {
      bool any = false;
#pragma unroll
      for (int g = 0; g < RG; ++g) any |= store_a(as[g], a_hi[buf], a_lo[buf], am + 32 * g);
      return any;
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (d < steps) fetch(d, d);
    AStage as[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) load_a(as[g], a_src[g], a_valid[g], 0);
    bool lo_any = __syncthreads_or(stage(as, 0));
    for (int s0 = 0; s0 < steps; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int s = s0 + d;
        if (s >= steps) break;
        const int buf = s & 1;
        const bool more = s + 1 < steps;
        if (more) {
#pragma unroll
          for (int g = 0; g < RG; ++g) load_a(as[g], a_src[g], a_valid[g], (s + 1) * kKS);
        }
        BRaw<FMT> c0[NP], c1[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          c0[q] = r0[d][q];
          if constexpr (PAIR) c1[q] = r1[d][q];
        }
        if (s + DEPTH < steps) fetch(d, s + DEPTH);  // refill this ring slot DEPTH steps ahead
        const u16* hi = a_hi[buf];
        const u16* lo = a_lo[buf];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 f0[NP], f1[NP];
#pragma unroll
          for (int q = 0; q < NP; ++q) {
            f0[q] = decode_b<FMT>(c0[q], j);
            if constexpr (PAIR) f1[q] = decode_b<FMT>(c1[q], j);
          }
          const int kf = frag_k<FMT>(j, lq);
#pragma unroll
          for (int mb = 0; mb < NMB; ++mb) {
            const bf16x8 ah = lds_frag(hi, mb * 16 + ln, kf);
#pragma unroll
            for (int q = 0; q < NP; ++q) {
              acc0[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, f0[q], acc0[q][mb], 0, 0, 0);
              if constexpr (PAIR)
                acc1[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, f1[q], acc1[q][mb], 0, 0, 0);
            }
            if (lo_any) {
              const bf16x8 al = lds_frag(lo, mb * 16 + ln, kf);
#pragma unroll
              for (int q = 0; q < NP; ++q) {
                acc0[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, f0[q], acc0[q][mb], 0, 0, 0);
                if constexpr (PAIR)
                  acc1[q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, f1[q], acc1[q][mb], 0, 0, 0);
              }
            }
          }
        }
        if (more) lo_any = __syncthreads_or(stage(as, buf ^ 1));
      }
    }
  };
  using Stream = std::true_type;
  using Cached = std::false_type;
  if constexpr (MT == 64) {
    if (mrows > 32) body(Int<4>{}, Cached{});
    else if (mrows > 16) body(Int<2>{}, Cached{});
    else body(Int<1>{}, Cached{});
  } else if (stream) {
    if (mrows > 16) body(Int<2>{}, Stream{});
    else body(Int<1>{}, Stream{});
  } else {
    if (mrows > 16) body(Int<2>{}, Cached{});
    else body(Int<1>{}, Cached{});
  }

  // ---- epilogue: lane holds column `row` of panel q, rows 4*lq + i of each 16-row block
  bool bad = false;
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
        if constexpr (PAIR)
          out[p * rows + row] = epi_gate_up(epi, acc0[q][mb][i], acc1[q][mb][i], bad);
        else
          out[p * rows + row] = epi_down<FMT>(epi, acc0[q][mb][i], bad);
      }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
}

template <int FMT, bool PAIR, int DEPTH, int NP, int MT = kMT>
static void launch_shape(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                         const float* in, float* out, Epi epi, int* status, hipStream_t s) {
  dim3 grid(rows / (kNT * NP), max_tiles);
  gemm_kernel<FMT, PAIR, DEPTH, NP, MT><<<grid, 256, 0, s>>>(mats, perm, rows, K, in, out, epi,
                                                              status);
}

// Weight steps in flight per wave (DEPTH) and panels per wave (NP), per format.  BF16 steps are
// 4 KiB per panel, so one panel one step deep; the MX formats stream 1-2 KiB per panel and
// step and need more panels per staged activation tile (activations are 2-4x their bytes).
// Rows are multiples of 128 (urb_moe_create), so NP = 2 always tiles them.
template <int FMT, bool PAIR>
static void launch(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                   const float* in, float* out, Epi epi, int* status, hipStream_t s) {
  if constexpr (FMT == kFmtBF16)
    launch_shape<FMT, PAIR, 1, 1>(mats, perm, max_tiles, rows, K, in, out, epi, status, s);
  else if constexpr (FMT == kFmtMXFP8)
    launch_shape<FMT, PAIR, 1, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status, s);
  else if (rows % (kNT * 4) == 0)
    launch_shape<FMT, PAIR, 1, 4>(mats, perm, max_tiles, rows, K, in, out, epi, status, s);
  else
    launch_shape<FMT, PAIR, 2, 2>(mats, perm, max_tiles, rows, K, in, out, epi, status, s);
}

void launch_gemm_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                         int I, const float* x, float* act, Epi epi, int* status,
                         hipStream_t s) {
  if (fmt == kFmtBF16) launch<kFmtBF16, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s);
  else if (fmt == kFmtMXFP4) launch<kFmtMXFP4, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s);
  else launch<kFmtMXFP8, true>(mats, perm, max_tiles, I, H, x, act, epi, status, s);
}

void launch_gemm_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                      int I, const float* act, float* y, Epi epi, int* status, hipStream_t s) {
  if (fmt == kFmtBF16) launch<kFmtBF16, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s);
  else if (fmt == kFmtMXFP4) launch<kFmtMXFP4, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s);
  else launch<kFmtMXFP8, false>(mats, perm, max_tiles, H, I, act, y, epi, status, s);
}

}  // namespace urb
