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

constexpr int kMT = kGemmMTile;   // 32 tokens: two 16-row MFMA blocks
constexpr int kNT = kGemmNTile;   // 64 weight rows: one 16-row panel per wave
constexpr int kKS = kGemmKStep;   // 128 k per step
constexpr int kALd = kKS + 8;     // LDS row pitch in bf16 (16 B pad against bank conflicts)




// A staging: thread t covers row t/8 and 16 consecutive k at 16*(t%8) of the K step.
struct AStage { float4 v[4]; };

__device__ __forceinline__ void load_a(AStage& a, const float* __restrict__ src, bool valid,
                                       int k0) {
  const int kc = (threadIdx.x & 7) * 16;
  if (valid) {
    const float4* p = reinterpret_cast<const float4*>(src + k0 + kc);
    a.v[0] = p[0]; a.v[1] = p[1]; a.v[2] = p[2]; a.v[3] = p[3];
  } else {
    a.v[0] = a.v[1] = a.v[2] = a.v[3] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Writes hi/lo BF16 halves of the staged values; returns whether any lo half is non-zero.
__device__ __forceinline__ bool store_a(const AStage& a, u16* hi, u16* lo) {
  const int m = threadIdx.x >> 3, kc = (threadIdx.x & 7) * 16;
  const float* v = reinterpret_cast<const float*>(a.v);
  u16 h[16], l[16];
  bool any = false;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    h[i] = bf16_rne_bits(v[i]);
    float rest = v[i] - u2f((uint32_t)h[i] << 16);
    l[i] = bf16_rne_bits(rest);
    any |= (l[i] & 0x7fff) != 0;
  }
  uint4* dh = reinterpret_cast<uint4*>(hi + m * kALd + kc);
  uint4* dl = reinterpret_cast<uint4*>(lo + m * kALd + kc);
  dh[0] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
  dh[1] = make_uint4(h[8] | (h[9] << 16), h[10] | (h[11] << 16), h[12] | (h[13] << 16), h[14] | (h[15] << 16));
  dl[0] = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
  dl[1] = make_uint4(l[8] | (l[9] << 16), l[10] | (l[11] << 16), l[12] | (l[13] << 16), l[14] | (l[15] << 16));
  return any;
}

__device__ __forceinline__ bf16x8 lds_frag(const u16* base, int m, int k) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + m * kALd + k));
}

template <int N>
using Int = std::integral_constant<int, N>;

// NP panels per wave (the workgroup covers 4 NP panels = 64 NP weight rows): every staged
// activation fragment feeds NP (x2 for gate+up) MFMAs.
template <int FMT, bool PAIR, int DEPTH, int NP>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const ExpertMats* __restrict__ mats,
                                                      Perm perm, int rows, int K,
                                                      const float* __restrict__ in,
                                                      float* __restrict__ out, int qwen,
                                                      int* status) {
  __shared__ __attribute__((aligned(16))) u16 a_hi[2][kMT * kALd];
  __shared__ __attribute__((aligned(16))) u16 a_lo[2][kMT * kALd];

  // ---- which tile
  const int w = blockIdx.y;
  int expert, base, count, m0;
  if (perm.dense_tokens > 0) {
    expert = 0;
    base = 0;
    count = perm.dense_tokens;
    m0 = w * kMT;
    if (m0 >= count) return;
  } else {
    if (w >= perm.meta[1]) return;
    expert = perm.tiles[2 * w];
    m0 = perm.tiles[2 * w + 1];
    base = perm.offsets[expert];
    count = perm.counts[expert];
  }
  const int mrows = min(kMT, count - m0);
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

  // ---- A source row of this thread's staging slot
  const int am = threadIdx.x >> 3;
  const bool a_valid = am < mrows;
  const float* a_src = in;
  if (a_valid) {
    const int p = base + m0 + am;
    const int src_row = PAIR ? (perm.dense_tokens > 0 ? p : perm.perm_token[p]) : p;
    a_src = in + (size_t)src_row * K;
  }

  f32x4 acc0[NP][2], acc1[NP][2];
#pragma unroll
  for (int q = 0; q < NP; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      acc0[q][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc1[q][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const int steps = K / kKS;
  auto body = [&](auto nmb) {
    constexpr int NMB = decltype(nmb)::value;  // 16-token MFMA blocks this tile needs
    BRaw<FMT> r0[DEPTH][NP], r1[DEPTH][NP];
    auto fetch = [&](int d, int s) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        load_b<FMT>(r0[d][q], pd0 + q * pbytes, ps0 + q * pscales, s);
        if constexpr (PAIR) load_b<FMT>(r1[d][q], pd1 + q * pbytes, ps1 + q * pscales, s);
      }
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (d < steps) fetch(d, d);
    AStage as;
    load_a(as, a_src, a_valid, 0);
    bool lo_any = __syncthreads_or(store_a(as, a_hi[0], a_lo[0]));
    for (int s0 = 0; s0 < steps; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int s = s0 + d;
        if (s >= steps) break;
        const int buf = s & 1;
        const bool more = s + 1 < steps;
        if (more) load_a(as, a_src, a_valid, (s + 1) * kKS);
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
        if (more) lo_any = __syncthreads_or(store_a(as, a_hi[buf ^ 1], a_lo[buf ^ 1]));
      }
    }
  };
  if (mrows > 16) body(Int<2>{});
  else body(Int<1>{});

  // ---- epilogue: lane holds column `row` of panel q, rows 4*lq + i of each 16-row block
  bool bad = false;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int row = (panel0 + q) * kPanelRows + ln;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mm = mb * 16 + 4 * lq + i;
        if (mm >= mrows) continue;
        const size_t p = (size_t)(base + m0 + mm);
        if constexpr (PAIR) {
          const float g0 = acc0[q][mb][i], u0 = acc1[q][mb][i];
          float act;
          if (qwen) {
            float g, u, ag;
            bool ok = rne_bf16(g0, &g) && rne_bf16(u0, &u) && rne_bf16(silu(g), &ag);
            float v = ag * u;
            ok = ok && rne_bf16(v, &act);
            if (!ok) { bad = true; act = v; }
          } else {
            act = silu(g0) * u0;
            if (!finite(act)) bad = true;
          }
          out[p * rows + row] = act;
        } else {
          float y = acc0[q][mb][i];
          if (qwen) {
            float r;
            if (!rne_bf16(y, &r)) bad = true; else y = r;
          } else if (FMT == kFmtMXFP8 && !finite(y)) {
            bad = true;
          }
          out[p * rows + row] = y;
        }
      }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
}

// ------------------------------------------------------------------------------------------
// Router logits (`router.matvec`, src/model/bf16.rs:121-216, ordered f64) for the GLM
// composition: logits[t, e] = sum_k w[e, k] x[t, k].  BF16 weight times the hi/lo BF16 halves
// of x are exact products; each MFMA sums 32 of them in f32 and that partial is added into an
// f64 accumulator, so the f32 logit is the correctly rounded sum up to a few units in the last
// place.  The router weight is in the panel layout with its rows padded to a multiple of 64
// (zero rows).  Workgroup (x, y, z) covers experts [64 x, 64 x + 64), tokens [32 y, 32 y + 32)
// and K steps [z * slice, (z + 1) * slice) and writes f64 partial sums part[z][t][e]; the
// routing kernel adds the slices in order.
// ------------------------------------------------------------------------------------------
template <int DEPTH>
__global__ __launch_bounds__(256, 2) void router_mfma_kernel(const uint8_t* __restrict__ wp,
                                                             int Epad, int H,
                                                             const float* __restrict__ x,
                                                             int T, int slice,
                                                             double* __restrict__ part,
                                                             int* status) {
  __shared__ __attribute__((aligned(16))) u16 a_hi[2][kMT * kALd];
  __shared__ __attribute__((aligned(16))) u16 a_lo[2][kMT * kALd];
  const int m0 = blockIdx.y * kMT;
  const int mrows = min(kMT, T - m0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lq = lane >> 4;
  const int panel = blockIdx.x * 4 + wave;
  const int steps = H / kKS;
  const int s_begin = blockIdx.z * slice, s_end = min(steps, s_begin + slice);
  const uint8_t* pd = wp + (size_t)panel * (kPanelRows * panel_row_bytes<kFmtBF16>(H)) + 16 * lane;
  const int am = threadIdx.x >> 3;
  const bool a_valid = am < mrows;
  const float* a_src = x + (size_t)(m0 + (a_valid ? am : 0)) * H;

  double acc[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mb][i] = 0.0;

  bool bad = false;
  auto check = [&](const AStage& as) {
    const float* v = reinterpret_cast<const float*>(as.v);
#pragma unroll
    for (int i = 0; i < 16; ++i) bad |= !finite(v[i]);
  };
  auto body = [&](auto nmb) {
    constexpr int NMB = decltype(nmb)::value;
    BRaw<kFmtBF16> r[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (s_begin + d < s_end) load_b<kFmtBF16>(r[d], pd, nullptr, s_begin + d);
    AStage as;
    load_a(as, a_src, a_valid, s_begin * kKS);
    check(as);
    bool lo_any = __syncthreads_or(store_a(as, a_hi[0], a_lo[0]));
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = s_begin; s0 < s_end; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int s = s0 + d;
        if (s >= s_end) break;
        const int buf = (s - s_begin) & 1;
        const bool more = s + 1 < s_end;
        if (more) load_a(as, a_src, a_valid, (s + 1) * kKS);
        const BRaw<kFmtBF16> c = r[d];
        if (s + DEPTH < s_end) load_b<kFmtBF16>(r[d], pd, nullptr, s + DEPTH);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8 f = __builtin_bit_cast(bf16x8, c.q[j]);
          const int kf = frag_k<kFmtBF16>(j, lq);
#pragma unroll
          for (int mb = 0; mb < NMB; ++mb) {
            f32x4 pp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                lds_frag(a_hi[buf], mb * 16 + ln, kf), f, zero, 0, 0, 0);
            if (lo_any)
              pp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  lds_frag(a_lo[buf], mb * 16 + ln, kf), f, pp, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mb][i] += (double)pp[i];
          }
        }
        if (more) {
          check(as);
          lo_any = __syncthreads_or(store_a(as, a_hi[buf ^ 1], a_lo[buf ^ 1]));
        }
      }
    }
  };
  if (mrows > 16) body(Int<2>{});
  else body(Int<1>{});
  if (bad && blockIdx.x == 0) flag(status, kStatusNonFinite);
  const int e = panel * kPanelRows + ln;
  double* out = part + (size_t)blockIdx.z * T * Epad;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = mb * 16 + 4 * lq + i;
      if (mm < mrows) out[(size_t)(m0 + mm) * Epad + e] = acc[mb][i];
    }
}

int router_slices(int E, int H, int T) {
  const int steps = H / kKS;
  const int base = (router_rows(E) / kNT) * ((T + kMT - 1) / kMT);
  int slices = std::min(kRouterMaxSlices, std::max(1, (512 + base - 1) / base));
  slices = std::min(slices, std::max(1, steps / 2));
  const int per = (steps + slices - 1) / slices;
  return (steps + per - 1) / per;
}

void launch_router_mfma(const uint8_t* wp, int E, int H, const float* x, int T, double* part,
                        int slices, int* status, hipStream_t s) {
  const int steps = H / kKS;
  const int per = (steps + slices - 1) / slices;
  dim3 grid(router_rows(E) / kNT, (T + kMT - 1) / kMT, slices);
  router_mfma_kernel<4><<<grid, 256, 0, s>>>(wp, router_rows(E), H, x, T, per, part, status);
}

template <int FMT, bool PAIR, int DEPTH, int NP>
static void launch_shape(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                         const float* in, float* out, int qwen, int* status, hipStream_t s) {
  dim3 grid(rows / (kNT * NP), max_tiles);
  gemm_kernel<FMT, PAIR, DEPTH, NP><<<grid, 256, 0, s>>>(mats, perm, rows, K, in, out, qwen,
                                                          status);
}

// Weight steps in flight per wave (DEPTH) and panels per wave (NP), per format.  BF16 steps are
// 4 KiB per panel, so one panel one step deep; the MX formats stream 1-2 KiB per panel and
// step and need more panels per staged activation tile (activations are 2-4x their bytes).
// Rows are multiples of 128 (urb_moe_create), so NP = 2 always tiles them.
template <int FMT, bool PAIR>
static void launch(const ExpertMats* mats, const Perm& perm, int max_tiles, int rows, int K,
                   const float* in, float* out, int qwen, int* status, hipStream_t s) {
  if constexpr (FMT == kFmtBF16)
    launch_shape<FMT, PAIR, 1, 1>(mats, perm, max_tiles, rows, K, in, out, qwen, status, s);
  else if constexpr (FMT == kFmtMXFP8)
    launch_shape<FMT, PAIR, 1, 2>(mats, perm, max_tiles, rows, K, in, out, qwen, status, s);
  else if (rows % (kNT * 4) == 0)
    launch_shape<FMT, PAIR, 1, 4>(mats, perm, max_tiles, rows, K, in, out, qwen, status, s);
  else
    launch_shape<FMT, PAIR, 2, 2>(mats, perm, max_tiles, rows, K, in, out, qwen, status, s);
}

void launch_gemm_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                         int I, const float* x, float* act, int qwen, int* status,
                         hipStream_t s) {
  if (fmt == kFmtBF16) launch<kFmtBF16, true>(mats, perm, max_tiles, I, H, x, act, qwen, status, s);
  else if (fmt == kFmtMXFP4) launch<kFmtMXFP4, true>(mats, perm, max_tiles, I, H, x, act, qwen, status, s);
  else launch<kFmtMXFP8, true>(mats, perm, max_tiles, I, H, x, act, qwen, status, s);
}

void launch_gemm_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                      int I, const float* act, float* y, int qwen, int* status, hipStream_t s) {
  if (fmt == kFmtBF16) launch<kFmtBF16, false>(mats, perm, max_tiles, H, I, act, y, qwen, status, s);
  else if (fmt == kFmtMXFP4) launch<kFmtMXFP4, false>(mats, perm, max_tiles, H, I, act, y, qwen, status, s);
  else launch<kFmtMXFP8, false>(mats, perm, max_tiles, H, I, act, y, qwen, status, s);
}

}  // namespace urb
