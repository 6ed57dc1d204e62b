// urb_decode.hip -- one-token expert projections on the matrix cores (decode).
//
// A decode projection is a GEMV: every weight byte is used once, so the kernel's job is to keep
// enough bytes in flight to saturate HBM while spending few instructions per byte.  Dot
// products on the FMA lanes cost two VALU operations per MXFP4 weight (decode + FMA) plus an
// LDS read of the input per weight, more than a CU can issue at HBM speed.  Here the weights go
// to v_mfma_f32_16x16x32_bf16 as the B operand straight from the panel layout (BF16 as loaded;
// MX blocks through the scaled CDNA4 conversions, exact), and the A operand holds the input
// vector as BF16 pieces (hi, lo: 16 significant bits, urb_panel.hpp), one piece per A row.
// C rows 0 and 1 of lane (ln, 0) are the two pieces' partial sums of weight row ln, added in
// f32.  15 of the 16 A rows are padding, but the matrix cores have ~5x the throughput this
// needs, and the VALU is left with the MX decode alone.
//
// Bytes in flight: a workgroup stages its input pieces in LDS once, so the only vector-memory
// loads in the main loop are weights.  (Vector-memory loads complete in order: an input load
// sharing the counter with the weight loads would make every step wait for all older weight
// loads, capping the useful prefetch at the input's distance.)  Each wave keeps DW weight steps
// in flight in a register ring of DW + 1 slots, the step loop unrolled DW + 1 times.
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
// times KSPLIT parts of K, for one slot (blockIdx.y).  Dynamic LDS: the slot's input pieces,
// cols / 8 units of 32 B.
template <int FMT, bool PAIR, int NP, int DW, int WMAX>
__global__ __launch_bounds__(64 * WMAX) void gemv_mfma_kernel(
    const ExpertMats* __restrict__ mats, Perm perm, int rows, int cols, int ksplit,
    const uint16_t* __restrict__ xp, float* __restrict__ out, uint16_t* __restrict__ out_xp,
    Epi epi, int* status) {
  extern __shared__ uint4 xs[];
  __shared__ float red[WMAX][NP][16][2];
  int expert, pos;
  if (!decode_slot(perm, blockIdx.y, expert, pos)) return;
  const ExpertMats m = mats[expert];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lq = lane >> 4, piece = ln & 1;
  const int part = wave % ksplit;
  const int groups = (int)(blockDim.x >> 6) / ksplit;  // panel groups per workgroup
  const int panel0 = (blockIdx.x * groups + wave / ksplit) * NP;
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
  const uint32_t doff = 16u * lane, soff = lane;

  constexpr int R = DW + 1;
  BRaw<FMT> r0[R][NP], r1[R][NP];
  auto fetch = [&](int slot, int s) {
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
            if constexpr (PAIR)
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

template <int FMT, bool PAIR>
static void launch_gemv_mfma(const ExpertMats* mats, const Perm& perm, int max_active, int rows,
                             int cols, const uint16_t* xp, float* out, uint16_t* out_xp, Epi epi,
                             int* status, hipStream_t s) {
  constexpr int NP = decode_panels<FMT, PAIR>();
  constexpr int D = decode_depth<FMT, PAIR>();
  constexpr int WMAX = decode_max_waves<FMT, PAIR>();
  const int panels = rows / kPanelRows, steps = cols / kGemmKStep;
  // split K until the launch has ~8192 waves, keeping at least two steps a part; a workgroup
  // holds max(4, ksplit) waves
  int ksplit = 1;
  while (ksplit < WMAX && (long)panels / NP * max_active * ksplit < 8192 &&
         steps / (2 * ksplit) >= 1)
    ksplit *= 2;
  const int waves = std::max(4, ksplit);
  const int per_wg = waves / ksplit * NP;
  const dim3 grid((panels + per_wg - 1) / per_wg, max_active);
  const size_t lds = (size_t)cols / 8 * 32;
  gemv_mfma_kernel<FMT, PAIR, NP, D, WMAX><<<grid, 64 * waves, lds, s>>>(
      mats, perm, rows, cols, ksplit, xp, out, out_xp, epi, status);
}

void launch_gemv_mfma_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                              int H, int I, const uint16_t* xp, float* act, uint16_t* act_xp,
                              Epi epi, int* status, hipStream_t s) {
  if (fmt == kFmtBF16)
    launch_gemv_mfma<kFmtBF16, true>(mats, perm, max_active, I, H, xp, act, act_xp, epi, status, s);
  else if (fmt == kFmtMXFP4)
    launch_gemv_mfma<kFmtMXFP4, true>(mats, perm, max_active, I, H, xp, act, act_xp, epi, status, s);
  else
    launch_gemv_mfma<kFmtMXFP8, true>(mats, perm, max_active, I, H, xp, act, act_xp, epi, status, s);
}

void launch_gemv_mfma_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                           int H, int I, const uint16_t* act_xp, float* y, Epi epi, int* status,
                           hipStream_t s) {
  if (fmt == kFmtBF16)
    launch_gemv_mfma<kFmtBF16, false>(mats, perm, max_active, H, I, act_xp, y, nullptr, epi, status, s);
  else if (fmt == kFmtMXFP4)
    launch_gemv_mfma<kFmtMXFP4, false>(mats, perm, max_active, H, I, act_xp, y, nullptr, epi, status, s);
  else
    launch_gemv_mfma<kFmtMXFP8, false>(mats, perm, max_active, H, I, act_xp, y, nullptr, epi, status, s);
}

// ------------------------------------------------------------------------------------------
// The down projection of the k routed experts fused with the combine (one token).  A
// workgroup owns one 16-row output panel; its waves are tasks (slot a, K part z),
// a * ksplit + z, one each.  The k SwiGLU rows' pieces are staged in LDS once; task partials
// meet in LDS; 16 threads add each slot's parts in order, apply the down epilogue and combine
// the slots in the composition's order -- the per-slot outputs never leave the chip and no
// combine kernel runs.  `comp` = composition (0 QWEN36, 1 GLM, 2 HY4, 3 DSV41).
// ------------------------------------------------------------------------------------------
template <int FMT, int DW>
__global__ __launch_bounds__(64 * kDecodeMaxWaves) void gemv_mfma_down_combine_kernel(
    const ExpertMats* __restrict__ mats, const int32_t* __restrict__ ids,
    const float* __restrict__ w, const int32_t* __restrict__ asc, int K, int H, int I, int ksplit,
    const uint16_t* __restrict__ act_xp, const float* __restrict__ shared, int comp, Epi epi,
    const float* __restrict__ residual, const float* __restrict__ gate, float* __restrict__ out,
    int* status) {
  extern __shared__ uint4 xs[];  // K x I / 8 piece units
  __shared__ float red[kDecodeMaxWaves][16];
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's task
  const int ln = lane & 15, lq = lane >> 4, piece = ln & 1;
  const int panel = blockIdx.x;
  const int steps = I / kGemmKStep;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(I);
  const size_t pscales = (size_t)kPanelRows * (I / 32);
  const uint32_t doff = 16u * lane, soff = lane;
  const int a = t / ksplit, z = t - a * ksplit;
  const int s_begin = steps * z / ksplit, n = steps * (z + 1) / ksplit - s_begin;
  const ExpertMats m = mats[ids[a]];
  const uint8_t* pd = m.data[2] + (size_t)panel * pbytes;
  const uint8_t* ps = FMT == kFmtBF16 ? nullptr : m.scales[2] + (size_t)panel * pscales;
  constexpr int R = DW + 1;
  BRaw<FMT> r[R];
#pragma unroll
  for (int d = 0; d < DW; ++d)
    if (d < n) load_b<FMT, true>(r[d], pd, doff, ps, soff, s_begin + d);
  stage_pieces(act_xp, xs, K * (I / 8));
  __syncthreads();
  const uint4* xa = xs + (size_t)a * (I / 8) * 2;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < n; i0 += R) {
#pragma unroll
    for (int d = 0; d < R; ++d) {
      const int i = i0 + d;
      if (i >= n) break;
      if (i + DW < n) load_b<FMT, true>(r[(d + DW) % R], pd, doff, ps, soff, s_begin + i + DW);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_piece<FMT>(xa, s_begin + i, j, lq, piece),
                                                      decode_b<FMT>(r[d], j), acc, 0, 0, 0);
    }
  }
  if (lq == 0) red[t][ln] = acc[0] + acc[1];
  __syncthreads();

  if (threadIdx.x < 16) {
    const int row = panel * kPanelRows + threadIdx.x;
    bool bad = false;
    auto y = [&](int a) {
      float v = 0.0f;
      for (int z = 0; z < ksplit; ++z) v += red[a * ksplit + z][threadIdx.x];
      return epi_down<FMT>(epi, v, bad);
    };
    float res;
    if (comp == 1) {
      // GLM (src/models/glm/runtime/moe.rs:162-171): f64 from the shared expert, ranking order
      double acc = shared ? (double)shared[row] : 0.0;
      for (int j = 0; j < K; ++j) acc += (double)w[j] * (double)y(j);
      res = (float)acc;
    } else {
      float acc = 0.0f;
      for (int j = 0; j < K; ++j) {
        const int a = asc[j];
        const float v = y(a);
        if (comp == 0) {
          // Qwen (src/models/qwen3_6/runtime.rs:1398-1415): c = bf16(w y), acc = bf16(acc + c)
          float c;
          if (!rne_bf16(w[a] * v, &c)) { bad = true; c = w[a] * v; }
          const float t = acc + c;
          if (!rne_bf16(t, &acc)) { bad = true; acc = t; }
        } else if (comp == 2) {
          acc = acc + w[a] * v;  // Hy4 (src/models/hy4/runtime.rs:1436-1441): f32
        } else {
          acc = acc + v;  // DeepSeek V4.1 (deepseek_v41/runtime.rs:1995-1998): weight applied
        }
      }
      if (comp == 0 && shared) {
        // the gated shared expert (src/models/qwen3_6/runtime.rs:1436-1461)
        const float sc = qwen_shared_scale(gate[0], bad);
        float c;
        if (!rne_bf16(sc * shared[row], &c)) { bad = true; c = sc * shared[row]; }
        const float t = acc + c;
        if (!rne_bf16(t, &acc)) { bad = true; acc = t; }
      }
      if (comp >= 2) {
        if (shared) acc = acc + shared[row];
        float b;
        if (!rne_bf16(acc, &b)) { bad = true; b = acc; }
        acc = b;
      }
      res = acc;
    }
    if (residual) {
      // add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494)
      const float t = residual[row] + res;
      if (!rne_bf16(t, &res)) { bad = true; res = t; }
    }
    out[row] = res;
    if (bad) flag(status, kStatusNonFinite);
  }
}

// The k SwiGLU rows' pieces (4 I bytes each) must fit the LDS the fused kernel stages, and its
// tasks one wave each.
constexpr size_t kDownComboLds = 96 * 1024;
bool mfma_down_combine_fits(int K, int I) {
  return K <= kDecodeMaxWaves && (size_t)K * I * 4 <= kDownComboLds;
}

bool launch_gemv_mfma_down_combine(int fmt, const ExpertMats* mats, const int32_t* ids,
                                   const float* weights, const int32_t* asc, int K, int H, int I,
                                   const uint16_t* act_xp, const float* shared, int comp, Epi epi,
                                   float* out, int* status, hipStream_t s,
                                   const float* residual, const float* gate) {
  if (!mfma_down_combine_fits(K, I)) return false;
  const int steps = I / kGemmKStep;
  // one task per wave: split K while the workgroup stays within 16 waves, 2+ steps a part
  int ksplit = 1;
  while (K * ksplit * 2 <= kDecodeMaxWaves && steps / (2 * ksplit) >= 2) ksplit *= 2;
  const dim3 grid(H / kPanelRows), block(64 * K * ksplit);
  const size_t lds = (size_t)K * I * 4;
  auto go = [&](auto kernel) {
    // dynamic LDS beyond 64 KiB must be allowed per kernel
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDownComboLds);
    kernel<<<grid, block, lds, s>>>(mats, ids, weights, asc, K, H, I, ksplit, act_xp, shared,
                                    comp, epi, residual, gate, out, status);
  };
  if (fmt == kFmtBF16) go(gemv_mfma_down_combine_kernel<kFmtBF16, decode_depth<kFmtBF16, false>()>);
  else if (fmt == kFmtMXFP4) go(gemv_mfma_down_combine_kernel<kFmtMXFP4, decode_depth<kFmtMXFP4, false>()>);
  else go(gemv_mfma_down_combine_kernel<kFmtMXFP8, decode_depth<kFmtMXFP8, false>()>);
  return true;
}

// ------------------------------------------------------------------------------------------
// Piece vectors of f32 rows [rows, cols] (cols % 8 == 0): one thread per unit.
// ------------------------------------------------------------------------------------------
__global__ void split_pieces_kernel(const float* __restrict__ x, size_t units,
                                    uint16_t* __restrict__ out) {
  for (size_t u = blockIdx.x * (size_t)blockDim.x + threadIdx.x; u < units;
       u += (size_t)gridDim.x * blockDim.x) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * u];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * u + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    store_piece_unit(v, out + u * kPieceUnit);
  }
}

void launch_split_pieces(const float* x, size_t rows, size_t cols, uint16_t* out,
                         hipStream_t s) {
  const size_t units = rows * cols / 8;
  const int blocks = (int)std::min<size_t>(std::max<size_t>((units + 255) / 256, 1), 4096);
  split_pieces_kernel<<<blocks, 256, 0, s>>>(x, units, out);
}

}  // namespace urb
