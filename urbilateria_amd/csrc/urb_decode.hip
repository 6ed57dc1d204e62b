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
#include "urb_decode.hpp"

namespace urb {

// The MFMA GEMV of one slot's panel groups (gemv_mfma_body, urb_decode.hpp) as a kernel.
template <int FMT, bool PAIR, int NP, int DW, int WMAX>
__global__ __launch_bounds__(64 * WMAX) void gemv_mfma_kernel(
    const ExpertMats* __restrict__ mats, Perm perm, int rows, int cols, int ksplit,
    const uint16_t* __restrict__ xp, float* __restrict__ out, uint16_t* __restrict__ out_xp,
    Epi epi, int* status) {
  extern __shared__ uint4 xs[];
  gemv_mfma_body<FMT, PAIR, NP, DW, WMAX>(mats, perm, rows, cols, ksplit, xp, out, out_xp, epi,
                                          status, xs, blockIdx.x, blockIdx.y);
}

template <int FMT, bool PAIR>
static void launch_gemv_mfma(const ExpertMats* mats, const Perm& perm, int max_active, int rows,
                             int cols, const uint16_t* xp, float* out, uint16_t* out_xp, Epi epi,
                             int* status, hipStream_t s) {
  const GemvShape g = gemv_mfma_shape<FMT, PAIR>(rows, cols, max_active);
  gemv_mfma_kernel<FMT, PAIR, decode_panels<FMT, PAIR>(), decode_depth<FMT, PAIR>(),
                   decode_max_waves<FMT, PAIR>()><<<g.grid, 64 * g.waves, g.lds, s>>>(
      mats, perm, rows, cols, g.ksplit, xp, out, out_xp, epi, status);
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
// One token with a shared expert: the routed experts' gate+up and the shared expert's down
// projection in one launch.  Workgroups [0, gx_r * slots) run the routed GEMV (workgroup b:
// panel group b % gx_r of slot b / gx_r), the others the shared down GEMV.  Both read inputs
// that earlier launches wrote and write disjoint outputs, so the shared down's weights stream
// beside the routed ones without a kernel boundary.  Every workgroup has kPairWaves waves;
// each part splits K at most that many ways.
// ------------------------------------------------------------------------------------------
constexpr int kPairWaves = 8;

template <int FR, int FS>
__global__ __launch_bounds__(64 * kPairWaves) void gemv_gate_up_and_down_kernel(
    const ExpertMats* __restrict__ mats_r, Perm perm, int I, int H, int ksplit_r, int gx_r,
    int slots, const uint16_t* __restrict__ xp, float* __restrict__ act,
    uint16_t* __restrict__ act_xp, const ExpertMats* __restrict__ mats_s, int Is, int ksplit_s,
    const uint16_t* __restrict__ shared_xp, float* __restrict__ shared_out, Epi epi_r,
    Epi epi_s, int* status) {
  extern __shared__ uint4 xs[];
  const int nr = gx_r * slots;
  if ((int)blockIdx.x < nr) {
    gemv_mfma_body<FR, true, decode_panels<FR, true>(), decode_depth<FR, true>(), kPairWaves>(
        mats_r, perm, I, H, ksplit_r, xp, act, act_xp, epi_r, status, xs, blockIdx.x % gx_r,
        blockIdx.x / gx_r);
  } else {
    const Perm dense{nullptr, nullptr, nullptr, nullptr, nullptr, 1, nullptr, nullptr, 0};
    gemv_mfma_body<FS, false, decode_panels<FS, false>(), decode_depth<FS, false>(),
                   kPairWaves>(mats_s, dense, H, Is, ksplit_s, shared_xp, shared_out, nullptr,
                               epi_s, status, xs, blockIdx.x - nr, 0);
  }
}

template <int FR, int FS>
static void launch_gate_up_and_down(const ExpertMats* mats_r, const Perm& perm, int slots, int H,
                                    int I, const uint16_t* xp, float* act, uint16_t* act_xp,
                                    const ExpertMats* mats_s, int Is, const uint16_t* shared_xp,
                                    float* shared_out, Epi epi_r, Epi epi_s, int* status,
                                    hipStream_t s) {
  static_assert(decode_panels<FR, true>() == 1 && decode_panels<FS, false>() == 1,
                "one panel per wave");
  const int kr = std::min(gemv_mfma_shape<FR, true>(I, H, slots).ksplit, kPairWaves);
  const int ks = std::min(gemv_mfma_shape<FS, false>(H, Is, 1).ksplit, kPairWaves);
  const int per_r = kPairWaves / kr, per_s = kPairWaves / ks;  // panels per workgroup
  const int gx_r = (I / kPanelRows + per_r - 1) / per_r;
  const int gx_s = (H / kPanelRows + per_s - 1) / per_s;
  const size_t lds = (size_t)std::max(H, Is) / 8 * 32;
  gemv_gate_up_and_down_kernel<FR, FS><<<gx_r * slots + gx_s, 64 * kPairWaves, lds, s>>>(
      mats_r, perm, I, H, kr, gx_r, slots, xp, act, act_xp, mats_s, Is, ks, shared_xp,
      shared_out, epi_r, epi_s, status);
}

template <int FR>
static void launch_gate_up_and_down_fr(int fs, const ExpertMats* mats_r, const Perm& perm,
                                       int slots, int H, int I, const uint16_t* xp, float* act,
                                       uint16_t* act_xp, const ExpertMats* mats_s, int Is,
                                       const uint16_t* shared_xp, float* shared_out, Epi epi_r,
                                       Epi epi_s, int* status, hipStream_t s) {
  if (fs == kFmtBF16)
    launch_gate_up_and_down<FR, kFmtBF16>(mats_r, perm, slots, H, I, xp, act, act_xp, mats_s,
                                          Is, shared_xp, shared_out, epi_r, epi_s, status, s);
  else if (fs == kFmtMXFP4)
    launch_gate_up_and_down<FR, kFmtMXFP4>(mats_r, perm, slots, H, I, xp, act, act_xp, mats_s,
                                           Is, shared_xp, shared_out, epi_r, epi_s, status, s);
  else
    launch_gate_up_and_down<FR, kFmtMXFP8>(mats_r, perm, slots, H, I, xp, act, act_xp, mats_s,
                                           Is, shared_xp, shared_out, epi_r, epi_s, status, s);
}

void launch_gemv_mfma_gate_up_and_shared_down(int fmt, const ExpertMats* mats, const Perm& perm,
                                              int max_active, int H, int I, const uint16_t* xp,
                                              float* act, uint16_t* act_xp, Epi epi,
                                              int shared_fmt, const ExpertMats* shared_mats,
                                              int Is, const uint16_t* shared_xp,
                                              float* shared_out, Epi shared_epi, int* status,
                                              hipStream_t s) {
  if (fmt == kFmtBF16)
    launch_gate_up_and_down_fr<kFmtBF16>(shared_fmt, mats, perm, max_active, H, I, xp, act,
                                         act_xp, shared_mats, Is, shared_xp, shared_out, epi,
                                         shared_epi, status, s);
  else if (fmt == kFmtMXFP4)
    launch_gate_up_and_down_fr<kFmtMXFP4>(shared_fmt, mats, perm, max_active, H, I, xp, act,
                                          act_xp, shared_mats, Is, shared_xp, shared_out, epi,
                                          shared_epi, status, s);
  else
    launch_gate_up_and_down_fr<kFmtMXFP8>(shared_fmt, mats, perm, max_active, H, I, xp, act,
                                          act_xp, shared_mats, Is, shared_xp, shared_out, epi,
                                          shared_epi, status, s);
}

// ------------------------------------------------------------------------------------------
// The down projection of the k routed experts fused with the combine (one token).  A
// workgroup owns one 16-row output panel; its waves are tasks (slot a, K part z),
// a * ksplit + z, one each.  The k SwiGLU rows' pieces are staged in LDS once; task partials
// meet in LDS; the first wave of each slot adds the slot's parts in order and applies the down
// epilogue; 16 threads combine the slots in the composition's order -- the per-slot outputs
// never leave the chip and no combine kernel runs.  `comp` = composition (0 QWEN36, 1 GLM,
// 2 HY4, 3 DSV41).  The combine's inputs (route weights and order, shared and residual rows,
// gate) are loaded while the weights stream, and the combine reads every slot before it adds:
// with dependent loads per slot, the 16-thread tail cost ~1.3 us of a 14.5 us launch.
// ------------------------------------------------------------------------------------------
// HALF: a workgroup owns 8 output rows (half a panel; lanes ln >= 8 load the same rows as
// ln - 8, from the same cache lines, and their MFMA columns are dropped), so H / 8 workgroups
// keep every CU streaming where H / 16 would not (hidden below 4096).
template <int FMT, int DW, bool HALF>
__global__ __launch_bounds__(64 * kDecodeMaxWaves) void gemv_mfma_down_combine_kernel(
    const ExpertMats* __restrict__ mats, const int32_t* __restrict__ ids,
    const float* __restrict__ w, const int32_t* __restrict__ asc, int K, int H, int I, int ksplit,
    const uint16_t* __restrict__ act_xp, const float* __restrict__ shared, int comp, Epi epi,
    const float* __restrict__ residual, const float* __restrict__ gate, float* __restrict__ out,
    int* status) {
  extern __shared__ uint4 xs[];  // K x I / 8 piece units
  __shared__ float red[kDecodeMaxWaves][16];
  __shared__ float ys[kDecodeMaxWaves][16];  // slot outputs after the down epilogue
  __shared__ float wl[kDecodeMaxWaves];
  __shared__ int al[kDecodeMaxWaves];
  // combine inputs, in flight during the weight stream
  float wv = 0.0f, sv = 0.0f, rv = 0.0f, gv = 0.0f;
  int av = 0;
  if (threadIdx.x < K) {
    wv = w[threadIdx.x];
    if (comp != 1) av = asc[threadIdx.x];
  }
  constexpr int kRows = HALF ? 8 : kPanelRows;  // output rows of this workgroup
  const int panel = HALF ? blockIdx.x >> 1 : blockIdx.x;
  const int row0 = panel * kPanelRows + (HALF ? (blockIdx.x & 1) * 8 : 0);
  if (threadIdx.x < kRows) {
    const int row = row0 + threadIdx.x;
    if (shared) sv = shared[row];
    if (residual) rv = residual[row];
    if (gate) gv = gate[0];
  }
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's task
  const int ln = lane & 15, lq = lane >> 4, piece = ln & 1;
  const int steps = I / kGemmKStep;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(I);
  const size_t pscales = (size_t)kPanelRows * (I / 32);
  // HALF: lane (ln, lq) takes the panel lane of row (row0 % 16) + ln % 8 at k-quad lq
  const int src = HALF ? lq * 16 + (row0 & 15) + (ln & 7) : lane;
  const uint32_t doff = 16u * src, soff = src;
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
  if (threadIdx.x < K) {
    wl[threadIdx.x] = wv;
    al[threadIdx.x] = av;
  }
  __syncthreads();
  if (z == 0 && lq == 0) {
    bool bad = false;
    float v = 0.0f;
    for (int zz = 0; zz < ksplit; ++zz) v += red[t + zz][ln];  // K parts in order
    ys[a][ln] = epi_down<FMT>(epi, v, bad);
    if (bad) flag(status, kStatusNonFinite);
  }
  __syncthreads();

  if (threadIdx.x < kRows) {
    const int row = row0 + threadIdx.x;
    bool bad = false;
    // slot j's output and weight in combine order: ranking order (GLM) or ascending id
    float yv[kDecodeMaxWaves], wr[kDecodeMaxWaves];
#pragma unroll
    for (int j = 0; j < kDecodeMaxWaves; ++j) {
      const int a = j < K ? (comp == 1 ? j : al[j]) : 0;
      yv[j] = ys[a][threadIdx.x];
      wr[j] = wl[a];
    }
    float res;
    if (comp == 1) {
      // GLM (src/models/glm/runtime/moe.rs:162-171): f64 from the shared expert, ranking order
      double acc = shared ? (double)sv : 0.0;
#pragma unroll
      for (int j = 0; j < kDecodeMaxWaves; ++j)
        if (j < K) acc += (double)wr[j] * (double)yv[j];
      res = (float)acc;
    } else {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < kDecodeMaxWaves; ++j) {
        if (j >= K) break;
        const float v = yv[j];
        if (comp == 0) {
          // Qwen (src/models/qwen3_6/runtime.rs:1398-1415): c = bf16(w y), acc = bf16(acc + c)
          float c;
          if (!rne_bf16(wr[j] * v, &c)) { bad = true; c = wr[j] * v; }
          const float t = acc + c;
          if (!rne_bf16(t, &acc)) { bad = true; acc = t; }
        } else if (comp == 2) {
          acc = acc + wr[j] * v;  // Hy4 (src/models/hy4/runtime.rs:1436-1441): f32
        } else {
          acc = acc + v;  // DeepSeek V4.1 (deepseek_v41/runtime.rs:1995-1998): weight applied
        }
      }
      if (comp == 0 && shared) {
        // the gated shared expert (src/models/qwen3_6/runtime.rs:1436-1461)
        const float sc = qwen_shared_scale(gv, bad);
        float c;
        if (!rne_bf16(sc * sv, &c)) { bad = true; c = sc * sv; }
        const float t = acc + c;
        if (!rne_bf16(t, &acc)) { bad = true; acc = t; }
      }
      if (comp >= 2) {
        if (shared) acc = acc + sv;
        float b;
        if (!rne_bf16(acc, &b)) { bad = true; b = acc; }
        acc = b;
      }
      res = acc;
    }
    if (residual) {
      // add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494)
      const float t = rv + res;
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
  // half panels where whole ones leave CUs idle (hidden 2048: 128 -> 256 workgroups)
  const bool half = H / kPanelRows < 256;
  const dim3 grid(half ? H / 8 : H / kPanelRows), block(64 * K * ksplit);
  const size_t lds = (size_t)K * I * 4;
  auto go = [&](auto kernel) {
    // dynamic LDS beyond 64 KiB must be allowed per kernel
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDownComboLds);
    kernel<<<grid, block, lds, s>>>(mats, ids, weights, asc, K, H, I, ksplit, act_xp, shared,
                                    comp, epi, residual, gate, out, status);
  };
  auto pick = [&](auto fmtc) {
    constexpr int F = decltype(fmtc)::value;
    if (half) go(gemv_mfma_down_combine_kernel<F, decode_depth<F, false>(), true>);
    else go(gemv_mfma_down_combine_kernel<F, decode_depth<F, false>(), false>);
  };
  if (fmt == kFmtBF16) pick(Int<kFmtBF16>{});
  else if (fmt == kFmtMXFP4) pick(Int<kFmtMXFP4>{});
  else pick(Int<kFmtMXFP8>{});
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
