// urb_gemv.hip -- decode-path expert projections, combines, validation and dequantisation.
//
// Decode projections (one token per active expert) stream the panel layout
// (urb_kernels.hpp).  A 256-thread workgroup is 4 / KSPLIT panels x KSPLIT parts of K; each
// wave sweeps its part of one panel front to back, DEPTH K steps of 1 KiB slabs in flight.
// Lane l = ln + 16 lq accumulates panel row ln over the columns its 16-byte units hold
// (BF16: 8 columns per unit; MX: one whole 32-column block, decoded with the CDNA4
// v_cvt_scalef32_pk_f32_fp4/fp8 conversions and scaled once per block, which is exact
// multiplication by 2^k of the block partial), against the input vector staged in LDS.  The
// four lq lanes are summed by shuffles and the K parts through LDS, in a fixed order.  (FMA
// lanes beat the matrix cores here: with one token, 15 of an MFMA's 16 rows would be zero.)
// Each weight is read once per call, so the weight loads are non-temporal.
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {

// Staged input vectors carry 4 floats of padding after every 32, so the four lane groups'
// 32-column blocks (128 B apart) start in different LDS banks.
__device__ __forceinline__ int xs_index(int k) { return k + 4 * (k >> 5); }
__host__ __device__ constexpr size_t xs_floats(int K) { return (size_t)K + (size_t)K / 8; }

// acc += lane's units of one K step . x.  BF16 unit j covers k = 128 s + 32 j + 8 lq + [0, 8);
// an MX unit covers k = 128 s + 32 lq + [0, 32).
template <int FMT>
__device__ __forceinline__ void raw_dot(const BRaw<FMT>& r, int step, int lq,
                                        const float* __restrict__ xs, float& acc) {
  if constexpr (FMT == kFmtBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 q = r.q[j];
      const float4* xv = reinterpret_cast<const float4*>(xs + xs_index(128 * step + 32 * j + 8 * lq));
      const float4 a = xv[0], b = xv[1];
      float p0 = bf16_lo(q.x) * a.x, p1 = bf16_hi(q.x) * a.y;
      p0 = fmaf(bf16_lo(q.y), a.z, p0);
      p1 = fmaf(bf16_hi(q.y), a.w, p1);
      p0 = fmaf(bf16_lo(q.z), b.x, p0);
      p1 = fmaf(bf16_hi(q.z), b.y, p1);
      p0 = fmaf(bf16_lo(q.w), b.z, p0);
      p1 = fmaf(bf16_hi(q.w), b.w, p1);
      acc += p0 + p1;
    }
  } else {
    const float scale = e8m0_to_f32(r.s);
    const float4* xv = reinterpret_cast<const float4*>(xs + xs_index(128 * step + 32 * lq));
    uint32_t words[8];
    if constexpr (FMT == kFmtMXFP4) {
      words[0] = r.q.x; words[1] = r.q.y; words[2] = r.q.z; words[3] = r.q.w;
    } else {
      words[0] = r.q[0].x; words[1] = r.q[0].y; words[2] = r.q[0].z; words[3] = r.q[0].w;
      words[4] = r.q[1].x; words[5] = r.q[1].y; words[6] = r.q[1].z; words[7] = r.q[1].w;
    }
    float part[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {  // 8 columns each
      float v[8];
      if constexpr (FMT == kFmtMXFP4) {
        decode_fp4x8(words[h], v);
      } else {
        decode_fp8x4(words[2 * h], v);
        decode_fp8x4(words[2 * h + 1], v + 4);
      }
      const float4 a = xv[2 * h], b = xv[2 * h + 1];
      float p = v[0] * a.x;
      p = fmaf(v[1], a.y, p);
      p = fmaf(v[2], a.z, p);
      p = fmaf(v[3], a.w, p);
      p = fmaf(v[4], b.x, p);
      p = fmaf(v[5], b.y, p);
      p = fmaf(v[6], b.z, p);
      p = fmaf(v[7], b.w, p);
      part[h] = p;
    }
    acc = fmaf((part[0] + part[1]) + (part[2] + part[3]), scale, acc);
  }
}

// Resolves an active slot -> expert and its first permuted position.
__device__ __forceinline__ bool perm_expert(const Perm& perm, int a, int& expert, int& base,
                                            int& count) {
  if (perm.dense_tokens > 0) {
    if (a != 0) return false;
    expert = 0;
    base = 0;
    count = perm.dense_tokens;
    return true;
  }
  if (perm.direct) {
    if (a >= perm.direct_k) return false;
    expert = perm.direct[a];
    base = a;
    count = 1;
    return true;
  }
  if (a >= perm.meta[0]) return false;
  expert = perm.active[a];
  base = perm.offsets[expert];
  count = perm.counts[expert];
  return true;
}

template <int FMT, bool PAIR, int DEPTH>
__global__ __launch_bounds__(256) void gemv_kernel(const ExpertMats* __restrict__ mats,
                                                   Perm perm, int rows, int cols, int ksplit,
                                                   const float* __restrict__ in,
                                                   float* __restrict__ out, Epi epi,
                                                   int* status) {
  extern __shared__ float xs[];  // xs_floats(cols) staged input + [4][16][2] part sums
  int expert, base, count;
  if (!perm_expert(perm, blockIdx.y, expert, base, count)) return;
  const ExpertMats m = mats[expert];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lq = lane >> 4;
  const int part = wave % ksplit;
  const int panel = blockIdx.x * (4 / ksplit) + wave / ksplit;
  const bool valid = panel < rows / kPanelRows;
  const int steps = cols / kGemmKStep;
  const int s_begin = steps * part / ksplit, s_end = steps * (part + 1) / ksplit;
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(cols);
  const size_t pscales = (size_t)kPanelRows * (cols / 32);
  const uint8_t* pd0 = m.data[PAIR ? 0 : 2] + (size_t)panel * pbytes + 16 * lane;
  const uint8_t* ps0 =
      FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + (size_t)panel * pscales + lane;
  const uint8_t* pd1 = PAIR ? m.data[1] + (size_t)panel * pbytes + 16 * lane : nullptr;
  const uint8_t* ps1 =
      (PAIR && FMT != kFmtBF16) ? m.scales[1] + (size_t)panel * pscales + lane : nullptr;

  // The first DEPTH steps of weights are requested before the input vector is staged, so the
  // two memory latencies overlap.
  BRaw<FMT> r0[DEPTH], r1[DEPTH];
  if (valid) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (s_begin + d < s_end) {
        load_b<FMT, true>(r0[d], pd0, ps0, s_begin + d);
        if constexpr (PAIR) load_b<FMT, true>(r1[d], pd1, ps1, s_begin + d);
      }
  }
  const int p = base;  // the expert's one permuted position
  const int token = perm.dense_tokens > 0 ? p : (perm.direct ? 0 : perm.perm_token[p]);
  const float* src = PAIR ? in + (size_t)token * cols
                          : in + (size_t)p * cols;
  {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    for (int i = threadIdx.x; i < cols / 4; i += blockDim.x)
      *reinterpret_cast<float4*>(xs + xs_index(4 * i)) = s4[i];
  }
  __syncthreads();

  float acc0 = 0.0f, acc1 = 0.0f;
  if (valid) {
    for (int s0 = s_begin; s0 < s_end; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int s = s0 + d;
        if (s >= s_end) break;
        BRaw<FMT> c0 = r0[d], c1;
        if constexpr (PAIR) c1 = r1[d];
        if (s + DEPTH < s_end) {
          load_b<FMT, true>(r0[d], pd0, ps0, s + DEPTH);
          if constexpr (PAIR) load_b<FMT, true>(r1[d], pd1, ps1, s + DEPTH);
        }
        raw_dot<FMT>(c0, s, lq, xs, acc0);
        if constexpr (PAIR) raw_dot<FMT>(c1, s, lq, xs, acc1);
      }
    }
  }
  acc0 += __shfl_xor(acc0, 16);
  acc0 += __shfl_xor(acc0, 32);
  if constexpr (PAIR) {
    acc1 += __shfl_xor(acc1, 16);
    acc1 += __shfl_xor(acc1, 32);
  }
  if (ksplit > 1) {
    float* red = xs + xs_floats(cols);
    if (lane < 16) {
      red[(wave * 16 + lane) * 2] = acc0;
      red[(wave * 16 + lane) * 2 + 1] = acc1;
    }
    __syncthreads();
    if (part == 0 && lane < 16) {
      acc0 = 0.0f;
      acc1 = 0.0f;
      for (int q = 0; q < ksplit; ++q) {
        acc0 += red[((wave + q) * 16 + lane) * 2];
        acc1 += red[((wave + q) * 16 + lane) * 2 + 1];
      }
    }
  }
  if (!valid || part != 0 || lane >= 16) return;
  const int r = panel * kPanelRows + ln;
  bool bad = false;
  if constexpr (PAIR)
    out[(size_t)p * rows + r] = epi_gate_up(epi, acc0, acc1, bad);
  else
    out[(size_t)p * rows + r] = epi_down<FMT>(epi, acc0, bad);
  if (bad) flag(status, kStatusNonFinite);
}

// Weight steps in flight per wave: one 4 KiB BF16 step or two 1-2 KiB MX steps (more only
// costs registers: measured on MI355X, deeper rings were slower).
template <int FMT, bool PAIR>
constexpr int gemv_depth() {
  return FMT == kFmtBF16 ? 1 : 2;
}

template <int FMT, bool PAIR>
static void launch_gemv(const ExpertMats* mats, const Perm& perm, int max_active, int rows,
                        int cols, const float* in, float* out, Epi epi, int* status,
                        hipStream_t s) {
  constexpr int D = gemv_depth<FMT, PAIR>();
  const int panels = rows / kPanelRows, steps = cols / kGemmKStep;
  // Split K until the launch has ~4096 waves (16 per CU), keeping at least DEPTH steps per part.
  int ksplit = 1;
  while (ksplit < 4 && (long)panels * max_active * ksplit < 4096 && steps / (2 * ksplit) >= D)
    ksplit *= 2;
  const int ppw = 4 / ksplit;
  dim3 grid((panels + ppw - 1) / ppw, max_active);
  const size_t lds = (xs_floats(cols) + 4 * 16 * 2) * sizeof(float);
  gemv_kernel<FMT, PAIR, D><<<grid, 256, lds, s>>>(mats, perm, rows, cols, ksplit, in, out, epi,
                                                   status);
}

void launch_gemv_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                         int H, int I, const float* x, float* act, Epi epi, int* status,
                         hipStream_t s) {
  if (fmt == kFmtBF16) launch_gemv<kFmtBF16, true>(mats, perm, max_active, I, H, x, act, epi, status, s);
  else if (fmt == kFmtMXFP4) launch_gemv<kFmtMXFP4, true>(mats, perm, max_active, I, H, x, act, epi, status, s);
  else launch_gemv<kFmtMXFP8, true>(mats, perm, max_active, I, H, x, act, epi, status, s);
}

void launch_gemv_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_active, int H,
                      int I, const float* act, float* y, Epi epi, int* status, hipStream_t s) {
  if (fmt == kFmtBF16) launch_gemv<kFmtBF16, false>(mats, perm, max_active, H, I, act, y, epi, status, s);
  else if (fmt == kFmtMXFP4) launch_gemv<kFmtMXFP4, false>(mats, perm, max_active, H, I, act, y, epi, status, s);
  else launch_gemv<kFmtMXFP8, false>(mats, perm, max_active, H, I, act, y, epi, status, s);
}

// ------------------------------------------------------------------------------------------
// Decode down projection fused with the combine (one token).  A workgroup owns one 16-row
// panel of the output and computes it for every routed expert (wave w takes slots w, w + W,
// ...), with all k SwiGLU activation rows staged in LDS.  The k partial rows meet in LDS and 16
// threads apply the down epilogue and combine them in the composition's order, so the per-slot
// outputs never leave the chip and no combine kernel runs.  (Splitting K over two waves per
// slot, for twice the waves, measured slower.)  `comp` = URB composition (0 QWEN36, 1 GLM,
// 2 HY4, 3 DSV41).
// ------------------------------------------------------------------------------------------
template <int FMT, int DEPTH>
__global__ __launch_bounds__(512) void gemv_down_combine_kernel(
    const ExpertMats* __restrict__ mats, const int32_t* __restrict__ ids,
    const float* __restrict__ w, const int32_t* __restrict__ asc, int K, int H, int I,
    const float* __restrict__ act, const float* __restrict__ shared, int comp, Epi epi,
    const float* __restrict__ residual, const float* __restrict__ gate, float* __restrict__ out,
    int* status) {
  extern __shared__ float xs[];  // K x xs_floats(I) staged activations, then [K][16] sums
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ln = lane & 15, lq = lane >> 4;
  const int S = blockDim.x >> 6;
  const int panel = blockIdx.x;
  const int steps = I / kGemmKStep;
  const size_t xf = xs_floats(I);
  const size_t pbytes = kPanelRows * panel_row_bytes<FMT>(I);
  const size_t pscales = (size_t)kPanelRows * (I / 32);
  float* red = xs + (size_t)K * xf;

  // the first slot's first weight steps go out before the activations are staged
  BRaw<FMT> r[DEPTH];
  const uint8_t *pd = nullptr, *ps = nullptr;
  auto bind = [&](int a) {
    const ExpertMats m = mats[ids[a]];
    pd = m.data[2] + (size_t)panel * pbytes + 16 * lane;
    ps = FMT == kFmtBF16 ? nullptr : m.scales[2] + (size_t)panel * pscales + lane;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (d < steps) load_b<FMT, true>(r[d], pd, ps, d);
  };
  const int a0 = wave;
  if (a0 < K) bind(a0);
  for (int i = threadIdx.x; i < K * (I / 4); i += blockDim.x) {
    const int a = i / (I / 4), c4 = i - a * (I / 4);
    *reinterpret_cast<float4*>(xs + a * xf + xs_index(4 * c4)) =
        reinterpret_cast<const float4*>(act + (size_t)a * I)[c4];
  }
  __syncthreads();

  for (int a = a0; a < K; a += S) {
    if (a != a0) bind(a);
    const float* xa = xs + a * xf;
    float acc = 0.0f;
    for (int s0 = 0; s0 < steps; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int st = s0 + d;
        if (st >= steps) break;
        BRaw<FMT> c = r[d];
        if (st + DEPTH < steps) load_b<FMT, true>(r[d], pd, ps, st + DEPTH);
        raw_dot<FMT>(c, st, lq, xa, acc);
      }
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (lane < 16) red[a * 16 + ln] = acc;
  }
  __syncthreads();

  if (threadIdx.x < 16) {
    const int row = panel * kPanelRows + threadIdx.x;
    bool bad = false;
    auto y = [&](int a) { return epi_down<FMT>(epi, red[a * 16 + threadIdx.x], bad); };
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

// Largest LDS the fused kernel stages (k activation rows); above it the down projection and the
// combine run as separate kernels.
constexpr size_t kFusedLdsBytes = 96 * 1024;

size_t down_combine_lds(int K, int I) {
  return ((size_t)K * xs_floats(I) + (size_t)K * 16) * sizeof(float);
}

bool down_combine_fits(int K, int I) { return K <= 32 && down_combine_lds(K, I) <= kFusedLdsBytes; }

bool launch_gemv_down_combine(int fmt, const ExpertMats* mats, const int32_t* ids,
                              const float* weights, const int32_t* asc, int K, int H, int I,
                              const float* act, const float* shared, int comp, Epi epi,
                              float* out, int* status, hipStream_t s, const float* residual,
                              const float* gate) {
  if (!down_combine_fits(K, I)) return false;
  const size_t lds = down_combine_lds(K, I);
  const dim3 grid(H / kPanelRows), block(64 * std::min(K, 8));
  auto go = [&](auto kernel) {
    // dynamic LDS beyond 64 KiB must be allowed per kernel
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFusedLdsBytes);
    kernel<<<grid, block, lds, s>>>(mats, ids, weights, asc, K, H, I, act, shared, comp, epi,
                                    residual, gate, out, status);
  };
  if (fmt == kFmtBF16) go(gemv_down_combine_kernel<kFmtBF16, 1>);
  else if (fmt == kFmtMXFP4) go(gemv_down_combine_kernel<kFmtMXFP4, 2>);
  else go(gemv_down_combine_kernel<kFmtMXFP8, 2>);
  return true;
}

// ------------------------------------------------------------------------------------------
// Combines.
// Qwen (src/models/qwen3_6/runtime.rs:1398-1415): routes in ascending expert id,
//   c = bf16(w * y), acc = bf16(acc + c), acc from +0.0.
// GLM (src/models/glm/runtime/moe.rs:162-171): acc = f64(shared) (or 0), then in ranking
//   order acc += f64(w) * f64(y); out = f32(acc).
// ------------------------------------------------------------------------------------------
template <int KMAX>
__global__ __launch_bounds__(256) void combine_qwen_kernel(const float* __restrict__ y,
                                                           const int32_t* __restrict__ pos,
                                                           const float* __restrict__ w,
                                                           const int32_t* __restrict__ asc,
                                                           int T, int K, int H,
                                                           const float* __restrict__ res,
                                                           const float* __restrict__ shared,
                                                           const float* __restrict__ gate,
                                                           float* __restrict__ out,
                                                           int* status) {
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (h4 * 4 >= H) return;
  // all route metadata first, then every expert row: two dependent round trips in total
  int rk[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) rk[j] = j < K ? asc[(size_t)t * K + j] : 0;
  float wt[KMAX];
  float4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      wt[j] = w[(size_t)t * K + rk[j]];
      const int p = pos ? pos[(size_t)t * K + rk[j]] : rk[j];
      v[j] = reinterpret_cast<const float4*>(y + (size_t)p * H)[h4];
    }
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool bad = false;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      const float vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float c;
        if (!rne_bf16(wt[j] * vv[u], &c)) { bad = true; c = wt[j] * vv[u]; }
        const float s = acc[u] + c;
        if (!rne_bf16(s, &acc[u])) { bad = true; acc[u] = s; }
      }
    }
  }
  if (shared) {
    // the gated shared expert, added last (src/models/qwen3_6/runtime.rs:1449-1461):
    // c = bf16(scale * s), acc = bf16(acc + c)
    const float sc = qwen_shared_scale(gate[t], bad);
    const float4 s4 = reinterpret_cast<const float4*>(shared + (size_t)t * H)[h4];
    const float ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float c;
      if (!rne_bf16(sc * ss[u], &c)) { bad = true; c = sc * ss[u]; }
      const float a = acc[u] + c;
      if (!rne_bf16(a, &acc[u])) { bad = true; acc[u] = a; }
    }
  }
  if (res) {
    // add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494)
    const float4 r4 = reinterpret_cast<const float4*>(res + (size_t)t * H)[h4];
    const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float s = rr[u] + acc[u];
      if (!rne_bf16(s, &acc[u])) { bad = true; acc[u] = s; }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
  reinterpret_cast<float4*>(out + (size_t)t * H)[h4] = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

template <int KMAX>
__global__ __launch_bounds__(256) void combine_glm_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ pos,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ shared,
                                                          int T, int K, int H,
                                                          float* __restrict__ out) {
  const int h4 = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (h4 * 4 >= H) return;
  float wt[KMAX];
  float4 v[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      wt[j] = w[(size_t)t * K + j];
      const int p = pos ? pos[(size_t)t * K + j] : j;
      v[j] = reinterpret_cast<const float4*>(y + (size_t)p * H)[h4];
    }
  }
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  if (shared) {
    const float4 s = reinterpret_cast<const float4*>(shared + (size_t)t * H)[h4];
    acc[0] = s.x; acc[1] = s.y; acc[2] = s.z; acc[3] = s.w;
  }
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < K) {
      const double wd = (double)wt[j];
      acc[0] += wd * (double)v[j].x;
      acc[1] += wd * (double)v[j].y;
      acc[2] += wd * (double)v[j].z;
      acc[3] += wd * (double)v[j].w;
    }
  }
  reinterpret_cast<float4*>(out + (size_t)t * H)[h4] =
      make_float4((float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]);
}

void launch_combine_qwen(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                         const int32_t* asc, int T, int K, int H, float* out, int* status,
                         hipStream_t s, const float* residual, const float* shared,
                         const float* gate) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_qwen_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H,
                                                residual, shared, gate, out, status);
  else
    combine_qwen_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H,
                                                 residual, shared, gate, out, status);
}

void launch_combine_glm(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                        const float* shared, int T, int K, int H, float* out, hipStream_t s) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_glm_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, shared, T, K, H, out);
  else
    combine_glm_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, shared, T, K, H,
                                                out);
}

// ------------------------------------------------------------------------------------------
// Payload validation (one pass at create):
//   BF16  any element with an all-ones exponent (src/model/bf16.rs:743-773)     -> bit 1
//   MXFP8 any E4M3 code with magnitude 0x7F (src/math/mxfp.rs:880-888)          -> bit 1
//   MX    any E8M0 scale 0xFF (src/math/mxfp.rs:890-898, 1431-1435)             -> bit 2
// ------------------------------------------------------------------------------------------
__global__ void validate_kernel(int fmt, const uint8_t* __restrict__ data, size_t nbytes,
                                const uint8_t* __restrict__ scales, size_t sbytes, int* flags) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t tid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  int f = 0;
  if (fmt != kFmtMXFP4) {
    const size_t n4 = nbytes / 4;
    const uint32_t* d4 = reinterpret_cast<const uint32_t*>(data);
    for (size_t i = tid; i < n4; i += stride) {
      uint32_t v = d4[i];
      if (fmt == kFmtBF16) {
        if ((v & 0x7f80u) == 0x7f80u || ((v >> 16) & 0x7f80u) == 0x7f80u) f |= 1;
      } else {
        for (int b = 0; b < 4; ++b)
          if (((v >> (8 * b)) & 0x7fu) == 0x7fu) f |= 1;
      }
    }
    for (size_t i = n4 * 4 + tid; i < nbytes; i += stride) {
      if (fmt == kFmtBF16) {
        // a dangling half of a BF16 element cannot occur (nbytes is even and 4-aligned rows)
      } else if ((data[i] & 0x7fu) == 0x7fu) {
        f |= 1;
      }
    }
  }
  for (size_t i = tid; i < sbytes; i += stride)
    if (scales[i] == 0xffu) f |= 2;
  if (f) atomicOr(flags, f);
}

void launch_validate(int fmt, const uint8_t* data, size_t data_bytes, const uint8_t* scales,
                     size_t scale_bytes, int* flags, hipStream_t s) {
  size_t work = std::max(data_bytes / 4, scale_bytes);
  int blocks = (int)std::min<size_t>(std::max<size_t>((work + 255) / 256, 1), 4096);
  validate_kernel<<<blocks, 256, 0, s>>>(fmt, data, data_bytes, scales, scale_bytes, flags);
}

// Dequantised rows, value = decode(code) * scale in f32 (bit-exact parity hook).
__global__ void dequant_kernel(int fmt, const uint8_t* __restrict__ data,
                               const uint8_t* __restrict__ scales, int cols, int row0, int count,
                               float* __restrict__ out) {
  const size_t n = (size_t)count * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = row0 + i / cols;
    const int c = (int)(i % cols);
    float v;
    if (fmt == kFmtBF16) {
      const uint16_t* d = reinterpret_cast<const uint16_t*>(data);
      v = u2f((uint32_t)d[r * cols + c] << 16);
    } else if (fmt == kFmtMXFP4) {
      uint32_t byte = data[r * (cols / 2) + c / 2];
      f32x2 pair = fp4x2<0>(byte);
      // The conversion yields -0.0 for code 8; the reference table holds +0.0 there
      // (src/math/mxfp.rs:73-79).  Adding +0.0 maps -0.0 to +0.0 and leaves the rest exact.
      v = (pair[c & 1] + 0.0f) * e8m0_to_f32(scales[r * (cols / 32) + c / 32]);
    } else {
      uint32_t byte = data[r * cols + c];
      f32x2 pair = fp8x2<false>(byte);
      v = pair[0] * e8m0_to_f32(scales[r * (cols / 32) + c / 32]);
    }
    out[i] = v;
  }
}

void launch_dequant(int fmt, const uint8_t* data, const uint8_t* scales, int rows, int cols,
                    int row0, int count, float* out, hipStream_t s) {
  (void)rows;
  size_t n = (size_t)count * cols;
  int blocks = (int)std::min<size_t>((n + 255) / 256, 16384);
  dequant_kernel<<<std::max(blocks, 1), 256, 0, s>>>(fmt, data, scales, cols, row0, count, out);
}

__global__ void fill_i32_kernel(int32_t* p, int32_t v, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

void launch_fill_i32(int32_t* p, int32_t v, size_t n, hipStream_t s) {
  int blocks = (int)std::min<size_t>(std::max<size_t>((n + 255) / 256, 1), 1024);
  fill_i32_kernel<<<blocks, 256, 0, s>>>(p, v, n);
}

__global__ void check_finite_kernel(const float* __restrict__ x, size_t n, int* status) {
  bool bad = false;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    bad |= !finite(x[i]);
  if (bad) flag(status, kStatusNonFinite);
}

void launch_check_finite(const float* x, size_t n, int* status, hipStream_t s) {
  int blocks = (int)std::min<size_t>(std::max<size_t>((n + 255) / 256, 1), 1024);
  check_finite_kernel<<<blocks, 256, 0, s>>>(x, n, status);
}

}  // namespace urb
