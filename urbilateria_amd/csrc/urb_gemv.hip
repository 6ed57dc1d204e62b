// urb_gemv.hip -- decode-path expert projections, combines, validation and dequantisation.
//
// Decode projections are matrix-vector products over the rows of each active expert.  A
// wavefront splits into 64/LPR row groups of LPR lanes; each lane walks the row in "chunks"
// (BF16: 8 columns = 16 B; MXFP4: 32 columns = 16 B of nibbles + one E8M0 byte; MXFP8: 32
// columns = 32 B + one E8M0 byte) with 128-bit loads, decodes in registers (CDNA4
// v_cvt_scalef32_pk_f32_fp4/fp8), and FMA-accumulates against the input vector staged in LDS.
// MX chunks accumulate sum(code * x) in f32 and apply the power-of-two scale once per chunk,
// which is exact multiplication by 2^k of the chunk partial.
#include "urb_device.hpp"
#include "urb_kernels.hpp"

#include <algorithm>

namespace urb {

enum { kFmtBF16 = 0, kFmtMXFP4 = 1, kFmtMXFP8 = 2 };

template <int FMT>
struct Fmt;
template <>
struct Fmt<kFmtBF16> {
  static constexpr int kCols = 8;  // columns per chunk
  __device__ static size_t row_bytes(int cols) { return (size_t)cols * 2; }
};
template <>
struct Fmt<kFmtMXFP4> {
  static constexpr int kCols = 32;
  __device__ static size_t row_bytes(int cols) { return (size_t)cols / 2; }
};
template <>
struct Fmt<kFmtMXFP8> {
  static constexpr int kCols = 32;
  __device__ static size_t row_bytes(int cols) { return (size_t)cols; }
};

// One lane's chunk of a weight row, loaded ahead of its use.
template <int FMT>
struct Chunk;
template <>
struct Chunk<kFmtBF16> { uint4 q; };
template <>
struct Chunk<kFmtMXFP4> { uint4 q; uint32_t s; };
template <>
struct Chunk<kFmtMXFP8> { uint4 q0, q1; uint32_t s; };
// Chunks a lane loads before computing on them (a batch of independent 128-bit loads).
template <int FMT>
constexpr int kBatch = FMT == kFmtBF16 ? 8 : 4;

template <int FMT>
__device__ __forceinline__ void chunk_load(Chunk<FMT>& c, const uint8_t* __restrict__ row,
                                           const uint8_t* __restrict__ srow, int g) {
  if constexpr (FMT == kFmtBF16) {
    c.q = *reinterpret_cast<const uint4*>(row + (size_t)g * 16);
  } else if constexpr (FMT == kFmtMXFP4) {
    c.q = *reinterpret_cast<const uint4*>(row + (size_t)g * 16);
    c.s = srow[g];
  } else {
    const uint4* qp = reinterpret_cast<const uint4*>(row + (size_t)g * 32);
    c.q0 = qp[0];
    c.q1 = qp[1];
    c.s = srow[g];
  }
}

// acc += chunk . xs[g * kCols ...]
template <int FMT>
__device__ __forceinline__ void chunk_dot(const Chunk<FMT>& c, int g,
                                          const float* __restrict__ xs, float& acc) {
  if constexpr (FMT == kFmtBF16) {
    const uint4 q = c.q;
    const float4* xv = reinterpret_cast<const float4*>(xs + g * 8);
    float4 a = xv[0], b = xv[1];
    float p0 = bf16_lo(q.x) * a.x, p1 = bf16_hi(q.x) * a.y;
    p0 = fmaf(bf16_lo(q.y), a.z, p0);
    p1 = fmaf(bf16_hi(q.y), a.w, p1);
    p0 = fmaf(bf16_lo(q.z), b.x, p0);
    p1 = fmaf(bf16_hi(q.z), b.y, p1);
    p0 = fmaf(bf16_lo(q.w), b.z, p0);
    p1 = fmaf(bf16_hi(q.w), b.w, p1);
    acc += p0 + p1;
  } else if constexpr (FMT == kFmtMXFP4) {
    const float scale = e8m0_to_f32(c.s);
    const float4* xv = reinterpret_cast<const float4*>(xs + g * 32);
    const uint32_t words[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
    float part[4];
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      float v[8];
      decode_fp4x8(words[wd], v);
      float4 a = xv[2 * wd], b = xv[2 * wd + 1];
      float p = v[0] * a.x;
      p = fmaf(v[1], a.y, p);
      p = fmaf(v[2], a.z, p);
      p = fmaf(v[3], a.w, p);
      p = fmaf(v[4], b.x, p);
      p = fmaf(v[5], b.y, p);
      p = fmaf(v[6], b.z, p);
      p = fmaf(v[7], b.w, p);
      part[wd] = p;
    }
    acc = fmaf((part[0] + part[1]) + (part[2] + part[3]), scale, acc);
  } else {
    const float scale = e8m0_to_f32(c.s);
    const float4* xv = reinterpret_cast<const float4*>(xs + g * 32);
    const uint32_t words[8] = {c.q0.x, c.q0.y, c.q0.z, c.q0.w, c.q1.x, c.q1.y, c.q1.z, c.q1.w};
    float part[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float v[8];
      decode_fp8x4(words[2 * h], v);
      decode_fp8x4(words[2 * h + 1], v + 4);
      float4 a = xv[2 * h], b = xv[2 * h + 1];
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

// Resolves (active slot, token ordinal) -> expert, permuted position and token.
__device__ __forceinline__ bool perm_expert(const Perm& perm, int a, int& expert, int& base,
                                            int& count) {
  if (perm.dense_tokens > 0) {
    if (a != 0) return false;
    expert = 0;
    base = 0;
    count = perm.dense_tokens;
    return true;
  }
  if (a >= perm.meta[0]) return false;
  expert = perm.active[a];
  base = perm.offsets[expert];
  count = perm.counts[expert];
  return true;
}
__device__ __forceinline__ int perm_token(const Perm& perm, int p) {
  return perm.dense_tokens > 0 ? p : perm.perm_token[p];
}

__device__ __forceinline__ void stage(const float* __restrict__ src, int n, float* xs) {
  const float4* s4 = reinterpret_cast<const float4*>(src);
  float4* d4 = reinterpret_cast<float4*>(xs);
  for (int i = threadIdx.x; i < n / 4; i += blockDim.x) d4[i] = s4[i];
}

// PAIR = gate+up rows with the SwiGLU epilogue (rows I, cols H, input x[token]);
// otherwise down rows (rows H, cols I, input act[position]).
template <int FMT, int LPR, bool PAIR>
__global__ __launch_bounds__(256) void gemv_kernel(const ExpertMats* __restrict__ mats,
                                                   Perm perm, int rows, int cols,
                                                   int rows_per_block,
                                                   const float* __restrict__ in,
                                                   float* __restrict__ out, int qwen,
                                                   int* status) {
  extern __shared__ float xs[];
  const int nrb = (rows + rows_per_block - 1) / rows_per_block;
  const int a = blockIdx.x / nrb, rb = blockIdx.x - a * nrb;
  int expert, base, count;
  if (!perm_expert(perm, a, expert, base, count)) return;
  const ExpertMats m = mats[expert];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, li = lane % LPR;
  constexpr int kGroups = 64 / LPR;
  const int G = cols / Fmt<FMT>::kCols;
  const size_t rbytes = Fmt<FMT>::row_bytes(cols);
  const int sbytes = cols / 32;
  const int r_begin = rb * rows_per_block;
  const int r_end = min(rows, r_begin + rows_per_block);
  bool bad = false;
  constexpr int NB = kBatch<FMT>;
  const int r_first = r_begin + wave * kGroups + sub;
  for (int q = 0; q < count; ++q) {
    const int p = base + q;
    const float* src = PAIR ? in + (size_t)perm_token(perm, p) * cols : in + (size_t)p * cols;
    // The first batch of this lane's weights is requested before the input vector is staged,
    // so the two memory latencies overlap.
    Chunk<FMT> c0[NB], c1[NB];
    bool have = r_first < r_end;
    if (have) {
      const uint8_t* row0 = m.data[PAIR ? 0 : 2] + (size_t)r_first * rbytes;
      const uint8_t* s0 =
          FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + (size_t)r_first * sbytes;
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int g = li + u * LPR;
        if (g < G) {
          chunk_load<FMT>(c0[u], row0, s0, g);
          if constexpr (PAIR)
            chunk_load<FMT>(c1[u], m.data[1] + (size_t)r_first * rbytes,
                            FMT == kFmtBF16 ? nullptr
                                            : m.scales[1] + (size_t)r_first * sbytes,
                            g);
        }
      }
    }
    __syncthreads();
    stage(src, cols, xs);
    __syncthreads();
    for (int r = r_first; r < r_end; r += 4 * kGroups) {
      float acc0 = 0.0f, acc1 = 0.0f;
      const uint8_t* row0 = m.data[PAIR ? 0 : 2] + (size_t)r * rbytes;
      const uint8_t* s0 = FMT == kFmtBF16 ? nullptr : m.scales[PAIR ? 0 : 2] + (size_t)r * sbytes;
      const uint8_t* row1 = PAIR ? m.data[1] + (size_t)r * rbytes : nullptr;
      const uint8_t* s1 = (PAIR && FMT != kFmtBF16) ? m.scales[1] + (size_t)r * sbytes : nullptr;
      for (int g0 = li; g0 < G; g0 += NB * LPR) {
        if (!have) {
#pragma unroll
          for (int u = 0; u < NB; ++u) {
            const int g = g0 + u * LPR;
            if (g < G) {
              chunk_load<FMT>(c0[u], row0, s0, g);
              if constexpr (PAIR) chunk_load<FMT>(c1[u], row1, s1, g);
            }
          }
        }
        have = false;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const int g = g0 + u * LPR;
          if (g < G) {
            chunk_dot<FMT>(c0[u], g, xs, acc0);
            if constexpr (PAIR) chunk_dot<FMT>(c1[u], g, xs, acc1);
          }
        }
      }
      acc0 = wave_sum_f32(acc0, LPR);
      if constexpr (PAIR) acc1 = wave_sum_f32(acc1, LPR);
      if (li == 0) {
        if constexpr (PAIR) {
          // Qwen38Expert (src/models/qwen3_8/expert.rs:137-207): g, u, silu(g), g*u in BF16.
          // GatedMlp (src/model/mlp.rs:90-99): silu(g) * u in f32; a non-finite activation
          // is rejected by the down projection's input check.
          float act;
          if (qwen) {
            float g, u, ag, v;
            bool ok = rne_bf16(acc0, &g) && rne_bf16(acc1, &u) && rne_bf16(silu(g), &ag);
            v = ag * u;
            ok = ok && rne_bf16(v, &act);
            if (!ok) { bad = true; act = v; }
          } else {
            act = silu(acc0) * acc1;
            if (!finite(act)) bad = true;
          }
          out[(size_t)p * rows + r] = act;
        } else {
          float y = acc0;
          if (qwen) {
            float rr;
            if (!rne_bf16(y, &rr)) bad = true; else y = rr;
          } else if (FMT == kFmtMXFP8 && !finite(y)) {
            bad = true;  // MxFp8Matrix::matvec_rows rejects non-finite outputs (mxfp.rs:779-781)
          }
          out[(size_t)p * rows + r] = y;
        }
      }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
}

template <int FMT, bool PAIR>
static void launch_gemv(const ExpertMats* mats, const Perm& perm, int max_active, int rows,
                        int cols, const float* in, float* out, int qwen, int* status,
                        hipStream_t s) {
  const int G = cols / Fmt<FMT>::kCols;
  // Lanes per row: the widest split that leaves every lane at least 2 chunks.
  int lpr = 64;
  while (lpr > 16 && G < 2 * lpr) lpr /= 2;
  // Rows per workgroup: ~2048 workgroups to cover every CU several times, with at least 2x the
  // staged input vector's bytes of weights per workgroup and at most 8 row passes per wave.
  const int rows_per_pass = 4 * (64 / lpr);
  const long row_bytes = (long)cols * (FMT == kFmtBF16 ? 2 : 1) / (FMT == kFmtMXFP4 ? 2 : 1) *
                         (PAIR ? 2 : 1);
  const long reuse_rows = (2L * cols * 4 + row_bytes - 1) / row_bytes;
  const long spread_rows = ((long)rows * max_active + 2047) / 2048;
  const long want = std::max(reuse_rows, spread_rows);
  const int passes = (int)std::max(1L, std::min(8L, (want + rows_per_pass - 1) / rows_per_pass));
  const int rows_per_block = rows_per_pass * passes;
  const int nrb = (rows + rows_per_block - 1) / rows_per_block;
  dim3 grid(max_active * nrb);
  size_t lds = (size_t)cols * sizeof(float);
  switch (lpr) {
    case 64:
      gemv_kernel<FMT, 64, PAIR><<<grid, 256, lds, s>>>(mats, perm, rows, cols, rows_per_block,
                                                        in, out, qwen, status);
      break;
    case 32:
      gemv_kernel<FMT, 32, PAIR><<<grid, 256, lds, s>>>(mats, perm, rows, cols, rows_per_block,
                                                        in, out, qwen, status);
      break;
    default:
      gemv_kernel<FMT, 16, PAIR><<<grid, 256, lds, s>>>(mats, perm, rows, cols, rows_per_block,
                                                        in, out, qwen, status);
      break;
  }
}

void launch_gemv_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                         int H, int I, const float* x, float* act, int qwen, int* status,
                         hipStream_t s) {
  if (fmt == kFmtBF16) launch_gemv<kFmtBF16, true>(mats, perm, max_active, I, H, x, act, qwen, status, s);
  else if (fmt == kFmtMXFP4) launch_gemv<kFmtMXFP4, true>(mats, perm, max_active, I, H, x, act, qwen, status, s);
  else launch_gemv<kFmtMXFP8, true>(mats, perm, max_active, I, H, x, act, qwen, status, s);
}

void launch_gemv_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_active, int H,
                      int I, const float* act, float* y, int qwen, int* status, hipStream_t s) {
  if (fmt == kFmtBF16) launch_gemv<kFmtBF16, false>(mats, perm, max_active, H, I, act, y, qwen, status, s);
  else if (fmt == kFmtMXFP4) launch_gemv<kFmtMXFP4, false>(mats, perm, max_active, H, I, act, y, qwen, status, s);
  else launch_gemv<kFmtMXFP8, false>(mats, perm, max_active, H, I, act, y, qwen, status, s);
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
      const int p = pos[(size_t)t * K + rk[j]];
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
      const int p = pos[(size_t)t * K + j];
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
                         hipStream_t s) {
  dim3 grid((H / 4 + 255) / 256, T);
  if (K <= 8)
    combine_qwen_kernel<8><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H, out,
                                                status);
  else
    combine_qwen_kernel<32><<<grid, 256, 0, s>>>(y_perm, pos_of_slot, weights, asc, T, K, H, out,
                                                 status);
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
