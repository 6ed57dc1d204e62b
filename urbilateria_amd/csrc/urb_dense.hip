// urb_dense.hip -- the shared expert of a large batch: dense BF16 GEMMs on CDNA4 MFMA.
//
// C[T, N] = A[T, K] . W[N, K]^T with W a BF16 matrix in the panel layout (urb_kernels.hpp) and
// A f32 activations.  A workgroup of eight waves (two per SIMD, one workgroup per CU) owns a
// 256-token x 256-row tile and one of S equal K ranges (split K, so that the 1024 x 4096 shared
// gate/up of a 1024-token batch still gives 256 workgroups); each wave computes 128 tokens x 64
// rows with v_mfma_f32_16x16x32_bf16 (8 x 4 accumulator blocks, 128 accumulator registers).  Per 32-column K step both operands are
// staged in LDS in MFMA fragment order (1 KiB per 16 rows, lane l = row l % 16, columns
// 8 (l / 16) + [0, 8)), double buffered, from a register stage loaded two steps ahead:
//  * W: the panel layout's slabs are that fragment order already -- copied verbatim;
//  * A: each thread converts one token row's 32 values into BF16 hi + lo halves (16
//    significant bits, as the grouped GEMMs), and the lo MFMAs are skipped for a step whose lo
//    halves are all zero (BF16-valued activations).
// Against the grouped GEMM's 32-token dense tiles, every weight byte is read by 4 instead of 32
// tiles and every activation by 16 instead of 32.  The S partial sums [S, T, N] go to a
// workspace; the reduce kernels add them in order of K range (deterministic) and apply the
// gate/up epilogue (SwiGLU, the composition's boundaries) or the down epilogue.
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {

namespace {

constexpr int kDM = 256;       // tokens per tile
constexpr int kDN = 256;       // weight rows per tile
constexpr int kDK = 32;        // K per step (one MFMA)
constexpr int kDFrag = 512;    // u16 per 16-row fragment (1 KiB)

struct DenseLds {
  u16 a_hi[2][kDM / 16][kDFrag];
  u16 a_lo[2][kDM / 16][kDFrag];
  u16 b[2][kDN / 16][kDFrag];
  int lo_flag[2][8];
};

// Rows n0 .. n0 + 255 of the stacked matrix [W0; W1] (rows < n_split from W0): panel p's base.
__device__ __forceinline__ const uint8_t* dense_panel(const uint8_t* w0, const uint8_t* w1,
                                                      int n_split, size_t pbytes, int row) {
  return row < n_split ? w0 + (size_t)(row / kPanelRows) * pbytes
                       : w1 + (size_t)((row - n_split) / kPanelRows) * pbytes;
}

// LDS position of A fragment unit u (lane u of the MFMA operand): units 32..63 swap their
// quarters of 4, so the 8 consecutive threads that stage four rows (units r and r + 32 for four
// consecutive r) hit 8 distinct 16 B positions mod 8 (a conflict-free 16-byte store on MI355X),
// while each 16-lane read pass still covers 16 distinct bank slots.
__device__ __forceinline__ int a_swz(int u) { return u ^ ((u >> 5) << 2); }

// Tile placement: work item w = m + Mt (n + Nt z) (m fastest, so the m tiles that read the
// same weight rows and K range are consecutive); XCD c (block % 8) takes the contiguous run c of
// the items, so those tiles share its L2.
__device__ __forceinline__ bool dense_place(int block, int Mt, int Nt, int S, int* m, int* n,
                                            int* z) {
  const int total = Mt * Nt * S;
  const int xcd = block & 7, local = block >> 3;
  const int w = xcd * total / 8 + local;
  if (w >= (xcd + 1) * total / 8) return false;
  *m = w % Mt;
  *n = (w / Mt) % Nt;
  *z = w / (Mt * Nt);
  return true;
}

// A workgroup barrier that also ORs a per-thread flag over the eight waves of a 512-thread
// workgroup (one s_barrier; `slots`, 8 ints, double buffered with the data they describe).
__device__ __forceinline__ bool barrier_or8(bool pred, int* slots) {
  const bool any = __ballot(pred) != 0;
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = any;
  __syncthreads();
  const int4 v0 = *reinterpret_cast<const int4*>(slots);
  const int4 v1 = *reinterpret_cast<const int4*>(slots + 4);
  return (v0.x | v0.y | v0.z | v0.w | v1.x | v1.y | v1.z | v1.w) != 0;
}

__global__ __launch_bounds__(512, 1) void dense_gemm_kernel(
    const float* __restrict__ a, int T, int K, const uint8_t* __restrict__ w0,
    const uint8_t* __restrict__ w1, int n_split, int N, int S, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) DenseLds lds;
  const int Mt = (T + kDM - 1) / kDM, Nt = N / kDN;
  int mt, nt, z;
  if (!dense_place(blockIdx.x, Mt, Nt, S, &mt, &nt, &z)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;  // tokens 128 wm + [0, 128), rows 64 wn + [0, 64)
  const int ksteps = K / kDK;
  const int s_begin = ksteps * z / S, n_steps = ksteps * (z + 1) / S - s_begin;
  const size_t pbytes = (size_t)kPanelRows * K * 2;

  // ---- this thread's staging: half tid % 2 of token row m0 + tid / 2 (a row past T re-reads
  // row m0: its products land in accumulator rows that are never stored; two threads read one
  // 128-byte row segment), and two 16-byte units of the weight slabs: panel tid / 32, units
  // tid % 32 and tid % 32 + 32, so each group of 16 lanes writes 256 contiguous bytes of LDS.
  const int m0 = mt * kDM;
  const int tok = tid >> 1, half = tid & 1;
  const int arow = m0 + tok < T ? m0 + tok : m0;
  const float* a_src = a + (size_t)arow * K + 16 * half;
  const int bp = tid >> 5, bu = tid & 31;
  const uint8_t* b_src =
      dense_panel(w0, w1, n_split, pbytes, nt * kDN + bp * kPanelRows) + bu * 16;
  // LDS fragment slots of this thread's A values: block tok / 16, lanes (tok % 16) + 16 lq for
  // lq = 2 half, 2 half + 1
  const int a_blk = tok >> 4, a_ln = tok & 15;

  struct Stage {
    float4 a[4];
    uint4 b[2];
  };
  auto load = [&](Stage& st, int s) {
    const int k0 = (s_begin + s) * kDK;
    const float4* pa = reinterpret_cast<const float4*>(a_src + k0);
#pragma unroll
    for (int i = 0; i < 4; ++i) st.a[i] = pa[i];
    const uint8_t* pb = b_src + (size_t)(s_begin + s) * 1024;
#pragma unroll
    for (int i = 0; i < 2; ++i) st.b[i] = ldg16(pb + 512 * i);
  };
  // returns whether any lo half is non-zero
  auto store = [&](const Stage& st, int buf) {
    const float* v = reinterpret_cast<const float*>(st.a);
    uint32_t lor = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      uint32_t h[4], l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        split_bf16(v[8 * q + 2 * i], v[8 * q + 2 * i + 1], h[i], l[i]);
        lor |= l[i];
      }
      const int u = a_swz(a_ln + 16 * (2 * half + q));
      *reinterpret_cast<uint4*>(&lds.a_hi[buf][a_blk][8 * u]) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(&lds.a_lo[buf][a_blk][8 * u]) = make_uint4(l[0], l[1], l[2], l[3]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<uint4*>(&lds.b[buf][bp][8 * (bu + 32 * i)]) = st.b[i];
    return (lor & 0x7fff7fffu) != 0;
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mma = [&](int buf, bool with_lo) {
    bf16x8 bf[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      bf[nb] = __builtin_bit_cast(bf16x8,
                                  *reinterpret_cast<const uint4*>(&lds.b[buf][wn * 4 + nb][8 * lane]));
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const bf16x8 ah = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const uint4*>(&lds.a_hi[buf][wm * 8 + mb][8 * a_swz(lane)]));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bf[nb], acc[mb][nb], 0, 0, 0);
    }
    if (with_lo) {
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const bf16x8 al = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(&lds.a_lo[buf][wm * 8 + mb][8 * a_swz(lane)]));
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bf[nb], acc[mb][nb], 0, 0, 0);
      }
    }
  };

  // register stages two steps ahead, LDS double buffered; the steady state issues every load
  // unguarded (one issue order on every path, so the compiler's wait counts stay exact)
  Stage st[2];
  load(st[0], 0);
  if (n_steps > 1) load(st[1], 1);
  bool lo = barrier_or8(store(st[0], 0), lds.lo_flag[0]);
  int s = 0;
  for (; s + 4 <= n_steps; s += 2) {
    // step s from buffer 0, step s + 1 from buffer 1
    load(st[0], s + 2);
    mma(0, lo);
    lo = barrier_or8(store(st[1], 1), lds.lo_flag[1]);
    load(st[1], s + 3);
    mma(1, lo);
    lo = barrier_or8(store(st[0], 0), lds.lo_flag[0]);
  }
  // the last one to three steps (s is even: buffer 0 holds step s, st[1] step s + 1), with
  // compile-time stage indices (a runtime index would put the register stages in scratch)
  if (s < n_steps) {
    mma(0, lo);
    if (s + 1 < n_steps) {
      if (s + 2 < n_steps) load(st[0], s + 2);
      lo = barrier_or8(store(st[1], 1), lds.lo_flag[1]);
      mma(1, lo);
      if (s + 2 < n_steps) {
        lo = barrier_or8(store(st[0], 0), lds.lo_flag[0]);
        mma(0, lo);
      }
    }
  }

  // ---- the partial sums: lane holds rows (tokens) 4 lq + i, column (weight row) ln of each block
  const int ln = lane & 15, lq = lane >> 4;
  float* pz = part + (size_t)z * T * N;
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = m0 + wm * 128 + mb * 16 + 4 * lq + i;
      if (t >= T) continue;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        pz[(size_t)t * N + nt * kDN + wn * 64 + nb * 16 + ln] = acc[mb][nb][i];
    }
}

// ------------------------------------------------------------------------------------------
// The f16 down projection of the same batch: out[T, N] = A16[T, K] . W16[N, K]^T, A16 the
// SwiGLU rows as f16 at each row's scale (rowexp, dense_reduce_gate_up_f16_kernel) and W16 the
// f16 copy of the BF16 down matrix times 2^wshift (bf16_to_f16_kernel) in the panel layout.
// One f16 piece per value, so half the gate/up tile's MFMAs per byte staged: the tile is 128
// tokens x 256 rows (a 1024 x 7168 output gives 224 workgroups) and K is not split -- the
// epilogue scales each sum back (2^-(141 - rowexp) 2^-wshift, exact) and applies the down
// epilogue, with no partial sums and no reduce launch.  Eight waves of 64 tokens x 64 rows
// (4 x 4 accumulator blocks of v_mfma_f32_16x16x32_f16); both operands staged per 32-column K
// step in LDS in fragment order, double buffered, from registers loaded two steps ahead.
// ------------------------------------------------------------------------------------------
constexpr int kDM16 = 128;  // tokens per f16 down tile
constexpr int kDStages = 2;  // register stages of the f16 down tile (4 measured no faster)

struct DenseDownLds {
  u16 a[2][kDM16 / 16][kDFrag];
  u16 b[2][kDN / 16][kDFrag];
  int sh[kDM16];  // the tile's rows' epilogue shifts
};

__global__ __launch_bounds__(512, 1) void dense_down_f16_kernel(
    const u16* __restrict__ a16, const int* __restrict__ rowexp, int T, int K,
    const uint8_t* __restrict__ w16, int N, Epi epi, float* __restrict__ out, int* status) {
  __shared__ __attribute__((aligned(16))) DenseDownLds lds;
  const int Mt = (T + kDM16 - 1) / kDM16, Nt = N / kDN;
  int mt, nt, z;
  if (!dense_place(blockIdx.x, Mt, Nt, 1, &mt, &nt, &z)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;  // tokens 64 wm + [0, 64), rows 64 wn + [0, 64)
  const int ksteps = K / kDK;
  const size_t pbytes = (size_t)kPanelRows * K * 2;

  // ---- staging: A unit (row, k-quad c) per thread, 8 consecutive threads on 8 consecutive
  // rows of one k-quad (eight distinct 16-byte LDS positions mod 16: no store conflict; a
  // row past T re-reads row m0, whose products land in rows never stored); B as the gate/up
  // tile: panel tid / 32, units tid % 32 and tid % 32 + 32.
  const int m0 = mt * kDM16;
  const int c = (tid >> 3) & 3, tok = (tid & 7) + 8 * (tid >> 5);
  const int arow = m0 + tok < T ? m0 + tok : m0;
  const u16* a_src = a16 + (size_t)arow * K + 8 * c;
  const int a_blk = tok >> 4, a_unit = (tok & 15) + 16 * c;
  const int bp = tid >> 5, bu = tid & 31;
  const uint8_t* b_src = w16 + (size_t)(nt * (kDN / kPanelRows) + bp) * pbytes + bu * 16;

  struct Stage {
    uint4 a;
    uint4 b[2];
  };
  auto load = [&](Stage& st, int s) {
    st.a = ldg16(a_src + s * kDK);
    const uint8_t* pb = b_src + (size_t)s * 1024;
#pragma unroll
    for (int i = 0; i < 2; ++i) st.b[i] = ldg16(pb + 512 * i);
  };
  auto store = [&](const Stage& st, int buf) {
    *reinterpret_cast<uint4*>(&lds.a[buf][a_blk][8 * a_unit]) = st.a;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<uint4*>(&lds.b[buf][bp][8 * (bu + 32 * i)]) = st.b[i];
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](int buf) {
    f16x8 bf[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      bf[nb] = __builtin_bit_cast(f16x8,
                                  *reinterpret_cast<const uint4*>(&lds.b[buf][wn * 4 + nb][8 * lane]));
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const f16x8 af = __builtin_bit_cast(
          f16x8, *reinterpret_cast<const uint4*>(&lds.a[buf][wm * 4 + mb][8 * lane]));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[nb], acc[mb][nb], 0, 0, 0);
    }
  };

  // kDStages register stages (step s + kDStages loads while step s computes; its data has
  // kDStages - 1 steps to arrive before it is stored), LDS double buffered, one barrier per
  // step.  The steady state's loop has no exit between its steps and issues every load
  // unguarded, so that the compiler's wait counts follow one issue order on every path; the
  // last steps run in an unrolled tail.
  // each row's epilogue shift (2^-(141 - rowexp) 2^-wshift), read from LDS by the epilogue
  if (tid < kDM16) lds.sh[tid] = rowexp[min(m0 + tid, T - 1)] - 141 - epi.wshift;
  Stage st[kDStages];
#pragma unroll
  for (int i = 0; i < kDStages; ++i)
    if (i < ksteps) load(st[i], i);
  store(st[0], 0);
  __syncthreads();
  int s = 0;
  for (; s + 2 * kDStages <= ksteps; s += kDStages) {
#pragma unroll
    for (int d = 0; d < kDStages; ++d) {
      load(st[d], s + d + kDStages);               // st[d] held step s + d, stored last step
      mma(d & 1);                                  // step s + d
      store(st[(d + 1) % kDStages], (d + 1) & 1);  // step s + d + 1 into the other buffer
      __syncthreads();
    }
  }
#pragma unroll
  for (int d = 0; d < 2 * kDStages; ++d) {
    const int step = s + d;
    if (step >= ksteps) break;
    if (step + kDStages < ksteps) load(st[d % kDStages], step + kDStages);
    mma(d & 1);
    if (step + 1 < ksteps) {
      store(st[(d + 1) % kDStages], (d + 1) & 1);
      __syncthreads();
    }
  }

  // ---- epilogue: lane holds tokens 4 lq + i, row ln of each block
  const int ln = lane & 15, lq = lane >> 4;
  bool bad = false;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = m0 + wm * 64 + mb * 16 + 4 * lq + i;
      if (t >= T) continue;
      const int sh = lds.sh[t - m0];
      float* o = out + (size_t)t * N + nt * kDN + wn * 64 + ln;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const float v = epi_down<kFmtBF16>(epi, ldexpf(acc[mb][nb][i], sh), bad);
        if (epi.stream_out) __builtin_nontemporal_store(v, o + nb * 16);
        else o[nb * 16] = v;
      }
    }
  if (bad) flag(status, kStatusNonFinite);
}

// act[t, j] = epi_gate_up(sum_z gate partial, sum_z up partial): the gate rows are columns
// 0..I-1 of the partial sums, the up rows columns I..2I-1.  Four consecutive j per thread
// (I % 4 == 0), the K parts added in order.
__global__ void dense_reduce_gate_up_kernel(const float* __restrict__ part, int T, int I, int S,
                                            Epi epi, float* __restrict__ act, int* status) {
  const size_t n4 = (size_t)T * I / 4, stride = (size_t)T * 2 * I;
  bool bad = false;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t e = 4 * i, t = e / I, j = e - t * I;
    const float* p = part + t * 2 * I + j;
    float g[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int z = 0; z < S; ++z) {
      const float4 a = *reinterpret_cast<const float4*>(p + z * stride);
      const float4 b = *reinterpret_cast<const float4*>(p + z * stride + I);
      g[0] += a.x; g[1] += a.y; g[2] += a.z; g[3] += a.w;
      u[0] += b.x; u[1] += b.y; u[2] += b.z; u[3] += b.w;
    }
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = epi_gate_up(epi, g[k], u[k], bad);
    *reinterpret_cast<float4*>(act + e) = make_float4(o[0], o[1], o[2], o[3]);
  }
  if (bad) flag(status, kStatusNonFinite);
}

// The same sums and SwiGLU for one token row per workgroup, written as f16 times 2^(141 - e),
// e = the largest exponent field of the row's values (its largest |value| then lies in
// [2^14, 2^15)), and e in rowexp[t]: the input of an f16 down projection (Epi::rowexp with one
// group).  The row's values wait in LDS (I floats) while the workgroup finds e.
__global__ __launch_bounds__(256) void dense_reduce_gate_up_f16_kernel(
    const float* __restrict__ part, int T, int I, int S, Epi epi, u16* __restrict__ act16,
    int* __restrict__ rowexp, int* status) {
  extern __shared__ float4 rowv[];  // I / 4
  __shared__ int emax;
  const int t = blockIdx.x;
  const size_t stride = (size_t)T * 2 * I;
  const float* p = part + (size_t)t * 2 * I;
  if (threadIdx.x == 0) emax = 0;
  __syncthreads();
  bool bad = false;
  int e = 0;
  for (int j = 4 * threadIdx.x; j < I; j += 4 * blockDim.x) {
    float g[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int z = 0; z < S; ++z) {
      const float4 a = *reinterpret_cast<const float4*>(p + z * stride + j);
      const float4 b = *reinterpret_cast<const float4*>(p + z * stride + I + j);
      g[0] += a.x; g[1] += a.y; g[2] += a.z; g[3] += a.w;
      u[0] += b.x; u[1] += b.y; u[2] += b.z; u[3] += b.w;
    }
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[k] = epi_gate_up(epi, g[k], u[k], bad);
      e = max(e, (int)((__float_as_uint(o[k]) >> 23) & 0xffu));
    }
    rowv[j / 4] = make_float4(o[0], o[1], o[2], o[3]);
  }
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) e = max(e, __shfl_xor(e, x));
  if ((threadIdx.x & 63) == 0) atomicMax(&emax, e);
  __syncthreads();
  const int sh = 141 - emax;
  u16* out = act16 + (size_t)t * I;
  for (int j = 4 * threadIdx.x; j < I; j += 4 * blockDim.x) {
    const float4 v = rowv[j / 4];
    const _Float16 h[4] = {(_Float16)ldexpf(v.x, sh), (_Float16)ldexpf(v.y, sh),
                           (_Float16)ldexpf(v.z, sh), (_Float16)ldexpf(v.w, sh)};
    *reinterpret_cast<uint2*>(out + j) = __builtin_bit_cast(uint2, h);
  }
  if (threadIdx.x == 0) rowexp[t] = emax;
  if (bad) flag(status, kStatusNonFinite);
}

// Exponent fields of a BF16 matrix's non-zero values (subnormals as 1): range[0] = min,
// range[1] = max (pre-set to 255 and 0).  Eight values per thread and load; one pair of atomics
// per workgroup.
__global__ __launch_bounds__(256) void bf16_exp_range_kernel(const uint16_t* __restrict__ w,
                                                             size_t n, int* range) {
  __shared__ int lo_s, hi_s;
  if (threadIdx.x == 0) {
    lo_s = 255;
    hi_s = 0;
  }
  __syncthreads();
  int lo = 255, hi = 0;
  auto take = [&](uint32_t u) {
    if ((u & 0x7fffu) == 0) return;
    const int e = max((int)((u >> 7) & 0xffu), 1);
    lo = min(lo, e);
    hi = max(hi, e);
  };
  const size_t n8 = n / 8;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint4 q = *reinterpret_cast<const uint4*>(w + 8 * i);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      take(v[k] & 0xffffu);
      take(v[k] >> 16);
    }
  }
  for (size_t i = 8 * n8 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    take(w[i]);
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) {
    lo = min(lo, __shfl_xor(lo, x));
    hi = max(hi, __shfl_xor(hi, x));
  }
  if ((threadIdx.x & 63) == 0) {
    atomicMin(&lo_s, lo);
    atomicMax(&hi_s, hi);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicMin(&range[0], lo_s);
    atomicMax(&range[1], hi_s);
  }
}

// BF16 values times 2^shift as f16 (exact for the shifts bf16_f16_shift returns).
__global__ void bf16_to_f16_kernel(const uint16_t* __restrict__ w, size_t n, int shift,
                                   u16* __restrict__ out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = __builtin_bit_cast(u16, (_Float16)ldexpf(bf16_lo(w[i]), shift));
}

int reduce_blocks(size_t n) {
  return (int)std::min<size_t>(std::max<size_t>((n + 255) / 256, 1), 8192);
}

}  // namespace

// K splits of one dense launch: enough workgroups to cover the CUs (256), within the partial
// sums' room, each K range a multiple of the 32-column step.
// (one workgroup per CU: the doubling stops past ~1.25 rounds of the 256 CUs)
int dense_splits(int T, int N, int K, size_t part_floats) {
  const int tiles = ((T + kDM - 1) / kDM) * (N / kDN);
  int S = 1;
  while (S < 4 && tiles * 2 * S <= 320 && (size_t)(2 * S) * T * N <= part_floats &&
         (K / kDK) / (2 * S) >= 8)
    S *= 2;
  return S;
}

bool dense_fits(int T, int I, int H, size_t part_floats) {
  return T >= kDM && (2 * I) % kDN == 0 && H % kDN == 0 && I % kDK == 0 && H % kDK == 0 &&
         (size_t)T * 2 * I <= part_floats && (size_t)T * H <= part_floats;
}

void launch_dense_gate_up(const ExpertMats& m, int T, int H, int I, const float* x, float* act,
                          Epi epi, int* status, float* part, size_t part_floats, hipStream_t s) {
  const int S = dense_splits(T, 2 * I, H, part_floats);
  const int blocks = ((T + kDM - 1) / kDM) * (2 * I / kDN) * S;
  dense_gemm_kernel<<<(blocks + 7) / 8 * 8, 512, 0, s>>>(x, T, H, m.data[0], m.data[1], I,
                                                        2 * I, S, part);
  dense_reduce_gate_up_kernel<<<reduce_blocks((size_t)T * I / 4), 256, 0, s>>>(part, T, I, S, epi,
                                                                              act, status);
}

void launch_dense_gate_up_f16(const ExpertMats& m, int T, int H, int I, const float* x,
                              uint16_t* act16, int* rowexp, Epi epi, int* status, float* part,
                              size_t part_floats, hipStream_t s) {
  const int S = dense_splits(T, 2 * I, H, part_floats);
  const int blocks = ((T + kDM - 1) / kDM) * (2 * I / kDN) * S;
  dense_gemm_kernel<<<(blocks + 7) / 8 * 8, 512, 0, s>>>(x, T, H, m.data[0], m.data[1], I,
                                                        2 * I, S, part);
  dense_reduce_gate_up_f16_kernel<<<T, 256, (size_t)I * 4, s>>>(part, T, I, S, epi, act16,
                                                                 rowexp, status);
}

void launch_dense_down_f16(const uint16_t* w16, int T, int H, int I, const uint16_t* act16,
                           const int* rowexp, Epi epi, float* out, int* status, hipStream_t s) {
  const int blocks = ((T + kDM16 - 1) / kDM16) * (H / kDN);
  dense_down_f16_kernel<<<(blocks + 7) / 8 * 8, 512, 0, s>>>(
      act16, rowexp, T, I, reinterpret_cast<const uint8_t*>(w16), H, epi, out, status);
}

int bf16_f16_shift(const uint16_t* w, size_t n) {
  int* range = nullptr;
  if (hipMalloc(&range, 2 * sizeof(int)) != hipSuccess) return kNoF16Shift;
  const int init[2] = {255, 0};
  int got[2] = {255, 0};
  bool ok = hipMemcpy(range, init, sizeof(init), hipMemcpyHostToDevice) == hipSuccess;
  if (ok) {
    bf16_exp_range_kernel<<<(int)std::min<size_t>((n / 8 + 255) / 256 + 1, 1024), 256>>>(w, n,
                                                                                        range);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpy(got, range, sizeof(got), hipMemcpyDeviceToHost) == hipSuccess;
  }
  (void)hipFree(range);
  if (!ok) return kNoF16Shift;
  if (got[1] == 0) return 0;  // all zero
  // largest value below 2^16 (f16's largest finite value holds any 8-bit significand there);
  // every value's last significand bit at or above 2^-24 (the f16 grid)
  if (got[1] - got[0] > 32) return kNoF16Shift;
  return 142 - got[1];
}

void launch_bf16_to_f16(const uint16_t* w, size_t n, int shift, uint16_t* out, hipStream_t s) {
  bf16_to_f16_kernel<<<reduce_blocks(n), 256, 0, s>>>(w, n, shift, out);
}

}  // namespace urb
