// urb_route.hip -- router GEMV/GEMM, top-k routing and the token->expert permutation.
#include "urb_decode.hpp"
#include "urb_device.hpp"
#include "urb_kernels.hpp"
#include "urb_panel.hpp"
#include "urb_quant.hpp"

#include <algorithm>

namespace urb {

// A token's piece vector, written as a side job of a one-token router launch by lanes gtid,
// gtid + stride, ... of its grid: the hi/lo BF16 split of x (xq = 0), or for the MX-activation
// compositions simulate_e4m3_activation of x in blocks of xq = 32 or 128 values (pieces with
// a zero low half), which then needs no launch of its own.  stride is a multiple of 64 and
// gtid % 64 the lane, so a block's 32 lanes are one half wavefront, as the quantizer needs.
__device__ __forceinline__ void token_pieces(const float* __restrict__ x, int H, uint16_t* xp,
                                             int xq, int* status, size_t gtid, size_t stride) {
  if (xq == 0) {
    split_vector(x, H / 8, xp, gtid, stride);
    return;
  }
  const size_t nblocks = (size_t)H / xq;
  for (size_t g = gtid; g < nblocks * 32; g += stride) {
    if (xq == 128)
      quantize_lanes<4>(x, nblocks, H, nullptr, nullptr, nullptr, status, 0, nullptr, nullptr,
                        xp, g);
    else
      quantize_lanes<1>(x, nblocks, H, nullptr, nullptr, nullptr, status, 0, nullptr, nullptr,
                        xp, g);
  }
}

// ------------------------------------------------------------------------------------------
// Qwen router: `linear(router)` = Bf16Matrix::matvec_fp32 + BF16 (src/models/qwen3_8/math.rs:
// 10-26); DeepSeek-V4.1's `router.matvec_fp32_accum` is the same GEMV without the BF16 step
// (src/models/deepseek_v41/runtime.rs:2136).  The reference GEMV is the 8-lane FP32 FMA tree (src/model/bf16.rs:589-610): lane j
// accumulates columns == j (mod 8) in order, lanes are summed 0..7 (H is a multiple of 128
// here, so there is no tail).  One thread per (expert, lane) runs that exact chain, so the
// BF16 logits -- and hence their exact ties -- are bit-identical to the reference.  The
// weights are re-laid out once at create time so that every load instruction of a wavefront
// reads 1 KiB of consecutive chain elements.
// ------------------------------------------------------------------------------------------

// Lane-chain layout of the QWEN36 router: lane l = 8 el + j of the wavefront that owns experts
// [8 g, 8 g + 8) accumulates chain (expert 8 g + el, lane j) = columns j, 8 + j, 16 + j, ...
// of that expert.  Chain elements are stored so that each 16-element batch b of every lane is
// two 1 KiB runs (halves h) in lane order: element 16 b + 8 h + k of lane l sits at
// (((g * H / 128 + b) * 2 + h) * 64 + l) * 8 + k.  `w` has rows zero-padded to a multiple of 8.
__global__ void relayout_lane8_kernel(const uint16_t* __restrict__ w, int E8, int H,
                                      uint16_t* __restrict__ w8) {
  const size_t n = (size_t)E8 * H;
  const int nb = H / 128;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int k = (int)(idx & 7);
    const int l = (int)((idx >> 3) & 63);
    const size_t rest = idx >> 9;  // (g * nb + b) * 2 + h
    const int h = (int)(rest & 1);
    const size_t gb = rest >> 1;
    const int b = (int)(gb % nb);
    const size_t g = gb / nb;
    const size_t e = 8 * g + (l >> 3);
    const int i = 16 * b + 8 * h + k;
    w8[idx] = w[e * H + 8 * (size_t)i + (l & 7)];
  }
}

// 16-element chain batches in flight per lane (8 x 32 B = 64 VGPRs of weights).
constexpr int kLane8Ring = 8;

// WAVES waves per workgroup, wave w running the chains of expert group WAVES blockIdx.x + w:
// the staged token row is shared by 8 WAVES experts.  RING chain batches are in flight per
// lane.
// `w8b` (optional): a second matrix of one row (Qwen3.6's shared-expert gate), run by one more
// workgroup (the last along x) into logits_b, so that row needs no launch of its own.
template <int kLane8Tokens, int WAVES = 1, int RING = kLane8Ring>
__global__ __launch_bounds__(64 * WAVES) void router_lane8_kernel(
    const uint16_t* __restrict__ w8, int E, int H, const float* __restrict__ x, int T,
    float* __restrict__ logits, int round_bf16, int* status, uint16_t* __restrict__ xp,
    const uint16_t* __restrict__ w8b = nullptr, float* __restrict__ logits_b = nullptr,
    int xq = 0, unsigned* lo_word = nullptr, unsigned lo_gen = 0) {
  // [tok][8][H8 + 4] transposed chains: the pad of 4 floats puts the 8 chains of a column in
  // different LDS banks and keeps 16-byte alignment.  H is a multiple of 128.
  extern __shared__ float xs[];
  const bool second = w8b && blockIdx.x == gridDim.x - 1;
  if (second) {
    w8 = w8b;
    E = 1;
    logits = logits_b;
  }
  const int H8 = H / 8, H8p = H8 + 4;
  const int t0 = blockIdx.y * kLane8Tokens;
  const int nt = min(kLane8Tokens, T - t0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int el = lane >> 3, j = lane & 7;
  const int g = (second ? 0 : blockIdx.x) * WAVES + wave;
  const bool live = g < (E + 7) / 8;
  const int e = g * 8 + el;
  const uint16_t* chains = w8 + (size_t)(live ? g : 0) * 8 * H + 8 * lane;
  const int nb = H8 / 16;
  // Stage x with coalesced float4 loads, transposed into per-lane chains, kXR loads per thread
  // in flight at a time.  The first kXR go out before the first RING weight batches (loads
  // complete in order: the stores then wait for x alone, one round trip, instead of for the
  // weights and then one round trip per float4); later ones, for long rows, after them.  A
  // load past the end re-reads (and restages) the last float4.  `lo`: some value is not BF16
  // (its hi/lo BF16 split, the grouped GEMMs' staging, has a non-zero lo half).
  constexpr int kXR = 8 / WAVES;
  const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)t0 * H);
  const int n4 = nt * H / 4, nth = 64 * WAVES;
  bool bad = false, lo = false;
  float4 xv[kXR];
  auto xload = [&](int i0) {
#pragma unroll
    for (int u = 0; u < kXR; ++u) xv[u] = x4[min(i0 + u * nth, n4 - 1)];
  };
  auto xstore = [&](int i0) {
#pragma unroll
    for (int u = 0; u < kXR; ++u) {
      const int i = min(i0 + u * nth, n4 - 1);
      const float vv[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // token and column of the value (one token per workgroup: no division; measured on
        // MI355X, the division in this loop was 0.5-0.7 of the one-token router's 6.8 us)
        const int flat = 4 * i + q, tt = kLane8Tokens == 1 ? 0 : flat / H, c = flat - tt * H;
        bad |= !finite(vv[q]);
        lo |= (__float_as_uint(vv[q]) & 0xffffu) != 0;
        xs[(tt * 8 + (c & 7)) * H8p + (c >> 3)] = vv[q];
      }
    }
  };
  // weight batch b into ring slot d; every fetch is issued, batches past the last clamped to
  // it (a re-read), so that no load sits on one path only: the compiler's wait counts then
  // stay exact instead of waiting for every load in flight
  uint4 ring[RING][2];
  auto fetch = [&](int d, int b) {
    b = min(b, nb - 1);
    ring[d][0] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * b) * 512);
    ring[d][1] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * b + 1) * 512);
  };
  xload(threadIdx.x);
  __builtin_amdgcn_sched_barrier(0);  // the x loads stay ahead of the weights'
#pragma unroll
  for (int d = 0; d < RING; ++d) fetch(d, d);
  __builtin_amdgcn_sched_barrier(0);
  xstore(threadIdx.x);
  for (int i0 = threadIdx.x + kXR * nth; i0 < n4; i0 += kXR * nth) {
    xload(i0);
    xstore(i0);
  }
  if (bad) flag(status, kStatusNonFinite);
  if (lo_word && __ballot(lo) != 0 && lane == 0) *lo_word = lo_gen;
  // one token, MX-activation input: the workgroups also write its quantized piece vector
  if (xp && T == 1 && xq != 0)
    token_pieces(x, H, xp, xq, status, blockIdx.x * blockDim.x + threadIdx.x,
                 gridDim.x * blockDim.x);
  __syncthreads();
  // one token: its piece vector (the decode GEMVs' input) from the staged row
  if (xp && T == 1 && xq == 0) {
    for (int u = blockIdx.x * blockDim.x + threadIdx.x; u < H8; u += gridDim.x * blockDim.x) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = xs[k * H8p + u];
      store_piece_unit(v, xp + (size_t)u * kPieceUnit);
    }
  }
  if (!live) return;
  float acc[kLane8Tokens];
#pragma unroll
  for (int tt = 0; tt < kLane8Tokens; ++tt) acc[tt] = 0.0f;
  const float* xj = xs + j * H8p;
  for (int b0 = 0; b0 < nb; b0 += RING) {
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      const int b = b0 + d;
      if (b >= nb) break;
      const uint4 qa = ring[d][0], qb = ring[d][1];
      fetch(d, b + RING);
      const float wv[16] = {bf16_lo(qa.x), bf16_hi(qa.x), bf16_lo(qa.y), bf16_hi(qa.y),
                            bf16_lo(qa.z), bf16_hi(qa.z), bf16_lo(qa.w), bf16_hi(qa.w),
                            bf16_lo(qb.x), bf16_hi(qb.x), bf16_lo(qb.y), bf16_hi(qb.y),
                            bf16_lo(qb.z), bf16_hi(qb.z), bf16_lo(qb.w), bf16_hi(qb.w)};
#pragma unroll
      for (int tt = 0; tt < kLane8Tokens; ++tt) {
        if (tt < nt) {
          const float4* xv = reinterpret_cast<const float4*>(xj + tt * 8 * H8p + 16 * b);
          const float4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
          const float xf[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
          for (int k = 0; k < 16; ++k) acc[tt] = fmaf(wv[k], xf[k], acc[tt]);
        }
      }
    }
  }
  // Lane sum in lane order 0..7 (the reference's horizontal sum of the 8 FMA lanes).
  const int base = el * 8;
  for (int tt = 0; tt < kLane8Tokens; ++tt) {
    float sum = __shfl(acc[tt], base + 0, 64);
#pragma unroll
    for (int u = 1; u < 8; ++u) sum = __fadd_rn(sum, __shfl(acc[tt], base + u, 64));
    if (e < E && j == 0 && tt < nt) {
      // Qwen's linear() rounds the logits to BF16; the plain FP32 GEMV rejects non-finite ones
      float r = sum;
      if (round_bf16 ? !rne_bf16(sum, &r) : !finite(sum)) {
        flag(status, kStatusNonFinite);
        r = sum;
      }
      logits[(size_t)(t0 + tt) * E + e] = r;
    }
  }
}

// Batched form of the same 8-lane FP32 tree: a 256-thread workgroup runs the chains of 32
// experts (wave w: expert group 4 blockIdx.x + w) for TB tokens at once, so each weight batch
// it streams feeds TB tokens.  x is staged 512 columns (4 chain batches) at a time in the
// transposed chain layout; chain order, FMA and the lane sum are exactly the single-token
// kernel's, so the logits are bit-identical.
constexpr int kLane8ChunkBatches = 4;  // 16-element chain batches per staged x chunk

template <int TB>
__global__ __launch_bounds__(256) void router_lane8_tiled_kernel(
    const uint16_t* __restrict__ w8, int E, int H, const float* __restrict__ x, int T,
    float* __restrict__ logits, int round_bf16, int* status, unsigned* lo_word,
    unsigned lo_gen) {
  constexpr int CP = 16 * kLane8ChunkBatches + 4;  // chunk chain pitch (4-float pad)
  __shared__ __attribute__((aligned(16))) float xs[TB * 8 * CP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int el = lane >> 3, j = lane & 7;
  const int G = (E + 7) / 8;
  const int g = blockIdx.x * 4 + wave;
  const bool live = g < G;
  const int e = g * 8 + el;
  const int t0 = blockIdx.y * TB;
  const int nt = min(TB, T - t0);
  const int nb = H / 128;
  const uint16_t* chains = w8 + (size_t)(live ? g : 0) * 8 * H + 8 * lane;
  uint4 ring[8][2];
  if (live) {
#pragma unroll
    for (int d = 0; d < 8; ++d)
      if (d < nb) {
        ring[d][0] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * d) * 512);
        ring[d][1] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * d + 1) * 512);
      }
  }
  float acc[TB];
#pragma unroll
  for (int tt = 0; tt < TB; ++tt) acc[tt] = 0.0f;
  bool bad = false, lo = false;  // lo: some value is not BF16 (router_lane8_kernel)
  for (int b0 = 0; b0 < nb; b0 += 8) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int cb = b0 + kLane8ChunkBatches * half;
      if (cb >= nb) break;
      const int ncols = 128 * min(kLane8ChunkBatches, nb - cb);
      __syncthreads();  // the previous chunk's readers are done
      for (int i = threadIdx.x; i < nt * ncols / 4; i += blockDim.x) {
        const int tt = (4 * i) / ncols, c0 = 4 * i - tt * ncols;
        const float4 v4 =
            *reinterpret_cast<const float4*>(x + (size_t)(t0 + tt) * H + 128 * cb + c0);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = c0 + u;
          bad |= !finite(vv[u]);
          lo |= (__float_as_uint(vv[u]) & 0xffffu) != 0;
          xs[(tt * 8 + (c & 7)) * CP + (c >> 3)] = vv[u];
        }
      }
      __syncthreads();
      if (!live) continue;
#pragma unroll
      for (int bb = 0; bb < kLane8ChunkBatches; ++bb) {
        const int d = kLane8ChunkBatches * half + bb, b = cb + bb;
        if (b >= nb) break;
        const uint4 qa = ring[d][0], qb = ring[d][1];
        if (b + 8 < nb) {
          ring[d][0] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * (b + 8)) * 512);
          ring[d][1] = *reinterpret_cast<const uint4*>(chains + (size_t)(2 * (b + 8) + 1) * 512);
        }
        const float wv[16] = {bf16_lo(qa.x), bf16_hi(qa.x), bf16_lo(qa.y), bf16_hi(qa.y),
                              bf16_lo(qa.z), bf16_hi(qa.z), bf16_lo(qa.w), bf16_hi(qa.w),
                              bf16_lo(qb.x), bf16_hi(qb.x), bf16_lo(qb.y), bf16_hi(qb.y),
                              bf16_lo(qb.z), bf16_hi(qb.z), bf16_lo(qb.w), bf16_hi(qb.w)};
        const float* xj = xs + j * CP + 16 * bb;
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
          if (tt < nt) {
            const float4* xv = reinterpret_cast<const float4*>(xj + tt * 8 * CP);
            const float4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
            const float xf[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                  x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[tt] = fmaf(wv[k], xf[k], acc[tt]);
          }
        }
      }
    }
  }
  if (bad) flag(status, kStatusNonFinite);
  if (lo_word && __ballot(lo) != 0 && lane == 0) *lo_word = lo_gen;
  if (!live) return;
  const int base = el * 8;
#pragma unroll
  for (int tt = 0; tt < TB; ++tt) {
    float sum = __shfl(acc[tt], base + 0, 64);
#pragma unroll
    for (int u = 1; u < 8; ++u) sum = __fadd_rn(sum, __shfl(acc[tt], base + u, 64));
    if (e < E && j == 0 && tt < nt) {
      float r = sum;
      if (round_bf16 ? !rne_bf16(sum, &r) : !finite(sum)) {
        flag(status, kStatusNonFinite);
        r = sum;
      }
      logits[(size_t)(t0 + tt) * E + e] = r;
    }
  }
}

// ------------------------------------------------------------------------------------------
// Top-k routing: one wavefront per token, expert e in lane e % 64, slot e / 64.  Ranking is
// iterated wave arg-max on (total-order key desc, expert id asc) -- the reference's sort
// comparator -- with DPP reductions.  Round r's winner is kept by lane r.  Sums the reference
// performs sequentially are performed sequentially here too (lane by lane via readlane).
// ------------------------------------------------------------------------------------------
constexpr int kMaxExperts = 512;
constexpr int kMaxTopK = 32;

__device__ __forceinline__ int dpp_max_i32(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xf, 0xf, false));  // row_mirror
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast15
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast31
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int dpp_min_i32(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float rdl(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The float whose total-order key is k (total_key is an involution on the bits).
__device__ __forceinline__ float key_value(int32_t k) {
  return __int_as_float(k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1));
}
// (k1 >= k2) := the two largest keys of this lane's set merged with the partner lane's
// (disjoint) set; the partner is the DPP lane CTRL, a ds_swizzle pattern, or lane ^ 32.
__device__ __forceinline__ void top2_fold(int32_t& k1, int32_t& k2, int32_t p1, int32_t p2) {
  k2 = max(min(k1, p1), max(k2, p2));
  k1 = max(k1, p1);
}
template <int CTRL>
__device__ __forceinline__ void top2_merge(int32_t& k1, int32_t& k2) {
  top2_fold(k1, k2, __builtin_amdgcn_update_dpp(k1, k1, CTRL, 0xf, 0xf, false),
            __builtin_amdgcn_update_dpp(k2, k2, CTRL, 0xf, 0xf, false));
}
template <int PATTERN>
__device__ __forceinline__ void top2_merge_swz(int32_t& k1, int32_t& k2) {
  top2_fold(k1, k2, __builtin_amdgcn_ds_swizzle(k1, PATTERN), __builtin_amdgcn_ds_swizzle(k2, PATTERN));
}
__device__ __forceinline__ void top2_merge_x32(int32_t& k1, int32_t& k2) {
  top2_fold(k1, k2, __shfl_xor(k1, 32, 64), __shfl_xor(k2, 32, 64));
}

// One ranking round over the lane's untaken slots: returns the winner id (uniform) and sets
// `val` (uniform) to the winner's `score2` value.
template <int EPL>
__device__ __forceinline__ int argmax_round(const int32_t (&key)[EPL], const float (&score2)[EPL],
                                            bool (&open)[EPL], float& val) {
  const int lane = threadIdx.x & 63;
  int32_t bk = INT32_MIN;
  int bid = INT32_MAX;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (open[i] && key[i] > bk) { bk = key[i]; bid = lane + 64 * i; }
  const int kmax = dpp_max_i32(bk);
  // the lowest id among the lanes holding the maximum: one lane (the usual case) names it
  const uint64_t at_max = __ballot(bk == kmax);
  const int id = __popcll(at_max) == 1
                     ? __builtin_amdgcn_readlane(bid, (int)__builtin_ctzll(at_max))
                     : dpp_min_i32(bk == kmax ? bid : INT32_MAX);
  float mine = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (lane + 64 * i == id) { open[i] = false; mine = score2[i]; }
  val = rdl(mine, id & 63);
  return id;
}

// Routes token t with the calling wavefront.  `sh` (kMaxExperts floats) and `grp` (64 floats)
// are the wave's LDS scratch.
// MODE: 0 softmax top-k, 1 sigmoid noaux_tc, 2 sqrt-softplus.
template <int EPL, int MODE>
__device__ void route_token(int t, float* __restrict__ logits, int T, int E, int K,
                            const RouteParams& rp, int32_t* __restrict__ ids,
                            float* __restrict__ weights, int32_t* __restrict__ asc, int* status,
                            float* sh, float* grpw, bool store_logits = true) {
  const int lane = threadIdx.x & 63;
  float* lt = logits + (size_t)t * E;
  float v[EPL];
  bool open[EPL];
  bool bad = false;
  // the selection bias is loaded first, so its latency overlaps the logits' (one token's routing
  // is a chain of dependent steps; this kernel is on the critical path of every decode call)
  float bias[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    bias[i] = (MODE != 0 && rp.bias && e < E) ? rp.bias[e] : 0.0f;
  }
  if (rp.part) {
    // logit = (f32) sum of the router's f64 partial slices, in slice order
    const size_t pitch = (size_t)router_rows(E), slice = (size_t)T * pitch;
    const double* pt = rp.part + (size_t)t * pitch;
    double acc[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) acc[i] = 0.0;
    // ZB slices' loads in flight at once, then added in slice order
    constexpr int ZB = EPL >= 8 ? 4 : (EPL >= 4 ? 8 : 16);
    for (int z0 = 0; z0 < rp.slices; z0 += ZB) {
      double pz[ZB][EPL];
#pragma unroll
      for (int zz = 0; zz < ZB; ++zz)
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int e = lane + 64 * i;
          pz[zz][i] = (z0 + zz < rp.slices && e < E) ? pt[(size_t)(z0 + zz) * slice + e] : 0.0;
        }
#pragma unroll
      for (int zz = 0; zz < ZB; ++zz)
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (z0 + zz < rp.slices) acc[i] += pz[zz][i];
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      open[i] = e < E;
      v[i] = (float)acc[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      open[i] = e < E;
      v[i] = open[i] ? lt[e] : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (open[i] && !finite(v[i])) bad = true;
  int my_id = 0;
  float my_val = 0.0f;
  float w = 0.0f;
  if constexpr (MODE == 0) {
    // route_softmax_top_k (src/models/qwen3_8/moe.rs:91-159).
    int32_t mk = INT32_MIN;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (open[i]) mk = max(mk, total_key(v[i]));
    // total-order key of the maximum; logits are finite here, so it is the float maximum
    int32_t kmax = dpp_max_i32(mk);
    const float m = __int_as_float(kmax ^ (int32_t)(((uint32_t)(kmax >> 31)) >> 1));
    float p[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) p[i] = open[i] ? exp_f32(v[i] - m) : 0.0f;
    // the denominator sums in expert order: every lane adds all E values from LDS in order
    // (broadcast reads), so each holds the sequential sum
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (open[i]) sh[64 * i + lane] = p[i];
    __builtin_amdgcn_wave_barrier();
    float den = 0.0f;
    const float4* sh4 = reinterpret_cast<const float4*>(sh);
    int e = 0;
    for (; e + 4 <= E; e += 4) {
      const float4 q = sh4[e >> 2];
      den = __fadd_rn(den, q.x);
      den = __fadd_rn(den, q.y);
      den = __fadd_rn(den, q.z);
      den = __fadd_rn(den, q.w);
    }
    for (; e < E; ++e) den = __fadd_rn(den, sh[e]);
    if (!finite(den) || den <= 0.0f) bad = true;
    int32_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      p[i] = p[i] / den;
      if (open[i] && !finite(p[i])) bad = true;
      key[i] = total_key(p[i]);
    }
    for (int r = 0; r < K; ++r) {
      float val;
      const int id = argmax_round<EPL>(key, p, open, val);
      if (lane == r) { my_id = id; my_val = val; }
    }
    float sel_sum = 0.0f;  // sequential in ranking order
    for (int r = 0; r < K; ++r) sel_sum = __fadd_rn(sel_sum, rdl(my_val, r));
    if (!finite(sel_sum) || sel_sum <= 0.0f) bad = true;
    w = my_val / sel_sum;
    if (lane < K) {
      if (!finite(w)) bad = true;
      if (rp.qwen) {  // qwen3_6/runtime.rs:1233-1238: route weights materialised in BF16
        float q;
        if (!rne_bf16(w, &q)) bad = true; else w = q;
      }
    }
  } else if constexpr (MODE == 2) {
    // route_sqrt_softplus (src/models/deepseek_v4/math.rs:451-516):
    // score = sqrt(softplus(l)) with softplus(v) = v + ln_1p(exp(-v)) for v > 0, else
    // ln_1p(exp(v)) (:604-610); selection = score + bias ranks, or the token's hash row gives
    // the experts in table order; the weight divides by the f32 sum of the chosen scores in
    // that order.
    float score[EPL];
    int32_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      float sp = 0.0f;
      if (open[i]) {
        const float x = v[i];
        const float ex = exp_f32(x > 0.0f ? -x : x);
        const float l1 = (float)log1p((double)ex);
        sp = x > 0.0f ? __fadd_rn(x, l1) : l1;
      }
      score[i] = open[i] ? sqrtf(sp) : 0.0f;  // correctly rounded (not the native root)
      key[i] = total_key(__fadd_rn(score[i], bias[i]));
    }
    if (rp.hash) {
      // the tid2eid row of the token (deepseek_v4/runtime.rs:2664-2681); lane r < K reads the
      // score of its expert from LDS
      uint32_t tok = rp.tokens[t];
      if (tok >= rp.vocab) {
        if (lane == 0) flag(status, kStatusBadToken);
        tok = 0;
      }
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (open[i]) sh[lane + 64 * i] = score[i];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (lane < K) {
        my_id = rp.hash[(size_t)tok * K + lane];
        my_val = sh[my_id];
      }
    } else {
      for (int r = 0; r < K; ++r) {
        float val;
        const int id = argmax_round<EPL>(key, score, open, val);
        if (lane == r) { my_id = id; my_val = val; }
      }
    }
    float den = -0.0f;  // Iterator::sum in ranking (or table) order
    for (int r = 0; r < K; ++r) den = __fadd_rn(den, rdl(my_val, r));
    if (!finite(den) || den <= 0.0f) bad = true;
    w = __fmul_rn(__fdiv_rn(my_val, den), rp.scale);
  } else {
    // route_noaux_tc (src/math/routing.rs:38-155).
    float g[EPL], sc[EPL];
    int32_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      g[i] = open[i] ? 1.0f / (1.0f + exp_f32(-v[i])) : 0.0f;
      sc[i] = __fadd_rn(g[i], bias[i]);
      key[i] = total_key(sc[i]);
    }
    if (rp.topk_group < rp.n_group) {
      // group score = sum of the two largest selection scores (:104-111).  (Equal keys are
      // equal values, so the order in which a group's members are visited does not change
      // the two values.)
      const int per = E / rp.n_group;
      const bool pow2 = (per & (per - 1)) == 0;
      const int lg = __builtin_ctz(per);
      if (per >= 2 && 64 % per == 0) {
        // A group is an aligned run of `per` lanes of one slot: a butterfly of top-2 merges
        // over that run leaves the group's two largest keys in every lane of it.
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          int32_t k1 = open[i] ? key[i] : INT32_MIN, k2 = INT32_MIN;
          top2_merge<0xB1>(k1, k2);                        // quad_perm 1,0,3,2
          if (per > 2) top2_merge<0x4E>(k1, k2);           // quad_perm 2,3,0,1
          if (per > 4) top2_merge<0x141>(k1, k2);          // row_half_mirror
          if (per > 8) top2_merge<0x140>(k1, k2);          // row_mirror
          if (per > 16) top2_merge_swz<0x401F>(k1, k2);    // lane ^ 16
          if (per > 32) top2_merge_x32(k1, k2);            // lane ^ 32
          const int e = lane + 64 * i;
          if (open[i] && (e & (per - 1)) == 0)
            grpw[e >> lg] = __fadd_rn(key_value(k1), key_value(k2));
        }
      } else {
        // Lane g scans group g in batches of eight independent LDS reads, starting at its
        // own offset g so the lanes read different banks.
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (open[i]) sh[lane + 64 * i] = sc[i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane < rp.n_group) {
          int32_t k1 = INT32_MIN, k2 = INT32_MIN;
          float b1 = 0.0f, b2 = 0.0f;
          const float* row = sh + lane * per;
          const int start = lane % per;
          for (int i0 = 0; i0 < per; i0 += 8) {
            float sv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              int i = i0 + j + start;  // the group's slots in rotated order
              i = i >= per ? i - per : i;
              i = i0 + j < per ? i : 0;  // past the group's end: any valid slot, unused
              sv[j] = row[i];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              if (i0 + j >= per) break;
              const int32_t k = total_key(sv[j]);
              const bool gt1 = k > k1, gt2 = k > k2;
              k2 = gt1 ? k1 : (gt2 ? k : k2);
              b2 = gt1 ? b1 : (gt2 ? sv[j] : b2);
              k1 = gt1 ? k : k1;
              b1 = gt1 ? sv[j] : b1;
            }
          }
          grpw[lane] = __fadd_rn(b1, b2);
        }
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      // keep the top `topk_group` groups (score desc, id asc): a group's rank is the number
      // of groups ahead of it in that order
      const bool is_group = lane < rp.n_group;
      const int32_t gk = is_group ? total_key(grpw[lane]) : INT32_MIN;
      int rank = 0;
      for (int h = 0; h < rp.n_group; ++h) {
        const int32_t kh = __builtin_amdgcn_readlane(gk, h);
        rank += (kh > gk || (kh == gk && h < lane)) ? 1 : 0;
      }
      const uint64_t gmask = __ballot(is_group && rank < rp.topk_group);
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        if (open[i] && !((gmask >> (pow2 ? e >> lg : e / per)) & 1ull)) open[i] = false;
      }
    }
    for (int r = 0; r < K; ++r) {
      float val;
      const int id = argmax_round<EPL>(key, g, open, val);
      if (lane == r) { my_id = id; my_val = val; }
    }
    float den = -0.0f;  // Iterator::sum in ranking order, plus the 1e-20 epsilon
    for (int r = 0; r < K; ++r) den = __fadd_rn(den, rdl(my_val, r));
    den = __fadd_rn(den, 1e-20f);
    if (rp.normalize && !finite(den)) bad = true;
    w = __fmul_rn(rp.normalize ? my_val / den : my_val, rp.scale);
  }
  if (rp.part && store_logits) {
    // the logits are stored last: a store counts against the same counter as the loads, so
    // an earlier store would be waited on by every later wait for a load
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i < E) lt[lane + 64 * i] = v[i];
  }
  if (bad) flag(status, kStatusNonFinite);
  if (lane < K) {
    ids[(size_t)t * K + lane] = my_id;
    weights[(size_t)t * K + lane] = w;
    if (asc) {
      // ranking position `lane` goes to its place in ascending expert id order
      // (qwen3_6/runtime.rs:1239-1240; the ids of one token are distinct)
      int before = 0;
      for (int r = 0; r < K; ++r) before += __builtin_amdgcn_readlane(my_id, r) < my_id;
      asc[(size_t)t * K + before] = lane;
    }
  }
}

template <int EPL, int MODE>
__global__ __launch_bounds__(256) void route_kernel(float* __restrict__ logits, int T,
                                                    int E, int K, RouteParams rp,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ weights,
                                                    int32_t* __restrict__ asc, int* status) {
  __shared__ __attribute__((aligned(16))) float lds[4][kMaxExperts];
  __shared__ float grp[4][64];
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  route_token<EPL, MODE>(t, logits, T, E, K, rp, ids, weights, asc, status, lds[wave],
                            grp[wave]);
}

// ------------------------------------------------------------------------------------------
// One-token calls with a shared expert: the shared expert's gate+up GEMV and the token's top-k
// routing in one launch.  The grid is the GEMV's plus one workgroup, whose first wave routes
// the token while the others stream the shared expert's weights.  The two read the router's
// output (logits or partial slices, and the token's pieces) and share nothing else, so no
// workgroup waits for another; the routing's latency hides under the GEMV.  The routing
// handles up to 64 * EPL experts.
// ------------------------------------------------------------------------------------------
// One-token BF16 gate+up GEMVs (the shared expert's, and the routed one that routes in every
// workgroup) run as half panel pairs: twice the workgroups, for matrices whose whole pairs
// would leave CUs idle or unevenly loaded.
template <int FMT>
constexpr bool kHalfPairs = FMT == kFmtBF16;

template <int FMT, int EPL, int MODE>
__global__ __launch_bounds__(64 * 8) void gemv_gate_up_route_kernel(
    const ExpertMats* __restrict__ mats, Perm perm, int rows, int cols, int ksplit,
    const uint16_t* __restrict__ xp, float* __restrict__ out, uint16_t* __restrict__ out_xp,
    Epi epi, int* status, RouteJob job, int E) {
  static_assert(decode_max_waves<FMT, true>() == 8, "workgroup bound of the gate_up GEMV");
  extern __shared__ uint4 pieces_lds[];
  if (blockIdx.x == gridDim.x - 1) {
    // the LDS of the GEMV's input pieces holds the routing's scratch (the launch sizes it)
    float* sh = reinterpret_cast<float*>(pieces_lds);
    if (threadIdx.x < 64)
      route_token<EPL, MODE>(0, job.logits, 1, E, job.K, job.rp, job.ids, job.weights, job.asc,
                             status, sh, sh + kMaxExperts);
    return;
  }
  // BF16: half panel pairs, so a dense 2048-row gate+up offers 256 workgroups, one per CU
  // (a 2 x 2048 x 7168 shared gate+up 16.3-17.6 -> 15.3-15.8 us).  The MX formats keep
  // whole pairs: their steps are 1-2 KiB per panel, and halving them made DeepSeek-V4 Flash's
  // MXFP4 shared gate+up 12.3 -> 13.7 us.
  gemv_mfma_body<FMT, true, 1, decode_depth<FMT, true>(), decode_max_waves<FMT, true>(),
                 kHalfPairs<FMT>>(mats, perm, rows, cols, ksplit, xp, out, out_xp, epi,
                                        status, pieces_lds, blockIdx.x, blockIdx.y);
}

template <int FMT, int EPL, int MODE>
static void launch_gate_up_route_as(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                    float* act, uint16_t* act_xp, Epi epi, int* status,
                                    hipStream_t s, int E, const RouteJob& job) {
  const Perm dense{nullptr, nullptr, nullptr, nullptr, nullptr, 1, nullptr, nullptr, 0};
  // half panel pairs: 2 I / 16 groups
  GemvShape g = gemv_mfma_shape<FMT, true>(kHalfPairs<FMT> ? 2 * I : I, H, 1);
  g.grid.x += 1;
  g.lds = std::max(g.lds, (size_t)(kMaxExperts + 64) * sizeof(float));
  gemv_gate_up_route_kernel<FMT, EPL, MODE><<<g.grid, 64 * g.waves, g.lds, s>>>(
      mats, dense, I, H, g.ksplit, xp, act, act_xp, epi, status, job, E);
}

template <int FMT, int EPL>
static void launch_gate_up_route_epl(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                     float* act, uint16_t* act_xp, Epi epi, int* status,
                                     hipStream_t s, int E, const RouteJob& job) {
  if (job.rp.router == 0)
    launch_gate_up_route_as<FMT, EPL, 0>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
  else if (job.rp.router == 1)
    launch_gate_up_route_as<FMT, EPL, 1>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
  else
    launch_gate_up_route_as<FMT, EPL, 2>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
}

template <int FMT>
static void launch_gate_up_route_fmt(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                     float* act, uint16_t* act_xp, Epi epi, int* status,
                                     hipStream_t s, int E, const RouteJob& job) {
  if (E <= 256)
    launch_gate_up_route_epl<FMT, 4>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
  else
    launch_gate_up_route_epl<FMT, 8>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
}

void launch_shared_gate_up_route(int fmt, const ExpertMats* mats, int H, int I,
                                 const uint16_t* xp, float* act, uint16_t* act_xp, Epi epi,
                                 int* status, hipStream_t s, int E, const RouteJob& job) {
  if (fmt == kFmtBF16)
    launch_gate_up_route_fmt<kFmtBF16>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
  else if (fmt == kFmtMXFP4)
    launch_gate_up_route_fmt<kFmtMXFP4>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
  else
    launch_gate_up_route_fmt<kFmtMXFP8>(mats, H, I, xp, act, act_xp, epi, status, s, E, job);
}

// ------------------------------------------------------------------------------------------
// One token without a shared expert: the routing inside the routed gate+up GEMV.  Every
// workgroup's first wave routes the token from the router's output (logits, or f64 partial
// slices) into LDS -- the same inputs through the same arithmetic, so every workgroup holds
// the same routes -- and the GEMV then reads its slot's expert from LDS.  Workgroup (0, 0)
// also writes the routes, and a sliced router's logits, for the down + combine launch.  Each
// workgroup spends one routing (its logits read and top-k) before its first weight load; the
// routing kernel and its launch are gone.  The host uses it after routers that write f32
// logits: reading a sliced router's f64 partials in every workgroup costs more than the launch.
// ------------------------------------------------------------------------------------------
constexpr int kRouteMaxK = 32;

template <int FMT, int EPL, int MODE>
__global__ __launch_bounds__(64 * 8) void gemv_route_gate_up_kernel(
    const ExpertMats* __restrict__ mats, int rows, int cols, int ksplit,
    const uint16_t* __restrict__ xp, uint16_t* __restrict__ out_xp, Epi epi, int* status,
    RouteJob job, int E) {
  static_assert(decode_max_waves<FMT, true>() == 8, "workgroup bound of the gate_up GEMV");
  extern __shared__ uint4 pieces_lds[];
  __shared__ __attribute__((aligned(16))) float rsh[kMaxExperts + 64];
  __shared__ int32_t ids_l[kRouteMaxK];
  __shared__ float w_l[kRouteMaxK];
  __shared__ int32_t asc_l[kRouteMaxK];
  const bool lead = blockIdx.x == 0 && blockIdx.y == 0;
  if (threadIdx.x < 64) {
    route_token<EPL, MODE>(0, job.logits, 1, E, job.K, job.rp, ids_l, w_l,
                           job.asc ? asc_l : nullptr, status, rsh, rsh + kMaxExperts, lead);
    if (lead && (int)threadIdx.x < job.K) {
      job.ids[threadIdx.x] = ids_l[threadIdx.x];
      job.weights[threadIdx.x] = w_l[threadIdx.x];
      if (job.asc) job.asc[threadIdx.x] = asc_l[threadIdx.x];
    }
  }
  __syncthreads();
  const Perm perm{nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, ids_l, job.K};
  gemv_mfma_body<FMT, true, 1, decode_depth<FMT, true>(), decode_max_waves<FMT, true>(),
                 kHalfPairs<FMT>>(mats, perm, rows, cols, ksplit, xp, nullptr, out_xp, epi,
                                        status, pieces_lds, blockIdx.x, blockIdx.y);
}

template <int FMT, int EPL, int MODE>
static void launch_route_gate_up_as(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                    uint16_t* act_xp, Epi epi, int* status, hipStream_t s, int E,
                                    const RouteJob& job) {
  const GemvShape g = gemv_mfma_shape<FMT, true>(kHalfPairs<FMT> ? 2 * I : I, H, job.K);
  gemv_route_gate_up_kernel<FMT, EPL, MODE><<<g.grid, 64 * g.waves, g.lds, s>>>(
      mats, I, H, g.ksplit, xp, act_xp, epi, status, job, E);
}

template <int FMT, int EPL>
static void launch_route_gate_up_epl(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                     uint16_t* act_xp, Epi epi, int* status, hipStream_t s, int E,
                                     const RouteJob& job) {
  if (job.rp.router == 0)
    launch_route_gate_up_as<FMT, EPL, 0>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else if (job.rp.router == 1)
    launch_route_gate_up_as<FMT, EPL, 1>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else
    launch_route_gate_up_as<FMT, EPL, 2>(mats, H, I, xp, act_xp, epi, status, s, E, job);
}

template <int FMT>
static void launch_route_gate_up_fmt(const ExpertMats* mats, int H, int I, const uint16_t* xp,
                                     uint16_t* act_xp, Epi epi, int* status, hipStream_t s, int E,
                                     const RouteJob& job) {
  if (E <= 128)
    launch_route_gate_up_epl<FMT, 2>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else if (E <= 256)
    launch_route_gate_up_epl<FMT, 4>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else
    launch_route_gate_up_epl<FMT, 8>(mats, H, I, xp, act_xp, epi, status, s, E, job);
}

bool launch_routed_gate_up_route(int fmt, const ExpertMats* mats, int H, int I,
                                 const uint16_t* xp, uint16_t* act_xp, Epi epi, int* status,
                                 hipStream_t s, int E, const RouteJob& job) {
  if (job.K > kRouteMaxK) return false;
  if (fmt == kFmtBF16)
    launch_route_gate_up_fmt<kFmtBF16>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else if (fmt == kFmtMXFP4)
    launch_route_gate_up_fmt<kFmtMXFP4>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  else
    launch_route_gate_up_fmt<kFmtMXFP8>(mats, H, I, xp, act_xp, epi, status, s, E, job);
  return true;
}

// ------------------------------------------------------------------------------------------
// Permutation (one workgroup, T <= 1024): a token bitmap per expert in LDS gives each
// (token, route) its stable position: offsets[e] + #earlier tokens routed to e.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive prefix sum over a 1024-thread block; *total receives the block sum.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
  const int incl = wave_incl_scan(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int w = 0; w < 16; ++w) {
      int t = wsum[w];
      wsum[w] = acc;
      acc += t;
    }
    wsum[16] = acc;
  }
  __syncthreads();
  const int r = incl - v + wsum[wave];
  *total = wsum[16];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(1024) void permute_kernel(const int32_t* __restrict__ ids, int T,
                                                       int E, int K, int32_t* meta,
                                                       int32_t* active, int32_t* offsets,
                                                       int32_t* counts, int32_t* perm_token,
                                                       int32_t* pos_of_slot, int32_t* tiles,
                                                       int32_t* slot_of_pos) {
  // LDS: bm[E][W] token bitmaps (64 tokens per word), then pre[E][W] = tokens routed to the
  // expert in the words before (u16), so a token's rank inside its expert is O(1).
  extern __shared__ uint64_t bm[];
  __shared__ int32_t off_s[kMaxExperts + 1];
  __shared__ int32_t wsum[17];
  const int W = (T + 63) / 64;
  uint16_t* pre = reinterpret_cast<uint16_t*>(bm + (size_t)E * W);
  const int n = T * K;
  for (int i = threadIdx.x; i < E * W; i += blockDim.x) bm[i] = 0ull;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = ids[i], t = i / K;
    atomicOr(reinterpret_cast<unsigned long long*>(&bm[e * W + (t >> 6)]), 1ull << (t & 63));
  }
  __syncthreads();
  // one expert per thread (E <= 512 < 1024): counts, offsets, active list, GEMM row tiles
  const int e = threadIdx.x;
  int c = 0;
  if (e < E)
    for (int w = 0; w < W; ++w) {
      pre[e * W + w] = (uint16_t)c;
      c += __popcll(bm[e * W + w]);
    }
  int total = 0, n_active = 0, n_tiles = 0;
  const int off = block_excl_scan(c, wsum, &total);
  const int slot = block_excl_scan(c > 0 ? 1 : 0, wsum, &n_active);
  const int nt = (c + kGemmMTile - 1) / kGemmMTile;
  const int toff = block_excl_scan(nt, wsum, &n_tiles);
  if (e < E) {
    counts[e] = c;
    offsets[e] = off;
    off_s[e] = off;
    if (c) active[slot] = e;
    for (int j = 0; j < nt; ++j) {
      tiles[2 * (toff + j)] = e;
      tiles[2 * (toff + j) + 1] = j * kGemmMTile;
    }
  }
  if (threadIdx.x == 0) {
    offsets[E] = total;
    meta[0] = n_active;
    meta[1] = n_tiles;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int ex = ids[i], t = i / K, w = t >> 6;
    const uint64_t below = bm[ex * W + w] & ((1ull << (t & 63)) - 1ull);
    const int p = off_s[ex] + pre[ex * W + w] + __popcll(below);
    pos_of_slot[i] = p;
    perm_token[p] = t;
    if (slot_of_pos) slot_of_pos[p] = i;
  }
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
                                                             int* status, unsigned* lo_word,
                                                             unsigned lo_gen,
                                                             u16* __restrict__ xb) {
  __shared__ __attribute__((aligned(16))) u16 a_hi[2][kMT * kALd];
  __shared__ __attribute__((aligned(16))) u16 a_lo[2][kMT * kALd];
  __shared__ __attribute__((aligned(16))) int lo_flag[2][4];  // per staging buffer, per wave
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
  // the workgroups also write x's hi halves (chunks c and 8 + c of the K step at k0, as
  // load_a read them) for the grouped GEMMs (Epi::xb): K step s of a token tile by expert
  // group s % gridDim.x, so each row and K step of x once, spread over the expert groups
  u16* xrow = xb && a_valid ? xb + (size_t)(m0 + am) * H : nullptr;
  auto put_xb = [&](const AStage& as, int k0) {
    if (!xrow || (k0 / kKS) % (int)gridDim.x != (int)blockIdx.x) return;
    const float* v = reinterpret_cast<const float*>(as.v);
    const int c = threadIdx.x & 7;
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = pk_bf16(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4*>(xrow + k0 + 8 * c) = make_uint4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<uint4*>(xrow + k0 + 64 + 8 * c) = make_uint4(h[4], h[5], h[6], h[7]);
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
    put_xb(as, s_begin * kKS);
    bool lo_any = barrier_or4(store_a(as, a_hi[0], a_lo[0]), lo_flag[0]);
    bool saw_lo = lo_any;
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
          put_xb(as, (s + 1) * kKS);
          lo_any = barrier_or4(store_a(as, a_hi[buf ^ 1], a_lo[buf ^ 1]), lo_flag[buf ^ 1]);
          saw_lo |= lo_any;
        }
      }
    }
    // the workgroup's rows had a non-zero lo half: the grouped GEMMs of this call keep theirs
    if (saw_lo && lo_word && threadIdx.x == 0) *lo_word = lo_gen;
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

// K slices of the batched router: as many as keep the launch within one round of two
// workgroups per CU (512), so no slice waits for a second round (1024 tokens over 384
// experts, hidden 7168: 3 slices, 576 workgroups -> 2 slices, 384: router 62 -> 48 us beside
// the shared expert, the layer 2.25 -> 2.24 ms).
int router_slices(int E, int H, int T) {
  const int steps = H / kKS;
  const int base = (router_rows(E) / kNT) * ((T + kMT - 1) / kMT);
  int slices = std::min(kRouterMaxSlices, std::max(1, 512 / base));
  slices = std::min(slices, std::max(1, steps / 2));
  const int per = (steps + slices - 1) / slices;
  return (steps + per - 1) / per;
}

// One token: the same f64 partial slices from a GEMV, one wavefront per (expert, slice) over
// the row-major router.  Lane l accumulates in f64 the exact products of its 8-column units
// l, l + 64, ... of the slice; the lanes' sums are then added in a fixed butterfly order.
__global__ __launch_bounds__(64) void router_gemv_f64_kernel(const uint16_t* __restrict__ w,
                                                             int E, int H,
                                                             const float* __restrict__ x,
                                                             int units_per_slice,
                                                             double* __restrict__ part,
                                                             int* status,
                                                             uint16_t* __restrict__ xp,
                                                             int xq) {
  const int e = blockIdx.x, z = blockIdx.y, lane = threadIdx.x;
  const int units = H / 8;
  const int u0 = z * units_per_slice, u1 = min(units, u0 + units_per_slice);
  const uint16_t* wr = w + (size_t)e * H;
  double acc = 0.0;
  bool bad = false;
  for (int u = u0 + lane; u < u1; u += 64) {
    const uint4 q = *reinterpret_cast<const uint4*>(wr + 8 * u);
    const float4 a = *reinterpret_cast<const float4*>(x + 8 * u);
    const float4 b = *reinterpret_cast<const float4*>(x + 8 * u + 4);
    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const float wv[8] = {bf16_lo(q.x), bf16_hi(q.x), bf16_lo(q.y), bf16_hi(q.y),
                         bf16_lo(q.z), bf16_hi(q.z), bf16_lo(q.w), bf16_hi(q.w)};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      bad |= !finite(xv[k]);
      acc += (double)wv[k] * (double)xv[k];
    }
  }
  if (bad) flag(status, kStatusNonFinite);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) part[(size_t)z * router_rows(E) + e] = acc;
  // the token's piece vector (the decode GEMVs' input), spread over the workgroups
  if (xp)
    token_pieces(x, H, xp, xq, status, (blockIdx.y * gridDim.x + blockIdx.x) * 64 + lane,
                 gridDim.x * gridDim.y * 64);
}

int router_gemv_slices(int E) {
  // enough waves to cover the chip four times over, at most kRouterMaxSlices
  return std::max(1, std::min(kRouterMaxSlices, (4 * 256 + E - 1) / E));
}

void launch_router_gemv_f64(const uint16_t* w, int E, int H, const float* x, double* part,
                            int slices, int* status, hipStream_t s, uint16_t* xp, int xq) {
  const int units = H / 8;
  const int per = (units + slices - 1) / slices;
  router_gemv_f64_kernel<<<dim3(E, slices), 64, 0, s>>>(w, E, H, x, per, part, status, xp, xq);
}

void launch_router_mfma(const uint8_t* wp, int E, int H, const float* x, int T, double* part,
                        int slices, int* status, hipStream_t s, unsigned* lo_word,
                        unsigned lo_gen, uint16_t* xb) {
  const int steps = H / kKS;
  const int per = (steps + slices - 1) / slices;
  dim3 grid(router_rows(E) / kNT, (T + kMT - 1) / kMT, slices);
  router_mfma_kernel<4><<<grid, 256, 0, s>>>(wp, router_rows(E), H, x, T, per, part, status,
                                             lo_word, lo_gen, xb);
}

void launch_relayout_lane8(const uint16_t* w, int E, int H, uint16_t* w8, hipStream_t s) {
  const int E8 = (E + 7) / 8 * 8;
  const size_t n = (size_t)E8 * H;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 65535);
  relayout_lane8_kernel<<<blocks, 256, 0, s>>>(w, E8, H, w8);
}

void launch_router_lane8(const uint16_t* w8, int E, int H, const float* x, int T, float* logits,
                         int round_bf16, int* status, hipStream_t s, uint16_t* xp,
                         const uint16_t* w8b, float* logits_b, int xq, unsigned* lo_word,
                         unsigned lo_gen) {
  const size_t per_tok = (size_t)8 * (H / 8 + 4) * sizeof(float);
  if (T < 64) {
    // One token per 64-thread workgroup: the most independent waves.  Each workgroup streams
    // its 8 experts' chains from L2, so the traffic grows with T x E x H ...
    const int gx = (E + 7) / 8 + (w8b ? 1 : 0);
    router_lane8_kernel<1><<<dim3(gx, T), 64, per_tok, s>>>(w8, E, H, x, T, logits, round_bf16,
                                                            status, xp, w8b, logits_b, xq,
                                                            lo_word, lo_gen);
    return;
  }
  if (w8b) {
    // batches: the one-row matrix as a launch of its own
    launch_router_lane8(w8b, 1, H, x, T, logits_b, round_bf16, status, s);
  }
  // ... from 64 tokens four waves share one staged token row (32 experts' chains per
  // workgroup; measured on MI355X at 128 tokens x 128 experts x 2048, 13.8 us with 64-thread
  // workgroups, 11.8 us with the chunked tiled kernel, 9.7 us with the whole row staged at
  // once; 128 x 256 x 2048, 22-26 -> 15-19 us), and beyond 512 tokens the tiled kernel divides
  // the weight traffic by streaming each chain batch for 8 or 16 tokens (bound by LDS reads of
  // the staged activations instead: 1024 tokens x 384 experts x 7168 from 1.74 ms to 0.29 ms).
  const int eg = (E + 31) / 32;
  if (T <= 512)
    router_lane8_kernel<1, 4><<<dim3(eg, T), 256, per_tok, s>>>(w8, E, H, x, T, logits,
                                                                round_bf16, status, nullptr,
                                                                nullptr, nullptr, 0, lo_word,
                                                                lo_gen);
  else if ((long)eg * ((T + 15) / 16) >= 256)
    router_lane8_tiled_kernel<16><<<dim3(eg, (T + 15) / 16), 256, 0, s>>>(w8, E, H, x, T, logits,
                                                                        round_bf16, status,
                                                                        lo_word, lo_gen);
  else
    router_lane8_tiled_kernel<8><<<dim3(eg, (T + 7) / 8), 256, 0, s>>>(w8, E, H, x, T, logits,
                                                                     round_bf16, status,
                                                                     lo_word, lo_gen);
}

template <int EPL>
static void launch_route_epl(float* logits, int T, int E, int K, const RouteParams& p,
                             int32_t* ids, float* weights, int32_t* asc, int* status,
                             hipStream_t s) {
  const dim3 grid((T + 3) / 4);
  if (p.router == 0)
    route_kernel<EPL, 0><<<grid, 256, 0, s>>>(logits, T, E, K, p, ids, weights, asc, status);
  else if (p.router == 1)
    route_kernel<EPL, 1><<<grid, 256, 0, s>>>(logits, T, E, K, p, ids, weights, asc, status);
  else
    route_kernel<EPL, 2><<<grid, 256, 0, s>>>(logits, T, E, K, p, ids, weights, asc, status);
}

void launch_route(float* logits, int T, int E, int K, const RouteParams& p, int32_t* ids,
                  float* weights, int32_t* asc, int* status, hipStream_t s) {
  const int epl = (E + 63) / 64;
  if (epl <= 1) launch_route_epl<1>(logits, T, E, K, p, ids, weights, asc, status, s);
  else if (epl <= 2) launch_route_epl<2>(logits, T, E, K, p, ids, weights, asc, status, s);
  else if (epl <= 4) launch_route_epl<4>(logits, T, E, K, p, ids, weights, asc, status, s);
  else launch_route_epl<8>(logits, T, E, K, p, ids, weights, asc, status, s);
}

void launch_permute(const int32_t* ids, int T, int E, int K, int32_t* meta, int32_t* active,
                    int32_t* offsets, int32_t* counts, int32_t* perm_token, int32_t* pos_of_slot,
                    int32_t* tiles, int32_t* slot_of_pos, hipStream_t s) {
  size_t lds = (size_t)E * ((T + 63) / 64) * (sizeof(uint64_t) + sizeof(uint16_t));
  permute_kernel<<<1, 1024, lds, s>>>(ids, T, E, K, meta, active, offsets, counts, perm_token,
                                      pos_of_slot, tiles, slot_of_pos);
}

}  // namespace urb
