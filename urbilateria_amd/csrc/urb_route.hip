// urb_route.hip -- router GEMV/GEMM, top-k routing and the token->expert permutation.
#include "urb_device.hpp"
#include "urb_kernels.hpp"

namespace urb {

// ------------------------------------------------------------------------------------------
// Qwen router: `linear(router)` = Bf16Matrix::matvec_fp32 + BF16 (src/models/qwen3_8/math.rs:
// 10-26).  The reference GEMV is the 8-lane FP32 FMA tree (src/model/bf16.rs:589-610): lane j
// accumulates columns == j (mod 8) in order, lanes are summed 0..7, the tail is added with a
// separate multiply and add.  One thread per (expert, lane) runs that exact chain, so the BF16
// logits -- and hence their exact ties -- are bit-identical to the reference.
// The weights are re-laid out once at create time so that each chain is contiguous:
//   w8[e][j][i] = w[e][8 i + j] for i < H/8, then the H % 8 tail columns of row e.
// ------------------------------------------------------------------------------------------
constexpr int kLane8Tokens = 4;

__global__ void relayout_lane8_kernel(const uint16_t* __restrict__ w, int E, int H,
                                      uint16_t* __restrict__ w8) {
  const int H8 = H / 8;
  size_t n = (size_t)E * H;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n;
       idx += (size_t)gridDim.x * blockDim.x) {
    size_t e = idx / H;
    int c = (int)(idx % H);
    size_t dst = c < 8 * H8 ? e * H + (size_t)(c % 8) * H8 + c / 8 : idx;
    w8[dst] = w[idx];
  }
}

__global__ __launch_bounds__(64) void router_lane8_kernel(const uint16_t* __restrict__ w8,
                                                          int E, int H,
                                                          const float* __restrict__ x, int T,
                                                          float* __restrict__ logits,
                                                          int* status) {
  extern __shared__ float xs[];  // [tok][8][H8 + 1] transposed chains, then [tok][tail]
  const int H8 = H / 8, tail = H - 8 * H8, H8p = H8 + 1;
  const int t0 = blockIdx.y * kLane8Tokens;
  const int nt = min(kLane8Tokens, T - t0);
  float* xt = xs + kLane8Tokens * 8 * H8p;
  for (int i = threadIdx.x; i < nt * H; i += blockDim.x) {
    int tt = i / H, c = i - tt * H;
    float v = x[(size_t)(t0 + tt) * H + c];
    if (!finite(v)) flag(status, kStatusNonFinite);
    if (c < 8 * H8) xs[(tt * 8 + (c & 7)) * H8p + (c >> 3)] = v;
    else xt[tt * tail + (c - 8 * H8)] = v;
  }
  __syncthreads();
  const int el = threadIdx.x >> 3, j = threadIdx.x & 7;
  const int e = blockIdx.x * 8 + el;
  float acc[kLane8Tokens] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (e < E) {
    const uint16_t* chain = w8 + (size_t)e * H + (size_t)j * H8;
    const float* xj = xs + j * H8p;
    if ((H8 & 7) == 0) {
      for (int i = 0; i < H8; i += 8) {
        uint4 q = *reinterpret_cast<const uint4*>(chain + i);
        float wv[8] = {bf16_lo(q.x), bf16_hi(q.x), bf16_lo(q.y), bf16_hi(q.y),
                       bf16_lo(q.z), bf16_hi(q.z), bf16_lo(q.w), bf16_hi(q.w)};
#pragma unroll
        for (int tt = 0; tt < kLane8Tokens; ++tt) {
          if (tt < nt) {
            const float* xv = xj + tt * 8 * H8p + i;
#pragma unroll
            for (int u = 0; u < 8; ++u) acc[tt] = fmaf(wv[u], xv[u], acc[tt]);
          }
        }
      }
    } else {
      for (int i = 0; i < H8; ++i) {
        float wv = u2f((uint32_t)chain[i] << 16);
        for (int tt = 0; tt < nt; ++tt) acc[tt] = fmaf(wv, xj[tt * 8 * H8p + i], acc[tt]);
      }
    }
  }
  // Lane sum in lane order 0..7, then the tail with separate multiply and add.
  const int base = el * 8;
  for (int tt = 0; tt < kLane8Tokens; ++tt) {
    float sum = __shfl(acc[tt], base + 0, 64);
#pragma unroll
    for (int u = 1; u < 8; ++u) sum = __fadd_rn(sum, __shfl(acc[tt], base + u, 64));
    if (e < E && j == 0 && tt < nt) {
      const uint16_t* tw = w8 + (size_t)e * H + 8 * H8;
      for (int c = 0; c < tail; ++c)
        sum = __fadd_rn(sum, __fmul_rn(u2f((uint32_t)tw[c] << 16), xt[tt * tail + c]));
      float r;
      if (!rne_bf16(sum, &r)) {
        flag(status, kStatusNonFinite);
        r = sum;
      }
      logits[(size_t)(t0 + tt) * E + e] = r;
    }
  }
}

// ------------------------------------------------------------------------------------------
// GLM router: `router.matvec` = Bf16Matrix::matvec_rows, ordered f64 (src/model/bf16.rs:
// 121-216).  Products bf16*f32 are exact in f64; the sum is reassociated across lanes (f64, so
// the f32 logit differs from the ordered sum only in rare last-bit cases).  One wavefront per
// expert, lanes over 8-column chunks, up to 8 tokens per block.
// ------------------------------------------------------------------------------------------
constexpr int kF64Tokens = 8;

__global__ __launch_bounds__(256) void router_f64_kernel(const uint16_t* __restrict__ w, int E,
                                                         int H, const float* __restrict__ x,
                                                         int T, float* __restrict__ logits,
                                                         int* status) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * kF64Tokens;
  const int nt = min(kF64Tokens, T - t0);
  if (e >= E) return;
  double acc[kF64Tokens];
#pragma unroll
  for (int tt = 0; tt < kF64Tokens; ++tt) acc[tt] = 0.0;
  const int H8 = H / 8;
  const uint16_t* row = w + (size_t)e * H;
  bool bad = false;
  for (int ch = lane; ch < H8; ch += 64) {
    uint4 q = *reinterpret_cast<const uint4*>(row + ch * 8);
    float wv[8] = {bf16_lo(q.x), bf16_hi(q.x), bf16_lo(q.y), bf16_hi(q.y),
                   bf16_lo(q.z), bf16_hi(q.z), bf16_lo(q.w), bf16_hi(q.w)};
#pragma unroll
    for (int tt = 0; tt < kF64Tokens; ++tt) {
      if (tt < nt) {
        const float4* xp = reinterpret_cast<const float4*>(x + (size_t)(t0 + tt) * H + ch * 8);
        float4 a = xp[0], b = xp[1];
        float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          bad |= !finite(xv[u]);
          acc[tt] = fma((double)wv[u], (double)xv[u], acc[tt]);
        }
      }
    }
  }
  for (int c = 8 * H8 + lane; c < H; c += 64) {
    double wv = (double)u2f((uint32_t)row[c] << 16);
    for (int tt = 0; tt < nt; ++tt) {
      float xv = x[(size_t)(t0 + tt) * H + c];
      bad |= !finite(xv);
      acc[tt] = fma(wv, (double)xv, acc[tt]);
    }
  }
  if (bad) flag(status, kStatusNonFinite);
#pragma unroll
  for (int tt = 0; tt < kF64Tokens; ++tt) {
    double s = wave_sum_f64(acc[tt]);
    if (lane == 0 && tt < nt) logits[(size_t)(t0 + tt) * E + e] = (float)s;
  }
}

// ------------------------------------------------------------------------------------------
// Top-k routing: one wavefront per token, experts spread over lanes (lane l holds experts
// l, l + 64, ...).  Ranking is iterated wave arg-max on (total-order key desc, expert id asc),
// the reference's sort comparator.  Sums the reference performs sequentially are performed
// sequentially here too (uniformly in every lane, reading from LDS).
// ------------------------------------------------------------------------------------------
constexpr int kMaxExperts = 512;
constexpr int kEPL = kMaxExperts / 64;
constexpr int kMaxTopK = 32;

// Packs (key desc, id asc) into one u64 whose maximum is the reference's first-ranked element.
__device__ __forceinline__ uint64_t rank_key(float v, int id) {
  return ((uint64_t)((uint32_t)total_key(v) ^ 0x80000000u) << 32) | (uint32_t)(0xffffffffu - id);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t other = __shfl_xor(v, o, 64);
    v = other > v ? other : v;
  }
  return v;
}

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int T,
                                                    int E, int K, RouteParams rp,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ weights,
                                                    int32_t* __restrict__ asc, int* status) {
  __shared__ float lds[4][kMaxExperts];
  __shared__ float grp[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  float* sh = lds[wave];
  const float* lt = logits + (size_t)t * E;
  float v[kEPL];
  bool valid[kEPL], taken[kEPL];
  bool bad = false;
#pragma unroll
  for (int i = 0; i < kEPL; ++i) {
    int e = lane + 64 * i;
    valid[i] = e < E;
    taken[i] = false;
    v[i] = valid[i] ? lt[e] : 0.0f;
    if (valid[i] && !finite(v[i])) bad = true;
  }
  int out_ids[kMaxTopK];
  float out_w[kMaxTopK];

  if (rp.router == 0) {
    // route_softmax_top_k (src/models/qwen3_8/moe.rs:91-159).
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kEPL; ++i)
      if (valid[i]) m = fmaxf(m, v[i]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float p[kEPL];
#pragma unroll
    for (int i = 0; i < kEPL; ++i) {
      p[i] = valid[i] ? exp_f32(v[i] - m) : 0.0f;
      if (valid[i]) sh[lane + 64 * i] = p[i];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float den = 0.0f;  // sequential, expert order
    for (int e = 0; e < E; ++e) den = __fadd_rn(den, sh[e]);
    if (!finite(den) || den <= 0.0f) bad = true;
#pragma unroll
    for (int i = 0; i < kEPL; ++i) {
      if (valid[i]) {
        p[i] = p[i] / den;
        if (!finite(p[i])) bad = true;
      }
    }
    float sel_sum = 0.0f;
    for (int r = 0; r < K; ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < kEPL; ++i)
        if (valid[i] && !taken[i]) {
          uint64_t k = rank_key(p[i], lane + 64 * i);
          best = k > best ? k : best;
        }
      best = wave_max_u64(best);
      int id = (int)(0xffffffffu - (uint32_t)best);
      float pv = 0.0f;
#pragma unroll
      for (int i = 0; i < kEPL; ++i)
        if (lane + 64 * i == id) { taken[i] = true; pv = p[i]; }
      pv = __shfl(pv, id & 63, 64);
      out_ids[r] = id;
      out_w[r] = pv;
      sel_sum = __fadd_rn(sel_sum, pv);
    }
    if (!finite(sel_sum) || sel_sum <= 0.0f) bad = true;
    for (int r = 0; r < K; ++r) {
      float w = out_w[r] / sel_sum;
      if (!finite(w)) bad = true;
      if (rp.qwen) {  // qwen3_6/runtime.rs:1233-1238: route weights materialised in BF16
        float q;
        if (!rne_bf16(w, &q)) { bad = true; q = w; }
        w = q;
      }
      out_w[r] = w;
    }
  } else {
    // route_noaux_tc (src/math/routing.rs:38-155).
    float g[kEPL], s[kEPL];
#pragma unroll
    for (int i = 0; i < kEPL; ++i) {
      int e = lane + 64 * i;
      g[i] = valid[i] ? 1.0f / (1.0f + exp_f32(-v[i])) : 0.0f;
      float b = (valid[i] && rp.bias) ? rp.bias[e] : 0.0f;
      s[i] = __fadd_rn(g[i], b);
      if (valid[i]) sh[e] = s[i];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int per = E / rp.n_group;
    // group score = sum of the two largest selection scores (:104-111)
    if (lane < rp.n_group) {
      int32_t k1 = INT32_MIN, k2 = INT32_MIN;
      float b1 = 0.0f, b2 = 0.0f;
      for (int i = 0; i < per; ++i) {
        float sv = sh[lane * per + i];
        int32_t k = total_key(sv);
        if (k > k1) { k2 = k1; b2 = b1; k1 = k; b1 = sv; }
        else if (k > k2) { k2 = k; b2 = sv; }
      }
      grp[wave][lane] = __fadd_rn(b1, b2);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // keep the top `topk_group` groups (score desc, id asc)
    bool gsel = false;
    float gs = lane < rp.n_group ? grp[wave][lane] : 0.0f;
    for (int r = 0; r < rp.topk_group; ++r) {
      uint64_t k = (lane < rp.n_group && !gsel) ? rank_key(gs, lane) : 0;
      k = wave_max_u64(k);
      int id = (int)(0xffffffffu - (uint32_t)k);
      if (lane == id) gsel = true;
    }
    uint64_t gmask = __ballot(gsel);
    for (int r = 0; r < K; ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < kEPL; ++i) {
        int e = lane + 64 * i;
        if (valid[i] && !taken[i] && ((gmask >> (e / per)) & 1ull)) {
          uint64_t k = rank_key(s[i], e);
          best = k > best ? k : best;
        }
      }
      best = wave_max_u64(best);
      int id = (int)(0xffffffffu - (uint32_t)best);
      float gv = 0.0f;
#pragma unroll
      for (int i = 0; i < kEPL; ++i)
        if (lane + 64 * i == id) { taken[i] = true; gv = g[i]; }
      gv = __shfl(gv, id & 63, 64);
      out_ids[r] = id;
      out_w[r] = gv;
    }
    float den = -0.0f;
    for (int r = 0; r < K; ++r) den = __fadd_rn(den, out_w[r]);
    den = __fadd_rn(den, 1e-20f);
    if (rp.normalize && !finite(den)) bad = true;
    for (int r = 0; r < K; ++r) {
      float w = rp.normalize ? out_w[r] / den : out_w[r];
      out_w[r] = __fmul_rn(w, rp.scale);
    }
  }
  if (bad) flag(status, kStatusNonFinite);
  if (lane == 0) {
    for (int r = 0; r < K; ++r) {
      ids[(size_t)t * K + r] = out_ids[r];
      weights[(size_t)t * K + r] = out_w[r];
    }
    if (asc) {
      // ranking positions ordered by ascending expert id (qwen3_6/runtime.rs:1239-1240)
      int order[kMaxTopK];
      for (int r = 0; r < K; ++r) order[r] = r;
      for (int a = 1; a < K; ++a) {
        int cur = order[a], b = a - 1;
        while (b >= 0 && out_ids[order[b]] > out_ids[cur]) { order[b + 1] = order[b]; --b; }
        order[b + 1] = cur;
      }
      for (int r = 0; r < K; ++r) asc[(size_t)t * K + r] = order[r];
    }
  }
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
                                                       int32_t* pos_of_slot, int32_t* tiles) {
  extern __shared__ uint32_t bm[];  // [E][W]
  __shared__ int32_t off_s[kMaxExperts + 1];
  __shared__ int32_t wsum[17];
  const int W = (T + 31) / 32;
  const int n = T * K;
  for (int i = threadIdx.x; i < E * W; i += blockDim.x) bm[i] = 0u;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    int e = ids[i], t = i / K;
    atomicOr(&bm[e * W + (t >> 5)], 1u << (t & 31));
  }
  __syncthreads();
  // one expert per thread (E <= 512 < 1024): counts, offsets, active list, GEMM row tiles
  const int e = threadIdx.x;
  int c = 0;
  if (e < E)
    for (int w = 0; w < W; ++w) c += __popc(bm[e * W + w]);
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
    int e = ids[i], t = i / K;
    const uint32_t* row = bm + e * W;
    int rank = __popc(row[t >> 5] & ((1u << (t & 31)) - 1u));
    for (int w = 0; w < (t >> 5); ++w) rank += __popc(row[w]);
    int p = off_s[e] + rank;
    pos_of_slot[i] = p;
    perm_token[p] = t;
  }
}

// ------------------------------------------------------------------------------------------
void launch_relayout_lane8(const uint16_t* w, int E, int H, uint16_t* w8, hipStream_t s) {
  size_t n = (size_t)E * H;
  int blocks = (int)std::min<size_t>((n + 255) / 256, 65535);
  relayout_lane8_kernel<<<blocks, 256, 0, s>>>(w, E, H, w8);
}

void launch_router_lane8(const uint16_t* w8, int E, int H, const float* x, int T, float* logits,
                         int* status, hipStream_t s) {
  const int H8 = H / 8, tail = H - 8 * H8;
  size_t lds = (size_t)kLane8Tokens * (8 * (H8 + 1) + tail) * sizeof(float);
  dim3 grid((E + 7) / 8, (T + kLane8Tokens - 1) / kLane8Tokens);
  router_lane8_kernel<<<grid, 64, lds, s>>>(w8, E, H, x, T, logits, status);
}

void launch_router_f64(const uint16_t* w, int E, int H, const float* x, int T, float* logits,
                       int* status, hipStream_t s) {
  dim3 grid((E + 3) / 4, (T + kF64Tokens - 1) / kF64Tokens);
  router_f64_kernel<<<grid, 256, 0, s>>>(w, E, H, x, T, logits, status);
}

void launch_route(const float* logits, int T, int E, int K, const RouteParams& p, int32_t* ids,
                  float* weights, int32_t* asc, int* status, hipStream_t s) {
  route_kernel<<<(T + 3) / 4, 256, 0, s>>>(logits, T, E, K, p, ids, weights, asc, status);
}

void launch_permute(const int32_t* ids, int T, int E, int K, int32_t* meta, int32_t* active,
                    int32_t* offsets, int32_t* counts, int32_t* perm_token, int32_t* pos_of_slot,
                    int32_t* tiles, hipStream_t s) {
  size_t lds = (size_t)E * ((T + 31) / 32) * sizeof(uint32_t);
  permute_kernel<<<1, 1024, lds, s>>>(ids, T, E, K, meta, active, offsets, counts, perm_token,
                                      pos_of_slot, tiles);
}

}  // namespace urb
