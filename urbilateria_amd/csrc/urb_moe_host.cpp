// urb_moe_host.cpp -- the C ABI (include/urb_moe.h): layer construction, validation, HBM
// arena, workspace and the per-call launch sequence.
#include "../../include/urb_moe.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "urb_kernels.hpp"

namespace {

using urb::ExpertMats;
using urb::Perm;

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

size_t matrix_bytes(urb_format f, size_t rows, size_t cols, size_t* scales) {
  *scales = f == URB_FMT_BF16 ? 0 : rows * (cols / 32);
  switch (f) {
    case URB_FMT_BF16: return rows * cols * 2;
    case URB_FMT_MXFP4: return rows * cols / 2;
    default: return rows * cols;
  }
}

struct Workspace {
  float* logits = nullptr;
  double* router_part = nullptr;  // GLM router f64 partial slices
  int32_t* ids = nullptr;
  float* weights = nullptr;
  int32_t* asc = nullptr;
  int32_t* meta = nullptr;
  int32_t* active = nullptr;
  int32_t* offsets = nullptr;
  int32_t* counts = nullptr;
  int32_t* perm_token = nullptr;
  int32_t* pos_of_slot = nullptr;
  int32_t* slot_of_pos = nullptr;  // DSV41, DSV4: route slot of each permuted position
  int32_t* tiles = nullptr;
  float* act = nullptr;
  float* y_perm = nullptr;
  float* shared_act = nullptr;
  float* shared_out = nullptr;
  float* xq = nullptr;  // HY4, DSV41, DSV4: the simulated E4M3 token activations [chunk, H]
  float* xn = nullptr;  // QWEN36 block calls: the normalized BF16 token activations [chunk, H]
  float* gate_logit = nullptr;  // QWEN36 shared expert: bf16(shared_expert_gate . x) [chunk]
  int32_t* rowexp = nullptr;    // GLM, MX experts: [chunk * k, gate/up panel groups]
  int32_t* shared_rowexp = nullptr;  // GLM, f16 shared down: [chunk] row exponents
  // one-token calls: BF16 piece vectors (urb_panel.hpp) of the token, the k SwiGLU rows and
  // the shared expert's SwiGLU row, the decode GEMVs' A operands
  uint16_t* xp = nullptr;
  uint16_t* act_xp = nullptr;
  uint16_t* shared_xp = nullptr;
  int* status = nullptr;  // [0] latched numerical failures, [1] validation flags
  // status + 4: the batched router's lo-half word (urb::Epi::lo_word), in the status block's
  // allocation so that it stays the context's own in no-alloc calls
  unsigned* lo_word = nullptr;
  // the batched MFMA router's BF16 copy of a chunk's token rows [chunk, H] (urb::Epi::xb;
  // contexts whose batches route with router_mfma_kernel, outside the allocation-free call)
  uint16_t* xb = nullptr;
};

// Sequential bump allocator over one device allocation.
struct Bump {
  char* base;
  size_t off = 0;
  template <class T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += align_up(count * sizeof(T));
    return p;
  }
};

}  // namespace

struct urb_moe_ctx {
  urb_moe_desc desc{};
  int device = 0;
  uint32_t chunk = 0;                  // tokens per internal launch sequence
  void* arena = nullptr;               // router, bias and (unless borrowed) the expert weights
  size_t arena_bytes = 0, weight_bytes = 0;
  void* work = nullptr;
  size_t work_bytes = 0;
  const uint16_t* router = nullptr;    // [E, H] BF16 (rows zero-padded to router_rows(E))
  uint16_t* router_lane8 = nullptr;    // per-lane chain layout (QWEN36, DSV41)
  uint16_t* shared_gate8 = nullptr;    // QWEN36 shared expert gate row, per-lane chain layout
  bool borrowed = false;               // experts borrowed in the panel layout (repointable)
  uint8_t* router_panel = nullptr;     // panel layout of the padded router (GLM)
  const float* bias = nullptr;         // [E] or nullptr
  const int32_t* hash = nullptr;       // [hash_vocab, K] tid2eid rows (sqrt-softplus) or nullptr
  uint32_t hash_vocab = 0;
  ExpertMats* table = nullptr;         // device [E]
  ExpertMats* shared_table = nullptr;  // device [1]
  ExpertMats shared_host{};            // the same pointers on the host
  // GLM with a BF16 shared expert: its down matrix as f16 times 2^shared_wshift, in the BF16
  // panel layout (urb::bf16_f16_shift; absent when its values span more than f16 holds
  // exactly, or when the weights are borrowed), for batches whose shared gate+up runs on the
  // dense kernel: the down projection then runs on f16 MFMAs from f16 SwiGLU rows
  // (urb::launch_dense_down_f16)
  uint16_t* shared16 = nullptr;
  int shared_wshift = 0;
  // GLM batches with MX experts: the down projection runs on f16 MFMAs from row-scaled f16
  // activations (urb::Epi::rowexp) -- every down matrix's E8M0 codes keep its weights exact in
  // f16 (checked at create and by urb_moe_set_expert, which clears it otherwise)
  bool down_f16 = false;
  unsigned lo_gen = 0;  // generation of the batched router's lo-half word, one per chunk
  Workspace ws;
  hipStream_t side = nullptr;          // shared expert runs here, concurrently with routing
  hipEvent_t fork = nullptr, join = nullptr;
  // stage spans (urb_moe_profile)
  bool profiling = false;
  hipEvent_t ev[URB_STAGE_COUNT][2] = {};
  bool pending[URB_STAGE_COUNT] = {};
  double stage_ms[URB_STAGE_COUNT] = {};
  uint64_t stage_calls[URB_STAGE_COUNT] = {};
};

namespace {

// Brackets one stage's launches with events on the stream they run on (profiling only).
struct Span {
  urb_moe_ctx* c;
  int stage;
  hipStream_t s;
  Span(urb_moe_ctx* c_, int stage_, hipStream_t s_) : c(c_), stage(stage_), s(s_) {
    if (c->profiling) (void)hipEventRecord(c->ev[stage][0], s);
  }
  ~Span() {
    if (c->profiling) {
      (void)hipEventRecord(c->ev[stage][1], s);
      c->pending[stage] = true;
    }
  }
};

urb_status collect_spans(urb_moe_ctx* c) {
  for (int st = 0; st < URB_STAGE_COUNT; ++st) {
    if (!c->pending[st]) continue;
    c->pending[st] = false;
    if (hipEventSynchronize(c->ev[st][1]) != hipSuccess) return URB_ERR_DEVICE;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, c->ev[st][0], c->ev[st][1]) != hipSuccess) return URB_ERR_DEVICE;
    c->stage_ms[st] += ms;
    c->stage_calls[st] += 1;
  }
  return URB_OK;
}

}  // namespace

#define URB_HIP(call)                            \
  do {                                           \
    hipError_t e_ = (call);                      \
    if (e_ == hipErrorOutOfMemory) return URB_ERR_OUT_OF_MEMORY; \
    if (e_ != hipSuccess) return URB_ERR_DEVICE; \
  } while (0)

extern "C" {

const char* urb_status_string(urb_status s) {
  switch (s) {
    case URB_OK: return "ok";
    case URB_ERR_SHAPE: return "invalid shape";
    case URB_ERR_INVALID_SCALE: return "E8M0 scale byte 0xff is NaN";
    case URB_ERR_NONFINITE: return "NaN or infinity";
    case URB_ERR_INVALID_GEOMETRY: return "invalid router geometry";
    case URB_ERR_DEVICE: return "HIP runtime error";
    case URB_ERR_OUT_OF_MEMORY: return "out of device memory";
    case URB_ERR_ARGUMENT: return "invalid argument";
  }
  return "unknown status";
}

}  // extern "C"

constexpr uint32_t kMaxDim = 12288;

// The MX-activation compositions (Hy4, DeepSeek V4.1, DeepSeek V4).
static bool mx_activation(urb_composition c) {
  return c == URB_COMPOSE_HY4 || c == URB_COMPOSE_DSV41 || c == URB_COMPOSE_DSV4;
}

static bool finite_host(float v) { return v == v && v <= 3.4028235e38f && v >= -3.4028235e38f; }

static urb_status check_desc(const urb_moe_desc* d) {
  if (d->hidden == 0 || d->n_experts == 0 || d->intermediate == 0 || d->max_tokens == 0)
    return URB_ERR_SHAPE;
  if (d->top_k == 0 || d->top_k > d->n_experts) return URB_ERR_INVALID_GEOMETRY;
  if (d->top_k > 32 || d->n_experts > 512) return URB_ERR_ARGUMENT;
  for (urb_format f : {d->expert_format, d->shared_format})
    if (f != URB_FMT_BF16 && f != URB_FMT_MXFP4 && f != URB_FMT_MXFP8) return URB_ERR_ARGUMENT;
  // Panel layout: every projection dimension a multiple of 128 columns (16-row panels follow).
  // The decode kernels stage one input vector in LDS: at most kMaxDim columns.
  for (uint32_t dim : {d->hidden, d->intermediate, d->shared_intermediate})
    if (dim % urb::kPanelCols || dim > kMaxDim) return URB_ERR_SHAPE;
  if (d->composition == URB_COMPOSE_QWEN36) {
    // The Qwen3.6 composition: BF16 experts, softmax router, an optional BF16 shared expert.
    if (d->expert_format != URB_FMT_BF16 || d->router != URB_ROUTER_SOFTMAX_TOPK ||
        (d->shared_intermediate && d->shared_format != URB_FMT_BF16))
      return URB_ERR_ARGUMENT;
  } else if (mx_activation(d->composition)) {
    // MX projections only (the activation mode exists for MX weights), and the routed experts'
    // SwiGLU limit must be finite and positive (Hy4Config validation, hy4/config.rs:235-236).
    if (d->expert_format == URB_FMT_BF16 ||
        (d->shared_intermediate && d->shared_format == URB_FMT_BF16))
      return URB_ERR_ARGUMENT;
    if (!finite_host(d->swiglu_limit)) return URB_ERR_NONFINITE;
    if (d->swiglu_limit <= 0.0f) return URB_ERR_INVALID_GEOMETRY;
  } else if (d->composition != URB_COMPOSE_GLM) {
    return URB_ERR_ARGUMENT;
  }
  if (d->router == URB_ROUTER_SIGMOID_NOAUX_TC) {
    // route_noaux_tc geometry (src/math/routing.rs:66-112), checked once at construction as
    // RuntimeMoeLayer::new does (src/models/glm/runtime/moe.rs:108-116).
    if (!finite_host(d->routed_scaling_factor)) return URB_ERR_NONFINITE;
    if (d->routed_scaling_factor <= 0.0f) return URB_ERR_INVALID_GEOMETRY;
    if (d->n_group == 0 || d->n_experts % d->n_group) return URB_ERR_INVALID_GEOMETRY;
    if (d->topk_group == 0 || d->topk_group > d->n_group) return URB_ERR_INVALID_GEOMETRY;
    uint32_t per = d->n_experts / d->n_group;
    if (per < 2) return URB_ERR_INVALID_GEOMETRY;
    if (per * d->topk_group < d->top_k) return URB_ERR_INVALID_GEOMETRY;
    if (d->n_group > 64) return URB_ERR_ARGUMENT;
  } else if (d->router == URB_ROUTER_SQRT_SOFTPLUS) {
    // route_sqrt_softplus: validate_positive(routed_scaling_factor) (deepseek_v4/math.rs:468)
    if (d->composition == URB_COMPOSE_QWEN36) return URB_ERR_ARGUMENT;
    if (!finite_host(d->routed_scaling_factor)) return URB_ERR_NONFINITE;
    if (d->routed_scaling_factor <= 0.0f) return URB_ERR_INVALID_GEOMETRY;
  } else if (d->router != URB_ROUTER_SOFTMAX_TOPK) {
    return URB_ERR_ARGUMENT;
  }
  return URB_OK;
}

static void destroy_ctx(urb_moe_ctx* c) {
  if (!c) return;
  for (auto& pair : c->ev)
    for (hipEvent_t e : pair)
      if (e) (void)hipEventDestroy(e);
  if (c->side) (void)hipStreamDestroy(c->side);
  if (c->fork) (void)hipEventDestroy(c->fork);
  if (c->join) (void)hipEventDestroy(c->join);
  if (c->arena) (void)hipFree(c->arena);
  if (c->work) (void)hipFree(c->work);
  if (c->shared16) (void)hipFree(c->shared16);
  delete c;
}

// The per-call buffers for chunks of up to `chunk` tokens, carved from one region into `w`
// (a Bump with a null base only sizes the region: every pointer it hands out is null).
// Panel groups of the routed gate/up launch (one rowexp column each).
static size_t rowexp_groups(const urb_moe_desc& d) {
  const int np = urb::gemm_panels_per_wave((int)d.expert_format, (int)d.intermediate, true, 0);
  return d.intermediate / (urb::kGemmNTile * (size_t)np);
}

static void carve_workspace(const urb_moe_ctx* c, Bump& b, size_t chunk, Workspace& w,
                            bool with_xb = true) {
  const urb_moe_desc& d = c->desc;
  const size_t C = chunk, E = d.n_experts, K = d.top_k, H = d.hidden, I = d.intermediate;
  w.status = b.take<int>(8);
  w.lo_word = reinterpret_cast<unsigned*>(w.status + 4);
  w.logits = b.take<float>(C * E);
  if (d.composition != URB_COMPOSE_QWEN36) {
    size_t most = 0;  // largest slices x tokens any call can need
    for (size_t t = 1; t <= C; ++t)
      most = std::max(most, (size_t)urb::router_slices((int)E, (int)H, (int)t) * t);
    most = std::max(most, (size_t)urb::router_gemv_slices((int)E));
    w.router_part = b.take<double>(most * urb::router_rows((int)E));
  }
  w.ids = b.take<int32_t>(C * K);
  w.weights = b.take<float>(C * K);
  w.asc = b.take<int32_t>(C * K);
  w.meta = b.take<int32_t>(4);
  w.active = b.take<int32_t>(E);
  w.offsets = b.take<int32_t>(E + 1);
  w.counts = b.take<int32_t>(E);
  w.perm_token = b.take<int32_t>(C * K);
  w.pos_of_slot = b.take<int32_t>(C * K);
  if (d.composition == URB_COMPOSE_DSV41 || d.composition == URB_COMPOSE_DSV4)
    w.slot_of_pos = b.take<int32_t>(C * K);
  w.tiles = b.take<int32_t>(2 * (size_t)urb::gemm_max_tiles((int)C, (int)K, (int)E));
  w.act = b.take<float>(C * K * I);
  w.y_perm = b.take<float>(C * K * H);
  w.shared_act = b.take<float>(C * std::max<size_t>(d.shared_intermediate, 1));
  w.shared_out = b.take<float>(C * H);
  if (mx_activation(d.composition)) w.xq = b.take<float>(C * H);
  // the routed gate+up reads the rows the router read only outside the MX-activation
  // compositions (those read their quantized rows); the 8-lane routers write no copy
  const bool lane8 = d.composition == URB_COMPOSE_QWEN36 || d.composition == URB_COMPOSE_DSV41;
  if (with_xb && !lane8 && !mx_activation(d.composition)) w.xb = b.take<uint16_t>(C * H);
  if (d.composition == URB_COMPOSE_QWEN36) w.xn = b.take<float>(C * H);
  if (d.composition == URB_COMPOSE_QWEN36 && d.shared_intermediate) w.gate_logit = b.take<float>(C);
  if (d.composition == URB_COMPOSE_GLM && d.expert_format != URB_FMT_BF16)
    w.rowexp = b.take<int32_t>(C * K * rowexp_groups(d));
  if (d.composition == URB_COMPOSE_GLM && d.shared_intermediate && d.shared_format == URB_FMT_BF16)
    w.shared_rowexp = b.take<int32_t>(C);
  w.xp = b.take<uint16_t>(H / 8 * urb::kPieceUnit);
  w.act_xp = b.take<uint16_t>(K * (I / 8) * urb::kPieceUnit);
  w.shared_xp = b.take<uint16_t>(std::max<size_t>(d.shared_intermediate, 8) / 8 *
                                 urb::kPieceUnit);
}

static urb_status create_impl(const urb_moe_desc* d, const urb_moe_weights* w,
                              urb_weight_source src, urb_moe_ctx* c) {
  const size_t H = d->hidden, E = d->n_experts, I = d->intermediate, Is = d->shared_intermediate;
  const bool has_shared = Is != 0;
  const bool qwen = d->composition == URB_COMPOSE_QWEN36;
  // the 8-lane FP32 router tree reads a lane-chain copy; the f64 MFMA router a panel copy
  const bool lane8 = qwen || d->composition == URB_COMPOSE_DSV41;
  if (!w->router_weight || !w->experts || (has_shared && !w->shared)) return URB_ERR_ARGUMENT;
  const bool qwen_gate = qwen && has_shared;
  if (qwen_gate && !w->shared_expert_gate) return URB_ERR_ARGUMENT;
  // hash experts: route_sqrt_softplus only, ids in range (deepseek_v4/math.rs:483-489) and,
  // for the permutation, distinct within a row
  const bool hashed = w->hash_experts != nullptr;
  if (hashed && d->router != URB_ROUTER_SQRT_SOFTPLUS) return URB_ERR_ARGUMENT;
  if (hashed && w->hash_vocab == 0) return URB_ERR_SHAPE;
  if (src != URB_SOURCE_HOST && src != URB_SOURCE_DEVICE_COPY && src != URB_SOURCE_DEVICE_BORROW)
    return URB_ERR_ARGUMENT;
  const bool mx = d->expert_format != URB_FMT_BF16;
  for (size_t i = 0; i < E * 3; ++i)
    if (!w->experts[i].data || (mx && !w->experts[i].scales)) return URB_ERR_ARGUMENT;
  if (has_shared)
    for (int i = 0; i < 3; ++i)
      if (!w->shared[i].data || (d->shared_format != URB_FMT_BF16 && !w->shared[i].scales))
        return URB_ERR_ARGUMENT;
  URB_HIP(hipGetDevice(&c->device));
  c->desc = *d;
  // The permutation keeps [E][chunk/64] 64-bit token bitmaps and u16 prefix counts in LDS:
  // cap them at 60 KiB.
  const uint32_t bitmap_chunk = (uint32_t)(60 * 1024 / (10 * E)) * 64;
  c->chunk = std::min<uint32_t>({d->max_tokens, (uint32_t)urb::kMaxChunkTokens, bitmap_chunk});

  const bool borrow = src == URB_SOURCE_DEVICE_BORROW;
  c->borrowed = borrow;
  const hipMemcpyKind kind = src == URB_SOURCE_HOST ? hipMemcpyHostToDevice
                                                    : hipMemcpyDeviceToDevice;
  if (!borrow) URB_HIP(hipDeviceSynchronize());  // device sources may come from any stream
  // Matrix geometry: gate [I, H], up [I, H], down [H, I].
  const size_t dims[3][2] = {{I, H}, {I, H}, {H, I}};
  const size_t sdims[3][2] = {{Is, H}, {Is, H}, {H, Is}};

  // ---- arena: router, lane-chain router, bias, then the expert payloads (unless borrowed)
  const size_t Ep = urb::router_rows((int)E);
  size_t arena = align_up(Ep * H * 2) + (lane8 ? align_up((E + 7) / 8 * 8 * H * 2) : align_up(Ep * H * 2)) +
                 align_up(E * 4) + (qwen_gate ? 2 * align_up(8 * H * 2) : 0) +
                 (hashed ? align_up((size_t)w->hash_vocab * d->top_k * 4) : 0);
  size_t wbytes = 0;
  if (!borrow) {
    for (int m = 0; m < 3; ++m) {
      size_t sb, db = matrix_bytes(d->expert_format, dims[m][0], dims[m][1], &sb);
      wbytes += E * (align_up(db) + align_up(sb));
      if (has_shared) {
        size_t ssb, sdb = matrix_bytes(d->shared_format, sdims[m][0], sdims[m][1], &ssb);
        wbytes += align_up(sdb) + align_up(ssb);
      }
    }
  }
  arena += wbytes + align_up(sizeof(ExpertMats) * (E + 1));
  URB_HIP(hipMalloc(&c->arena, arena));
  c->arena_bytes = arena;
  c->weight_bytes = wbytes;
  Bump ab{static_cast<char*>(c->arena)};
  uint16_t* router = ab.take<uint16_t>(Ep * H);
  c->router_lane8 = lane8 ? ab.take<uint16_t>((E + 7) / 8 * 8 * H) : nullptr;
  c->router_panel = lane8 ? nullptr : ab.take<uint8_t>(Ep * H * 2);
  float* bias = ab.take<float>(E);
  c->table = ab.take<ExpertMats>(E);
  c->shared_table = ab.take<ExpertMats>(1);
  // the shared expert's gate row as an 8-row lane-chain block (rows 1..7 zero)
  uint16_t* gate_rows = qwen_gate ? ab.take<uint16_t>(8 * H) : nullptr;
  c->shared_gate8 = qwen_gate ? ab.take<uint16_t>(8 * H) : nullptr;
  if (qwen_gate) {
    urb::launch_fill_i32(reinterpret_cast<int32_t*>(gate_rows), 0, 8 * H / 2, nullptr);
    URB_HIP(hipMemcpy(gate_rows, w->shared_expert_gate, H * 2, kind));
  }
  if (hashed) {
    // tid2eid as stored (i64), checked and narrowed on the host
    const size_t n = (size_t)w->hash_vocab * d->top_k, K = d->top_k;
    std::vector<int64_t> tab(n);
    URB_HIP(hipMemcpy(tab.data(), w->hash_experts, n * 8,
                      src == URB_SOURCE_HOST ? hipMemcpyHostToHost : hipMemcpyDeviceToHost));
    std::vector<int32_t> narrow(n);
    for (size_t i = 0; i < n; ++i) {
      if (tab[i] < 0 || tab[i] >= (int64_t)E) return URB_ERR_INVALID_GEOMETRY;
      narrow[i] = (int32_t)tab[i];
    }
    for (size_t r = 0; r < w->hash_vocab; ++r)
      for (size_t i = 0; i < K; ++i)
        for (size_t j = i + 1; j < K; ++j)
          if (narrow[r * K + i] == narrow[r * K + j]) return URB_ERR_ARGUMENT;
    int32_t* hash = ab.take<int32_t>(n);
    URB_HIP(hipMemcpy(hash, narrow.data(), n * 4, hipMemcpyHostToDevice));
    c->hash = hash;
    c->hash_vocab = w->hash_vocab;
  }
  URB_HIP(hipMemcpy(router, w->router_weight, E * H * 2, kind));
  if (Ep > E) urb::launch_fill_i32(reinterpret_cast<int32_t*>(router + E * H), 0, (Ep - E) * H / 2,
                                   nullptr);
  c->router = router;
  if (w->correction_bias) {
    URB_HIP(hipMemcpy(bias, w->correction_bias, E * 4, kind));
    c->bias = bias;
  }

  // Payloads enter HBM in the panel layout.  Host sources go through one staging buffer the
  // size of the largest matrix; device sources are converted directly.  Borrowed memory must
  // already be in the panel layout (urb_pack_matrix).
  void* staging = nullptr;
  if (src == URB_SOURCE_HOST) {
    size_t most = 0;
    for (int m = 0; m < 3; ++m) {
      size_t sb, db = matrix_bytes(d->expert_format, dims[m][0], dims[m][1], &sb);
      most = std::max(most, align_up(db) + sb);
      if (has_shared) {
        db = matrix_bytes(d->shared_format, sdims[m][0], sdims[m][1], &sb);
        most = std::max(most, align_up(db) + sb);
      }
    }
    URB_HIP(hipMalloc(&staging, most));
  }
  struct StagingFree {
    void* p;
    ~StagingFree() { if (p) { (void)hipDeviceSynchronize(); (void)hipFree(p); } }
  } staging_free{staging};
  std::vector<ExpertMats> table(E);
  auto place = [&](urb_format f, size_t rows, size_t cols, const urb_matrix& mat,
                   const uint8_t** data, const uint8_t** scales) -> urb_status {
    size_t sb, db = matrix_bytes(f, rows, cols, &sb);
    if (borrow) {
      *data = static_cast<const uint8_t*>(mat.data);
      *scales = sb ? mat.scales : nullptr;
      return URB_OK;
    }
    uint8_t* dd = ab.take<uint8_t>(db);
    uint8_t* ss = sb ? ab.take<uint8_t>(sb) : nullptr;
    const uint8_t* from = static_cast<const uint8_t*>(mat.data);
    const uint8_t* from_scales = mat.scales;
    if (staging) {
      uint8_t* st = static_cast<uint8_t*>(staging);
      URB_HIP(hipMemcpy(st, mat.data, db, hipMemcpyHostToDevice));
      if (sb) URB_HIP(hipMemcpy(st + align_up(db), mat.scales, sb, hipMemcpyHostToDevice));
      from = st;
      from_scales = sb ? st + align_up(db) : nullptr;
    }
    urb::launch_pack(f, from, from_scales, (int)rows, (int)cols, dd, ss, nullptr);
    URB_HIP(hipGetLastError());
    if (staging) URB_HIP(hipDeviceSynchronize());  // the staging buffer is reused
    *data = dd;
    *scales = ss;
    return URB_OK;
  };
  for (size_t e = 0; e < E; ++e)
    for (int m = 0; m < 3; ++m) {
      urb_status st = place(d->expert_format, dims[m][0], dims[m][1], w->experts[e * 3 + m],
                            &table[e].data[m], &table[e].scales[m]);
      if (st) return st;
    }
  ExpertMats shared{};
  if (has_shared)
    for (int m = 0; m < 3; ++m) {
      urb_status st = place(d->shared_format, sdims[m][0], sdims[m][1], w->shared[m],
                            &shared.data[m], &shared.scales[m]);
      if (st) return st;
    }
  URB_HIP(hipMemcpy(c->table, table.data(), sizeof(ExpertMats) * E, hipMemcpyHostToDevice));
  URB_HIP(hipMemcpy(c->shared_table, &shared, sizeof(ExpertMats), hipMemcpyHostToDevice));
  c->shared_host = shared;

  // ---- workspace
  Workspace unsized;
  Bump sizing{nullptr};
  carve_workspace(c, sizing, c->chunk, unsized);
  URB_HIP(hipMalloc(&c->work, sizing.off));
  c->work_bytes = sizing.off;
  Bump wb{static_cast<char*>(c->work)};
  carve_workspace(c, wb, c->chunk, c->ws);
  urb::launch_fill_i32(c->ws.status, 0, 4, nullptr);

  // ---- one validation pass over every payload
  int* flags = c->ws.status + 1;
  urb::launch_validate(URB_FMT_BF16, reinterpret_cast<const uint8_t*>(router), E * H * 2, nullptr,
                       0, flags, nullptr);
  const bool f16_check = d->composition == URB_COMPOSE_GLM && d->expert_format != URB_FMT_BF16;
  for (size_t e = 0; e < E; ++e)
    for (int m = 0; m < 3; ++m) {
      size_t sb, db = matrix_bytes(d->expert_format, dims[m][0], dims[m][1], &sb);
      urb::launch_validate(d->expert_format, table[e].data[m], db, table[e].scales[m], sb, flags,
                           nullptr, f16_check && m == 2);
    }
  if (has_shared)
    for (int m = 0; m < 3; ++m) {
      size_t sb, db = matrix_bytes(d->shared_format, sdims[m][0], sdims[m][1], &sb);
      urb::launch_validate(d->shared_format, shared.data[m], db, shared.scales[m], sb, flags,
                           nullptr);
    }
  if (c->bias) urb::launch_check_finite(c->bias, E, c->ws.status + 2, nullptr);
  if (qwen_gate)
    urb::launch_validate(URB_FMT_BF16, reinterpret_cast<const uint8_t*>(gate_rows), H * 2,
                         nullptr, 0, flags, nullptr);
  URB_HIP(hipGetLastError());
  int host_flags[4] = {0, 0, 0, 0};
  URB_HIP(hipDeviceSynchronize());
  URB_HIP(hipMemcpy(host_flags, c->ws.status, sizeof(host_flags), hipMemcpyDeviceToHost));
  // A non-finite bias: RuntimeMoeLayer::new's geometry error (glm/runtime/moe.rs:92-96), or
  // route_sqrt_softplus's NonFinite (deepseek_v4/math.rs:469-475).
  if (host_flags[2])
    return d->router == URB_ROUTER_SQRT_SOFTPLUS ? URB_ERR_NONFINITE : URB_ERR_INVALID_GEOMETRY;
  if (host_flags[1] & 1) return URB_ERR_NONFINITE;
  if (host_flags[1] & 2) return URB_ERR_INVALID_SCALE;
  c->down_f16 = f16_check && !(host_flags[1] & 4);
  urb::launch_fill_i32(c->ws.status, 0, 4, nullptr);

  // the BF16 shared down matrix as f16 (see urb_moe_ctx::shared16), own weights only
  if (!borrow && has_shared && d->composition == URB_COMPOSE_GLM &&
      d->shared_format == URB_FMT_BF16 && Is <= 16384) {
    const size_t n = H * Is;
    const uint16_t* down = reinterpret_cast<const uint16_t*>(shared.data[2]);
    const int shift = urb::bf16_f16_shift(down, n);
    if (shift != urb::kNoF16Shift) {
      URB_HIP(hipMalloc(&c->shared16, n * 2));
      urb::launch_bf16_to_f16(down, n, shift, c->shared16, nullptr);
      URB_HIP(hipGetLastError());
      c->shared_wshift = shift;
      c->weight_bytes += n * 2;
    }
  }

  if (qwen_gate) urb::launch_relayout_lane8(gate_rows, 1, (int)H, c->shared_gate8, nullptr);
  if (lane8)
    urb::launch_relayout_lane8(router, (int)E, (int)H, c->router_lane8, nullptr);
  else
    urb::launch_pack(URB_FMT_BF16, reinterpret_cast<const uint8_t*>(router), nullptr, (int)Ep,
                     (int)H, c->router_panel, nullptr, nullptr);
  URB_HIP(hipGetLastError());
  URB_HIP(hipDeviceSynchronize());

  URB_HIP(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking));
  URB_HIP(hipEventCreateWithFlags(&c->fork, hipEventDisableTiming));
  URB_HIP(hipEventCreateWithFlags(&c->join, hipEventDisableTiming));
  for (auto& pair : c->ev)
    for (hipEvent_t& e : pair) URB_HIP(hipEventCreate(&e));
  return URB_OK;
}

extern "C" {

urb_status urb_moe_create(const urb_moe_desc* desc, const urb_moe_weights* weights,
                          urb_weight_source source, urb_moe_ctx** out) {
  if (!desc || !weights || !out) return URB_ERR_ARGUMENT;
  *out = nullptr;
  urb_status st = check_desc(desc);
  if (st) return st;
  urb_moe_ctx* c = new urb_moe_ctx();
  st = create_impl(desc, weights, source, c);
  if (st) {
    (void)hipDeviceSynchronize();
    destroy_ctx(c);
    return st;
  }
  *out = c;
  return URB_OK;
}

void urb_moe_destroy(urb_moe_ctx* ctx) {
  if (!ctx) return;
  (void)hipDeviceSynchronize();
  destroy_ctx(ctx);
}

// Router logits for one chunk (the routing parameters returned carry the partial slices when
// the router writes them).  `xp` (one token): the router also writes the token's piece vector.
static urb::RouteParams launch_router_chunk(urb_moe_ctx* c, const float* x,
                                            const uint32_t* tokens, int n, float* logits,
                                            hipStream_t s, uint16_t* xp = nullptr,
                                            float* gate_logit = nullptr, int xq = 0) {
  const urb_moe_desc& d = c->desc;
  const bool qwen = d.composition == URB_COMPOSE_QWEN36;
  const int E = (int)d.n_experts, H = (int)d.hidden;
  urb::RouteParams rp{(int)d.router, qwen ? 1 : 0, (int)d.n_group, (int)d.topk_group,
                      d.normalize ? 1 : 0, d.routed_scaling_factor, c->bias, nullptr, 0,
                      c->hash, tokens, c->hash_vocab};
  Span span(c, URB_STAGE_ROUTER, s);
  if (c->router_lane8) {
    // gate_logit: the Qwen3.6 shared-expert gate row in the same launch
    urb::launch_router_lane8(c->router_lane8, E, H, x, n, logits, qwen ? 1 : 0, c->ws.status, s,
                             n == 1 ? xp : nullptr, gate_logit ? c->shared_gate8 : nullptr,
                             gate_logit, xq, c->ws.lo_word, c->lo_gen);
  } else if (n == 1) {
    // one token: a GEMV over the row-major router beats the 32-token MFMA tile
    rp.slices = urb::router_gemv_slices(E);
    rp.part = c->ws.router_part;
    urb::launch_router_gemv_f64(c->router, E, H, x, c->ws.router_part, rp.slices, c->ws.status,
                                s, xp, xq);
  } else {
    rp.slices = urb::router_slices(E, H, n);
    rp.part = c->ws.router_part;
    urb::launch_router_mfma(c->router_panel, E, H, x, n, c->ws.router_part, rp.slices,
                            c->ws.status, s, c->ws.lo_word, c->lo_gen, c->ws.xb);
  }
  return rp;
}

// Router and top-k for one chunk.  `xp` (one token): the router also writes the token's piece
// vector.
static urb_status route_chunk(urb_moe_ctx* c, const float* x, const uint32_t* tokens, int n,
                              float* logits, int32_t* ids, float* weights, hipStream_t s,
                              uint16_t* xp = nullptr, int xq = 0) {
  const urb_moe_desc& d = c->desc;
  const urb::RouteParams rp = launch_router_chunk(c, x, tokens, n, logits, s, xp, nullptr, xq);
  Span span(c, URB_STAGE_ROUTE, s);
  const bool ascending = d.composition != URB_COMPOSE_GLM;
  urb::launch_route(logits, n, (int)d.n_experts, (int)d.top_k, rp, ids, weights,
                    ascending ? c->ws.asc : nullptr, c->ws.status, s);
  return URB_OK;
}

// The stream the shared expert runs on: the side stream, concurrently with routing and the
// routed experts, except
//  * one-token calls, whose shared-expert kernels run in line on the caller's stream ahead of
//    the routing.  The fork and join cost the host ~23 us per call (two event records and two
//    stream waits, measured on MI355X), more than a one-token call's GPU work leaves to hide
//    it: with 4-6 kernel launches the call becomes host-bound.  Measured (one token, every
//    weight from HBM): c3_mxfp4_decode (88 MB BF16 shared expert) 75.5 -> 70-72 us in line,
//    the Qwen3.6 release layer (6 MB) 71-75 -> 51 us, DeepSeek-V4 Flash (13 MB) 71-72 -> 60 us;
//  * batches of 256+ tokens of the f32-activation compositions (mx == false), whose dense
//    shared GEMMs fill the GPU on their own: beside the MFMA router and the routed GEMMs they
//    only contend (c5_mxfp4_zipf_prefill, 1024 tokens: 2.53 -> 2.48 ms in line).  The
//    MX-activation compositions keep the overlap: their 8-lane FP32 router is LDS-bound and
//    hides under the shared GEMMs (1024 tokens in line: c5_mxfp4_dsv41 2.56 -> 2.67 ms,
//    dsv4_flash 1.09 -> 1.13 ms).
constexpr int kSharedInlineTokens = 256;
static hipStream_t shared_stream(const urb_moe_ctx* c, int n, hipStream_t s, bool mx) {
  if (n == 1) return s;
  return !mx && n >= kSharedInlineTokens ? s : c->side;
}

// One token, GLM and QWEN36 compositions: the projections run on the matrix cores from BF16
// piece vectors (urb_decode.hip).  The router writes the token's pieces; the shared expert runs
// in line after the routing, and its output and the k routed rows meet in the fused down
// projection + combine.
static urb_status forward_one(urb_moe_ctx* c, const float* xc, const uint32_t* tokens, float* yc,
                              int32_t* idc, float* wc, const float* resid, hipStream_t s) {
  const urb_moe_desc& d = c->desc;
  const bool qwen = d.composition == URB_COMPOSE_QWEN36;
  const bool has_shared = d.shared_intermediate != 0;
  const int E = (int)d.n_experts, H = (int)d.hidden, K = (int)d.top_k, I = (int)d.intermediate;
  const int Is = (int)d.shared_intermediate;
  Workspace& ws = c->ws;
  const urb::Epi epi{qwen ? urb::kEpiQwen : urb::kEpiGated, 0.0f};
  Perm perm{ws.meta, ws.active, ws.offsets, ws.counts, ws.perm_token, 0, ws.tiles, idc, K};
  if (has_shared) {
    // GLM: GatedMlp (src/models/glm/runtime/moe.rs:162).  QWEN36: a Qwen38Expert and its gate
    // logit linear(shared_expert_gate) (qwen3_6/runtime.rs:1417-1435).  In line on the caller's
    // stream (one token: see shared_stream), each shared projection in the launch of the
    // routed work beside it: the routing beside the shared gate+up, the routed gate+up beside
    // the shared down.
    // QWEN36 (an 8-lane router): the gate logit's row runs in the router's launch
    const urb::RouteParams rp = launch_router_chunk(c, xc, tokens, 1, ws.logits, s, ws.xp,
                                                    qwen ? ws.gate_logit : nullptr);
    {
      Span span(c, URB_STAGE_SHARED_GATE_UP, s);
      const urb::RouteJob job{ws.logits, K, rp, idc, wc, qwen ? ws.asc : nullptr};
      urb::launch_shared_gate_up_route(d.shared_format, c->shared_table, H, Is, ws.xp, nullptr,
                                       ws.shared_xp, epi, ws.status, s, E, job);
    }
    Span span(c, URB_STAGE_GATE_UP, s);
    urb::launch_gemv_mfma_gate_up_and_shared_down(d.expert_format, c->table, perm, std::min(E, K),
                                                  H, I, ws.xp, nullptr, ws.act_xp, epi,
                                                  d.shared_format, c->shared_table, Is,
                                                  ws.shared_xp, ws.shared_out, epi, ws.status, s);
  } else {
    // With f32 logits from the router (the 8-lane routers), the routing runs inside the routed
    // gate+up launch (every workgroup routes the token): one token through 128 BF16 experts of
    // 2048 x 768, 32.9 -> 31.9 us.  A sliced f64 router keeps its routing kernel: reading the
    // slices in every workgroup made one token's MXFP8 gate+up (160 experts, 6144 x 2048)
    // 36 -> 45 us.
    const urb::RouteParams rp = launch_router_chunk(c, xc, tokens, 1, ws.logits, s, ws.xp);
    const bool ascending = d.composition != URB_COMPOSE_GLM;
    const urb::RouteJob job{ws.logits, K, rp, idc, wc, ascending ? ws.asc : nullptr};
    bool fused = false;
    if (!rp.part) {
      Span span(c, URB_STAGE_GATE_UP, s);
      fused = urb::launch_routed_gate_up_route(d.expert_format, c->table, H, I, ws.xp,
                                               ws.act_xp, epi, ws.status, s, E, job);
    }
    if (!fused) {
      {
        Span span(c, URB_STAGE_ROUTE, s);
        urb::launch_route(ws.logits, 1, E, K, rp, idc, wc, job.asc, ws.status, s);
      }
      Span span(c, URB_STAGE_GATE_UP, s);
      urb::launch_gemv_mfma_gate_up(d.expert_format, c->table, perm, std::min(E, K), H, I,
                                    ws.xp, nullptr, ws.act_xp, epi, ws.status, s);
    }
  }
  if (urb::mfma_down_combine_fits(K, I)) {
    Span span(c, URB_STAGE_DOWN, s);
    urb::launch_gemv_mfma_down_combine(d.expert_format, c->table, idc, wc, ws.asc, K, H, I,
                                       ws.act_xp, has_shared ? ws.shared_out : nullptr,
                                       qwen ? 0 : 1, epi, yc, ws.status, s, resid,
                                       ws.gate_logit);
  } else {
    // k SwiGLU rows beyond the fused kernel's LDS: per-slot outputs, then the combine
    {
      Span span(c, URB_STAGE_DOWN, s);
      urb::launch_gemv_mfma_down(d.expert_format, c->table, perm, std::min(E, K), H, I,
                                 ws.act_xp, ws.y_perm, epi, ws.status, s);
    }
    Span span(c, URB_STAGE_COMBINE, s);
    if (qwen)
      urb::launch_combine_qwen(ws.y_perm, nullptr, wc, ws.asc, 1, K, H, yc, ws.status, s, resid,
                               has_shared ? ws.shared_out : nullptr, ws.gate_logit);
    else
      urb::launch_combine_glm(ws.y_perm, nullptr, wc, has_shared ? ws.shared_out : nullptr, 1, K,
                              H, yc, s);
  }
  if (c->profiling) return collect_spans(c);
  return URB_OK;
}

// One token, MX-activation compositions: the quantizer writes the token's pieces (exact in the
// first piece); the projections run on the matrix cores; between them the SwiGLU output is
// re-quantized into pieces.
static urb_status forward_mx_one(urb_moe_ctx* c, const float* xc, const uint32_t* tokens,
                                 float* yc, int32_t* idc, float* wc, hipStream_t s) {
  const urb_moe_desc& d = c->desc;
  const bool has_shared = d.shared_intermediate != 0;
  const int E = (int)d.n_experts, H = (int)d.hidden, K = (int)d.top_k, I = (int)d.intermediate;
  const int Is = (int)d.shared_intermediate;
  Workspace& ws = c->ws;
  const bool dsv = d.composition == URB_COMPOSE_DSV41 || d.composition == URB_COMPOSE_DSV4;
  const int block = d.composition == URB_COMPOSE_DSV4 ? 128 : 32;
  const urb::Epi routed{urb::kEpiHy4, d.swiglu_limit};
  const urb::Epi dense_mlp = dsv ? routed : urb::Epi{urb::kEpiHy4Shared, 0.0f};
  // The token's quantized pieces: a side job of the f64 GEMV router's launch (DeepSeek-V4 T=1
  // 41.7 -> 40.0 us, Hy4 with 160 MXFP8 experts 68.7 -> 67.7 us).  Beside the 8-lane router
  // (DeepSeek-V4.1) they keep a launch of their own: that router's 48 workgroups at E 384 took
  // 2.5 us longer with the 7168 values to quantize than the quantize launch costs.
  const int xq = c->router_lane8 ? 0 : block;
  uint16_t* rxp = xq ? ws.xp : nullptr;
  if (!xq)
    urb::launch_quantize(xc, 1, (size_t)H, nullptr, nullptr, nullptr, ws.status, s, 0, nullptr,
                         nullptr, block, ws.xp);
  Perm perm{ws.meta, ws.active, ws.offsets, ws.counts, ws.perm_token, 0, ws.tiles, idc, K};
  // Hy4 re-quantizes the SwiGLU output (expert.rs:677); DeepSeek first scales each row by its
  // route weight and rounds to BF16 (runtime.rs:2254-2258); one token: slot = row
  auto quantize_act = [&] {
    urb::launch_quantize(ws.act, (size_t)K, (size_t)I, nullptr, nullptr, nullptr, ws.status, s,
                         dsv ? 1 : 0, dsv ? wc : nullptr, nullptr, block, ws.act_xp);
  };
  if (has_shared) {
    // In line on the caller's stream (one token: see shared_stream), each shared projection in
    // the launch of the routed work beside it: the routing beside the shared gate+up, the
    // routed gate+up beside the shared down.
    const urb::RouteParams rp =
        launch_router_chunk(c, xc, tokens, 1, ws.logits, s, rxp, nullptr, xq);
    {
      Span span(c, URB_STAGE_SHARED_GATE_UP, s);
      const urb::RouteJob job{ws.logits, K, rp, idc, wc, ws.asc};
      urb::launch_shared_gate_up_route(d.shared_format, c->shared_table, H, Is, ws.xp,
                                       ws.shared_act, nullptr, dense_mlp, ws.status, s, E, job);
      urb::launch_quantize(ws.shared_act, 1, (size_t)Is, nullptr, nullptr, nullptr, ws.status,
                           s, dsv ? 1 : 0, nullptr, nullptr, block, ws.shared_xp);
    }
    Span span(c, URB_STAGE_GATE_UP, s);
    urb::launch_gemv_mfma_gate_up_and_shared_down(d.expert_format, c->table, perm, std::min(E, K),
                                                  H, I, ws.xp, ws.act, nullptr, routed,
                                                  d.shared_format, c->shared_table, Is,
                                                  ws.shared_xp, ws.shared_out, dense_mlp,
                                                  ws.status, s);
    quantize_act();
  } else {
    route_chunk(c, xc, tokens, 1, ws.logits, idc, wc, s, rxp, xq);
    Span span(c, URB_STAGE_GATE_UP, s);
    urb::launch_gemv_mfma_gate_up(d.expert_format, c->table, perm, std::min(E, K), H, I, ws.xp,
                                  ws.act, nullptr, routed, ws.status, s);
    quantize_act();
  }
  if (urb::mfma_down_combine_fits(K, I)) {
    Span span(c, URB_STAGE_DOWN, s);
    urb::launch_gemv_mfma_down_combine(d.expert_format, c->table, idc, wc, ws.asc, K, H, I,
                                       ws.act_xp, has_shared ? ws.shared_out : nullptr,
                                       dsv ? 3 : 2, routed, yc, ws.status, s);
  } else {
    {
      Span span(c, URB_STAGE_DOWN, s);
      urb::launch_gemv_mfma_down(d.expert_format, c->table, perm, std::min(E, K), H, I,
                                 ws.act_xp, ws.y_perm, routed, ws.status, s);
    }
    Span span(c, URB_STAGE_COMBINE, s);
    urb::launch_combine_hy4(ws.y_perm, nullptr, dsv ? nullptr : wc, ws.asc,
                            has_shared ? ws.shared_out : nullptr, 1, K, H, yc, ws.status, s);
  }
  if (c->profiling) return collect_spans(c);
  return URB_OK;
}

// The MX-activation compositions for one chunk of n tokens: Hy4 MoeWeights::forward
// (src/models/hy4/runtime.rs:1371-1447), DeepSeek-V4.1 MoeWeights::forward
// (src/models/deepseek_v41/runtime.rs:1963-2019) and DeepSeek-V4 MoeWeights::forward{,_batch}
// (src/models/deepseek_v4/runtime.rs:2484-2828: 128-value activation blocks).  Every MX
// projection reads simulated E4M3 activations (BF16-exact values); the BF16 MFMA / FMA kernels
// run them with the Hy4 epilogues.
static urb_status forward_mx(urb_moe_ctx* c, const float* xc, const uint32_t* tokens, int n,
                              float* yc, int32_t* idc, float* wc, hipStream_t s) {
  if (n == 1) return forward_mx_one(c, xc, tokens, yc, idc, wc, s);
  const urb_moe_desc& d = c->desc;
  const bool has_shared = d.shared_intermediate != 0;
  const int E = (int)d.n_experts, H = (int)d.hidden, K = (int)d.top_k, I = (int)d.intermediate;
  const int Is = (int)d.shared_intermediate;
  Workspace& ws = c->ws;
  const bool dsv = d.composition == URB_COMPOSE_DSV41 || d.composition == URB_COMPOSE_DSV4;
  hipStream_t ss = shared_stream(c, n, s, true);
  const int block = d.composition == URB_COMPOSE_DSV4 ? 128 : 32;  // activation block width
  // every projection's input is simulated E4M3 (4 significant bits, scales >= 2^-22): BF16-valued
  urb::Epi routed{urb::kEpiHy4, d.swiglu_limit};
  routed.no_lo = true;
  // Hy4's shared DenseMlp is a plain BF16 SwiGLU; DeepSeek's shared expert is a routed expert
  // without a weight
  urb::Epi dense_mlp = dsv ? routed : urb::Epi{urb::kEpiHy4Shared, 0.0f};
  dense_mlp.no_lo = true;
  // mx_activation(input) once per token (runtime.rs:1397); the shared expert quantizes the same
  // input the same way (runtime.rs:1312), so both read it.
  urb::launch_quantize(xc, (size_t)n, (size_t)H, ws.xq, nullptr, nullptr, ws.status, s, 0,
                       nullptr, nullptr, block);
  if (has_shared) {
    if (ss != s) {
      URB_HIP(hipEventRecord(c->fork, s));
      URB_HIP(hipStreamWaitEvent(ss, c->fork, 0));
    }
    Perm dense{nullptr, nullptr, nullptr, nullptr, nullptr, n, nullptr, nullptr, 0};
    const int dense_tiles = (n + urb::kGemmMTile - 1) / urb::kGemmMTile;
    {
      Span span(c, URB_STAGE_SHARED_GATE_UP, ss);
      urb::launch_gemm_gate_up(d.shared_format, c->shared_table, dense, dense_tiles, H, Is, ws.xq,
                               ws.shared_act, dense_mlp, ws.status, ss, ss != s);
      // the down projection re-quantizes its input (Hy4 mx_linear, runtime.rs:1321, 2425-2428;
      // DeepSeek `linear` after the BF16 step, deepseek_v41/runtime.rs:2258-2260)
      urb::launch_quantize(ws.shared_act, (size_t)n, (size_t)Is, ws.shared_act, nullptr, nullptr,
                           ws.status, ss, dsv ? 1 : 0, nullptr, nullptr, block);
    }
    {
      Span span(c, URB_STAGE_SHARED_DOWN, ss);
      urb::launch_gemm_down(d.shared_format, c->shared_table, dense, dense_tiles, H, Is,
                            ws.shared_act, ws.shared_out, dense_mlp, ws.status, ss, ss != s);
    }
    if (ss != s) URB_HIP(hipEventRecord(c->join, ss));
  }
  route_chunk(c, xc, tokens, n, ws.logits, idc, wc, s);
  Perm perm{ws.meta, ws.active, ws.offsets, ws.counts, ws.perm_token, 0, ws.tiles, nullptr, K};
  {
    Span span(c, URB_STAGE_PERMUTE, s);
    urb::launch_permute(idc, n, E, K, ws.meta, ws.active, ws.offsets, ws.counts, ws.perm_token,
                        ws.pos_of_slot, ws.tiles, ws.slot_of_pos, s);
  }
  const int max_tiles = urb::gemm_max_tiles(n, K, E);
  {
    Span span(c, URB_STAGE_GATE_UP, s);
    urb::launch_gemm_gate_up(d.expert_format, c->table, perm, max_tiles, H, I, ws.xq, ws.act,
                             routed, ws.status, s);
    // the SwiGLU output re-quantized for the down projection (Hy4 activate_gate_up,
    // expert.rs:677); DeepSeek first scales each row by its route weight and rounds to BF16
    // (runtime.rs:2254-2258)
    urb::launch_quantize(ws.act, (size_t)n * K, (size_t)I, ws.act, nullptr, nullptr, ws.status,
                         s, dsv ? 1 : 0, dsv ? wc : nullptr, dsv ? ws.slot_of_pos : nullptr,
                         block);
  }
  {
    Span span(c, URB_STAGE_DOWN, s);
    urb::launch_gemm_down(d.expert_format, c->table, perm, max_tiles, H, I, ws.act, ws.y_perm,
                          routed, ws.status, s);
  }
  if (has_shared && ss != s) URB_HIP(hipStreamWaitEvent(s, c->join, 0));
  {
    Span span(c, URB_STAGE_COMBINE, s);
    urb::launch_combine_hy4(ws.y_perm, ws.pos_of_slot, dsv ? nullptr : wc, ws.asc,
                            has_shared ? ws.shared_out : nullptr, n, K, H, yc, ws.status, s);
  }
  if (c->profiling) return collect_spans(c);
  return URB_OK;
}

// The decoder layer's steps either side of the MoE call (urb_moe_forward_block).
struct BlockArgs {
  const float* norm_weight;
  float eps;
};

static urb_status forward_impl(urb_moe_ctx* c, const float* x, const uint32_t* token_ids,
                               uint32_t tokens, float* y, int32_t* ids, float* weights,
                               void* stream, const BlockArgs* blk) {
  if (tokens == 0 || tokens > c->desc.max_tokens) return URB_ERR_SHAPE;
  if (c->hash && !token_ids) return URB_ERR_ARGUMENT;  // hash routing reads the token ids
  const urb_moe_desc& d = c->desc;
  const bool qwen = d.composition == URB_COMPOSE_QWEN36;
  const bool has_shared = d.shared_intermediate != 0;
  const int E = (int)d.n_experts, H = (int)d.hidden, K = (int)d.top_k, I = (int)d.intermediate;
  const int Is = (int)d.shared_intermediate;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace& ws = c->ws;
  const urb::Epi gated{urb::kEpiGated, 0.0f};
  const urb::Epi epi{qwen ? urb::kEpiQwen : urb::kEpiGated, 0.0f};
  for (uint32_t c0 = 0; c0 < tokens; c0 += c->chunk) {
    const int n = (int)std::min<uint32_t>(c->chunk, tokens - c0);
    const float* xc = x + (size_t)c0 * H;
    float* yc = y + (size_t)c0 * H;
    // block calls: x is the residual stream; the MoE reads its normalized BF16 form and the
    // combine adds the residual back
    const float* resid = nullptr;
    if (blk) {
      resid = xc;
      urb::launch_rms_norm(xc, blk->norm_weight, n, H, blk->eps, ws.xn, ws.status, s);
      xc = ws.xn;
    }
    int32_t* idc = ids ? ids + (size_t)c0 * K : ws.ids;
    float* wc = weights ? weights + (size_t)c0 * K : ws.weights;
    const uint32_t* tc = token_ids ? token_ids + c0 : nullptr;
    hipStream_t ss = shared_stream(c, n, s, mx_activation(d.composition));
    if (mx_activation(d.composition)) {
      urb_status st = forward_mx(c, xc, tc, n, yc, idc, wc, s);
      if (st) return st;
      continue;
    }
    if (n == 1) {
      urb_status st = forward_one(c, xc, tc, yc, idc, wc, resid, s);
      if (st) return st;
      continue;
    }
    // The routing and the permutation; with a shared expert in line (batches of 256+ tokens),
    // they run beside it on the side stream instead, and the routed GEMMs wait for both.
    const bool route_beside = has_shared && ss == s;
    // this chunk's generation of the batched router's lo-half word
    const unsigned lo_gen = ++c->lo_gen;
    Perm perm{ws.meta, ws.active, ws.offsets, ws.counts, ws.perm_token, 0, ws.tiles, nullptr, K};
    auto route_and_permute = [&](hipStream_t rs) {
      route_chunk(c, xc, tc, n, ws.logits, idc, wc, rs);
      Span span(c, URB_STAGE_PERMUTE, rs);
      urb::launch_permute(idc, n, E, K, ws.meta, ws.active, ws.offsets, ws.counts,
                          ws.perm_token, ws.pos_of_slot, ws.tiles, nullptr, rs);
    };
    if (route_beside) {
      URB_HIP(hipEventRecord(c->fork, s));
      URB_HIP(hipStreamWaitEvent(c->side, c->fork, 0));
      route_and_permute(c->side);
      URB_HIP(hipEventRecord(c->join, c->side));
    }
    if (has_shared) {
      // The shared expert does not depend on the routes: below 256 tokens it runs on the side
      // stream while the router, top-k and permutation run here (shared_stream).  GLM:
      // GatedMlp (src/models/glm/runtime/moe.rs:162).  QWEN36: a Qwen38Expert and its gate
      // logit linear(shared_expert_gate) -- the router's 8-lane FP32 tree with BF16 output, one
      // row (qwen3_6/runtime.rs:1417-1435).
      if (ss != s) {
        URB_HIP(hipEventRecord(c->fork, s));
        URB_HIP(hipStreamWaitEvent(ss, c->fork, 0));
      }
      // the shared gate/up reads the (normalized BF16) block input; a Qwen38Expert's down
      // reads its BF16 SwiGLU rows
      urb::Epi sepi = qwen ? epi : gated;
      urb::Epi sdepi = sepi;
      sepi.no_lo = blk != nullptr;
      sdepi.no_lo = qwen;
      sdepi.stream_out = true;  // read only by the combine, after the routed GEMMs
      Perm dense{nullptr, nullptr, nullptr, nullptr, nullptr, n, nullptr, nullptr, 0};
      const int dense_tiles = (n + urb::kGemmMTile - 1) / urb::kGemmMTile;
      bool dense_gu = false, f16_down = false;
      {
        Span span(c, URB_STAGE_SHARED_GATE_UP, ss);
        if (qwen)
          urb::launch_router_lane8(c->shared_gate8, 1, H, xc, n, ws.gate_logit, 1, ws.status,
                                   ss);
        // in line (256+ tokens): the dense split-K kernel (urb_dense.hip), its partial sums in
        // the routed outputs' buffer, which nothing reads until the routed down projection
        const size_t part_floats = (size_t)c->chunk * K * H;
        dense_gu = ss == s && d.shared_format == URB_FMT_BF16 &&
                   urb::dense_fits(n, Is, H, part_floats);
        // with the f16 shared down matrix: the SwiGLU rows as f16 for the f16 down projection
        f16_down = dense_gu && c->shared16 != nullptr;
        if (f16_down)
          urb::launch_dense_gate_up_f16(c->shared_host, n, H, Is, xc,
                                        reinterpret_cast<uint16_t*>(ws.shared_act),
                                        ws.shared_rowexp, sepi, ws.status, ws.y_perm,
                                        part_floats, s);
        else if (dense_gu)
          urb::launch_dense_gate_up(c->shared_host, n, H, Is, xc, ws.shared_act, sepi, ws.status,
                                    ws.y_perm, part_floats, s);
        else
          urb::launch_gemm_gate_up(d.shared_format, c->shared_table, dense, dense_tiles, H, Is,
                                   xc, ws.shared_act, sepi, ws.status, ss, ss != s);
      }
      {
        Span span(c, URB_STAGE_SHARED_DOWN, ss);
        if (f16_down) {
          urb::Epi e16 = sdepi;
          e16.wshift = c->shared_wshift;
          urb::launch_dense_down_f16(c->shared16, n, H, Is,
                                     reinterpret_cast<const uint16_t*>(ws.shared_act),
                                     ws.shared_rowexp, e16, ws.shared_out, ws.status, s);
        } else {
          urb::launch_gemm_down(d.shared_format, c->shared_table, dense, dense_tiles, H, Is,
                                ws.shared_act, ws.shared_out, sdepi, ws.status, ss, ss != s);
        }
      }
      if (ss != s) URB_HIP(hipEventRecord(c->join, ss));
    }
    if (route_beside)
      URB_HIP(hipStreamWaitEvent(s, c->join, 0));
    else
      route_and_permute(s);
    const int max_tiles = urb::gemm_max_tiles(n, K, E);
    urb::Epi repi = epi;
    if (c->down_f16) {
      repi.rowexp = ws.rowexp;
      repi.groups = (int)rowexp_groups(d);
    }
    // Which activation rows are BF16-valued: a block call's normalized input, a Qwen38Expert's
    // SwiGLU rows; otherwise the token input when the router saw no value off the BF16 grid.
    urb::Epi gepi = repi, depi = repi;
    if (blk) {
      gepi.no_lo = true;
    } else {
      gepi.lo_word = ws.lo_word;
      gepi.lo_gen = lo_gen;
    }
    // the router's BF16 copy of the same rows (batched MFMA router; null otherwise)
    gepi.xb = ws.xb;
    depi.no_lo = qwen;
    // grouped MFMA GEMMs over the row tiles
    {
      Span span(c, URB_STAGE_GATE_UP, s);
      urb::launch_gemm_gate_up(d.expert_format, c->table, perm, max_tiles, H, I, xc, ws.act,
                               gepi, ws.status, s);
    }
    {
      Span span(c, URB_STAGE_DOWN, s);
      urb::launch_gemm_down(d.expert_format, c->table, perm, max_tiles, H, I, ws.act, ws.y_perm,
                            depi, ws.status, s);
    }
    if (has_shared && ss != s) URB_HIP(hipStreamWaitEvent(s, c->join, 0));
    {
      Span span(c, URB_STAGE_COMBINE, s);
      if (qwen)
        urb::launch_combine_qwen(ws.y_perm, ws.pos_of_slot, wc, ws.asc, n, K, H, yc, ws.status, s,
                                 resid, has_shared ? ws.shared_out : nullptr, ws.gate_logit);
      else
        urb::launch_combine_glm(ws.y_perm, ws.pos_of_slot, wc, has_shared ? ws.shared_out : nullptr,
                                n, K, H, yc, s);
    }
    if (c->profiling) {
      urb_status st = collect_spans(c);
      if (st) return st;
    }
  }
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_moe_forward(urb_moe_ctx* c, const float* x, uint32_t tokens, float* y,
                           int32_t* ids, float* weights, void* stream) {
  if (!c || !x || !y) return URB_ERR_ARGUMENT;
  return forward_impl(c, x, nullptr, tokens, y, ids, weights, stream, nullptr);
}

urb_status urb_moe_forward_noalloc(urb_moe_ctx* c, const float* x, uint32_t tokens, float* y,
                                   int32_t* ids, float* weights, void* stream) {
  if (!c || !x || !y) return URB_ERR_ARGUMENT;
  if (c->hash) return URB_ERR_ARGUMENT;  // hash routing reads token ids
  if (tokens == 0 || tokens > c->chunk) return URB_ERR_SHAPE;
  // this call's buffers, carved from the GPU's static scratch instead of the context workspace
  Workspace ws;
  Bump sizing{nullptr};
  carve_workspace(c, sizing, tokens, ws, false);
  if (sizing.off > urb::kScratchBytes) return URB_ERR_SHAPE;
  void* region = nullptr;
  URB_HIP(urb::scratch_region(&region));
  Bump b{static_cast<char*>(region)};
  carve_workspace(c, b, tokens, ws, false);
  ws.status = c->ws.status;  // failures still latch in the context's status word
  ws.lo_word = c->ws.lo_word;
  const Workspace own = c->ws;
  const uint32_t chunk = c->chunk;
  c->ws = ws;
  c->chunk = tokens;  // one chunk: the scratch buffers are sized for `tokens`
  const urb_status st = forward_impl(c, x, nullptr, tokens, y, ids, weights, stream, nullptr);
  c->chunk = chunk;
  c->ws = own;
  return st;
}

urb_status urb_moe_forward_tokens(urb_moe_ctx* c, const float* x, const uint32_t* token_ids,
                                  uint32_t tokens, float* y, int32_t* ids, float* weights,
                                  void* stream) {
  if (!c || !x || !y || !token_ids) return URB_ERR_ARGUMENT;
  return forward_impl(c, x, token_ids, tokens, y, ids, weights, stream, nullptr);
}

urb_status urb_moe_forward_block(urb_moe_ctx* c, const float* h, const float* norm_weight,
                                 float eps, uint32_t tokens, float* out, int32_t* ids,
                                 float* weights, void* stream) {
  if (!c || !h || !norm_weight || !out) return URB_ERR_ARGUMENT;
  if (c->desc.composition != URB_COMPOSE_QWEN36) return URB_ERR_ARGUMENT;
  if (!finite_host(eps) || !(eps > 0.0f)) return URB_ERR_INVALID_GEOMETRY;
  const BlockArgs blk{norm_weight, eps};
  return forward_impl(c, h, nullptr, tokens, out, ids, weights, stream, &blk);
}

urb_status urb_zc_rms_norm_bf16(const float* x, const float* weight, uint32_t rows,
                                uint32_t hidden, float eps, float* out, void* stream) {
  if (!x || !weight || !out) return URB_ERR_ARGUMENT;
  if (rows == 0 || hidden == 0 || hidden % 4 || hidden > 16384) return URB_ERR_SHAPE;
  if (!finite_host(eps) || !(eps > 0.0f)) return URB_ERR_INVALID_GEOMETRY;
  urb::launch_rms_norm(x, weight, (int)rows, (int)hidden, eps, out, nullptr,
                       static_cast<hipStream_t>(stream));
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_moe_profile(urb_moe_ctx* c, int enable) {
  if (!c) return URB_ERR_ARGUMENT;
  URB_HIP(hipDeviceSynchronize());
  if (enable) {
    for (int st = 0; st < URB_STAGE_COUNT; ++st) {
      c->stage_ms[st] = 0.0;
      c->stage_calls[st] = 0;
      c->pending[st] = false;
    }
  }
  c->profiling = enable != 0;
  return URB_OK;
}

urb_status urb_moe_profile_read(const urb_moe_ctx* c, double* ms, uint64_t* launches) {
  if (!c) return URB_ERR_ARGUMENT;
  for (int st = 0; st < URB_STAGE_COUNT; ++st) {
    if (ms) ms[st] = c->stage_ms[st];
    if (launches) launches[st] = c->stage_calls[st];
  }
  return URB_OK;
}

static urb_status route_impl(urb_moe_ctx* c, const float* x, const uint32_t* token_ids,
                             uint32_t tokens, float* logits, int32_t* ids, float* weights,
                             void* stream) {
  if (tokens == 0 || tokens > c->desc.max_tokens) return URB_ERR_SHAPE;
  if (c->hash && !token_ids) return URB_ERR_ARGUMENT;  // hash routing reads the token ids
  const urb_moe_desc& d = c->desc;
  const int E = (int)d.n_experts, H = (int)d.hidden, K = (int)d.top_k;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (uint32_t c0 = 0; c0 < tokens; c0 += c->chunk) {
    const int n = (int)std::min<uint32_t>(c->chunk, tokens - c0);
    float* lc = logits ? logits + (size_t)c0 * E : c->ws.logits;
    int32_t* idc = ids ? ids + (size_t)c0 * K : c->ws.ids;
    float* wc = weights ? weights + (size_t)c0 * K : c->ws.weights;
    route_chunk(c, x + (size_t)c0 * H, token_ids ? token_ids + c0 : nullptr, n, lc, idc, wc, s);
  }
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_moe_route(urb_moe_ctx* c, const float* x, uint32_t tokens, float* logits,
                         int32_t* ids, float* weights, void* stream) {
  if (!c || !x) return URB_ERR_ARGUMENT;
  return route_impl(c, x, nullptr, tokens, logits, ids, weights, stream);
}

urb_status urb_moe_route_tokens(urb_moe_ctx* c, const float* x, const uint32_t* token_ids,
                                uint32_t tokens, float* logits, int32_t* ids, float* weights,
                                void* stream) {
  if (!c || !x || !token_ids) return URB_ERR_ARGUMENT;
  return route_impl(c, x, token_ids, tokens, logits, ids, weights, stream);
}

urb_status urb_moe_sync(urb_moe_ctx* c, void* stream) {
  if (!c) return URB_ERR_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int st = 0;
  URB_HIP(hipStreamSynchronize(s));
  URB_HIP(hipStreamSynchronize(c->side));
  URB_HIP(hipMemcpy(&st, c->ws.status, sizeof(int), hipMemcpyDeviceToHost));
  urb::launch_fill_i32(c->ws.status, 0, 1, s);
  URB_HIP(hipGetLastError());
  URB_HIP(hipStreamSynchronize(s));
  if (st & urb::kStatusNonFinite) return URB_ERR_NONFINITE;
  if (st & urb::kStatusBadToken) return URB_ERR_SHAPE;  // load_i64_matrix_row's bounds check
  return URB_OK;
}

urb_status urb_dequant_rows(urb_format format, const void* data, const uint8_t* scales,
                            uint32_t rows, uint32_t cols, uint32_t row0, uint32_t count,
                            float* out, void* stream) {
  if (!data || !out || (format != URB_FMT_BF16 && !scales)) return URB_ERR_ARGUMENT;
  if (format != URB_FMT_BF16 && format != URB_FMT_MXFP4 && format != URB_FMT_MXFP8)
    return URB_ERR_ARGUMENT;
  if (rows == 0 || cols == 0 || (format != URB_FMT_BF16 && cols % 32)) return URB_ERR_SHAPE;
  if ((uint64_t)row0 + count > rows) return URB_ERR_SHAPE;
  if (count == 0) return URB_OK;
  urb::launch_dequant(format, static_cast<const uint8_t*>(data), scales, (int)rows, (int)cols,
                      (int)row0, (int)count, out, static_cast<hipStream_t>(stream));
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_quantize_e4m3_blocks(const float* x, uint32_t rows, uint32_t cols,
                                    uint32_t block, uint8_t* codes, uint8_t* scales,
                                    void* stream) {
  if (!x || !codes || !scales) return URB_ERR_ARGUMENT;
  if (block != 32 && block != 128) return URB_ERR_ARGUMENT;
  if (rows == 0 || cols == 0 || cols % block) return URB_ERR_SHAPE;
  urb::launch_quantize(x, rows, cols, nullptr, codes, scales, nullptr,
                       static_cast<hipStream_t>(stream), 0, nullptr, nullptr, (int)block);
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_quantize_e4m3(const float* x, uint32_t rows, uint32_t cols, uint8_t* codes,
                             uint8_t* scales, void* stream) {
  return urb_quantize_e4m3_blocks(x, rows, cols, 32, codes, scales, stream);
}

urb_status urb_pack_matrix(urb_format format, const void* data, const uint8_t* scales,
                           uint32_t rows, uint32_t cols, void* packed_data,
                           uint8_t* packed_scales, void* stream) {
  if (format != URB_FMT_BF16 && format != URB_FMT_MXFP4 && format != URB_FMT_MXFP8)
    return URB_ERR_ARGUMENT;
  const bool mx = format != URB_FMT_BF16;
  if (!data || !packed_data || (mx && (!scales || !packed_scales))) return URB_ERR_ARGUMENT;
  if (!urb::panel_shape_ok(rows, cols)) return URB_ERR_SHAPE;
  urb::launch_pack(format, static_cast<const uint8_t*>(data), scales, (int)rows, (int)cols,
                   static_cast<uint8_t*>(packed_data), packed_scales,
                   static_cast<hipStream_t>(stream));
  URB_HIP(hipGetLastError());
  return URB_OK;
}

urb_status urb_expert_views(urb_format format, uint32_t n_experts, uint32_t hidden,
                            uint32_t intermediate, const void* gate_up,
                            const uint8_t* gate_up_scales, const void* down,
                            const uint8_t* down_scales, urb_matrix* out) {
  if (format != URB_FMT_BF16 && format != URB_FMT_MXFP4 && format != URB_FMT_MXFP8)
    return URB_ERR_ARGUMENT;
  const bool mx = format != URB_FMT_BF16;
  if (!gate_up || !down || !out || n_experts == 0) return URB_ERR_ARGUMENT;
  if (mx != (gate_up_scales != nullptr) || mx != (down_scales != nullptr)) return URB_ERR_ARGUMENT;
  if (hidden == 0 || intermediate == 0 || hidden % 32 || intermediate % 32) return URB_ERR_SHAPE;
  const size_t H = hidden, I = intermediate;
  size_t gs, gd = matrix_bytes(format, I, H, &gs);  // one [I, H] half of an expert's [2I, H]
  size_t ds, dd = matrix_bytes(format, H, I, &ds);
  const uint8_t* gu = static_cast<const uint8_t*>(gate_up);
  const uint8_t* dn = static_cast<const uint8_t*>(down);
  for (size_t e = 0; e < n_experts; ++e) {
    out[3 * e + 0] = urb_matrix{gu + e * 2 * gd, mx ? gate_up_scales + e * 2 * gs : nullptr};
    out[3 * e + 1] = urb_matrix{gu + e * 2 * gd + gd, mx ? gate_up_scales + e * 2 * gs + gs : nullptr};
    out[3 * e + 2] = urb_matrix{dn + e * dd, mx ? down_scales + e * ds : nullptr};
  }
  return URB_OK;
}

urb_status urb_moe_set_expert(urb_moe_ctx* c, uint32_t expert, const urb_matrix* mats,
                              void* stream) {
  if (!c || !mats || !c->borrowed) return URB_ERR_ARGUMENT;
  const urb_moe_desc& d = c->desc;
  if (expert >= d.n_experts) return URB_ERR_ARGUMENT;
  const bool mx = d.expert_format != URB_FMT_BF16;
  for (int m = 0; m < 3; ++m)
    if (!mats[m].data || (mx && !mats[m].scales)) return URB_ERR_ARGUMENT;
  const size_t H = d.hidden, I = d.intermediate;
  const size_t dims[3][2] = {{I, H}, {I, H}, {H, I}};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // validate the payload as urb_moe_create does (codes and scales are layout-independent), on
  // the caller's stream, after anything already queued there
  int* flags = c->ws.status + 3;
  urb::launch_fill_i32(flags, 0, 1, s);
  ExpertMats e{};
  for (int m = 0; m < 3; ++m) {
    size_t sb, db = matrix_bytes(d.expert_format, dims[m][0], dims[m][1], &sb);
    e.data[m] = static_cast<const uint8_t*>(mats[m].data);
    e.scales[m] = sb ? mats[m].scales : nullptr;
    urb::launch_validate(d.expert_format, e.data[m], db, e.scales[m], sb, flags, s,
                         c->down_f16 && m == 2);
  }
  URB_HIP(hipGetLastError());
  int host_flags = 0;
  URB_HIP(hipMemcpyAsync(&host_flags, flags, sizeof(int), hipMemcpyDeviceToHost, s));
  URB_HIP(hipStreamSynchronize(s));
  if (host_flags & 1) return URB_ERR_NONFINITE;
  if (host_flags & 2) return URB_ERR_INVALID_SCALE;
  if (host_flags & 4) c->down_f16 = false;  // this expert's down scales leave the f16 range
  // the table entry changes in stream order: calls queued before keep the previous matrices
  URB_HIP(hipMemcpyAsync(c->table + expert, &e, sizeof(ExpertMats), hipMemcpyHostToDevice, s));
  URB_HIP(hipStreamSynchronize(s));
  return URB_OK;
}

urb_status urb_inspect_matrix(const urb_tensor_meta* weight, const urb_tensor_meta* scale,
                              int packed_name, uint32_t rows, uint32_t cols, urb_format* format,
                              uint64_t* resident_bytes) {
  if (!weight || !format || !resident_bytes) return URB_ERR_ARGUMENT;
  if (rows == 0 || cols == 0) return URB_ERR_SHAPE;
  const uint64_t R = rows, Cc = cols, blocks = (Cc + 31) / 32;
  auto is2d = [](const urb_tensor_meta* t, uint64_t a, uint64_t b) {
    return t->ndim == 2 && t->shape[0] == a && t->shape[1] == b;
  };
  const urb_dtype wt = weight->dtype;
  if ((wt == URB_DTYPE_BF16 || wt == URB_DTYPE_F16 || wt == URB_DTYPE_F32) && !scale) {
    // a plain matrix (weight.rs:157-170)
    const uint64_t esize = wt == URB_DTYPE_F32 ? 4 : 2;
    if (!is2d(weight, R, Cc) || weight->data_len != R * Cc * esize) return URB_ERR_SHAPE;
    if (wt != URB_DTYPE_BF16) return URB_ERR_ARGUMENT;
    *format = URB_FMT_BF16;
    *resident_bytes = weight->data_len;
    return URB_OK;
  }
  if (wt == URB_DTYPE_F8_E4M3) {
    // MXFP8 (weight.rs:171-254): the sidecar's dtype and shape select the block geometry
    if (!scale) return URB_ERR_ARGUMENT;  // require_mx_scale: Unsupported
    const bool modelopt = scale->dtype == URB_DTYPE_U8 && is2d(scale, R, blocks);
    const bool block32 = scale->dtype == URB_DTYPE_F8_E8M0 && is2d(scale, (R + 31) / 32, blocks);
    const bool block128 = scale->dtype == URB_DTYPE_F8_E8M0 &&
                          is2d(scale, (R + 127) / 128, (Cc + 127) / 128);
    if (!modelopt && !block32 && !block128) return URB_ERR_SHAPE;
    if (!is2d(weight, R, Cc) || weight->data_len != R * Cc) return URB_ERR_SHAPE;
    if (!modelopt) return URB_ERR_ARGUMENT;  // 32x32 / 128x128 blocks: not taken here
    *format = URB_FMT_MXFP8;
    *resident_bytes = weight->data_len + scale->data_len;
    return URB_OK;
  }
  const bool native_mxfp4 = wt == URB_DTYPE_I8 || (wt == URB_DTYPE_U8 && packed_name);
  if (native_mxfp4 && scale) {
    // MXFP4 (weight.rs:261-286): packed nibbles, E8M0 per 32 (U8-typed for U8 weights)
    const urb_dtype sdt = wt == URB_DTYPE_U8 ? URB_DTYPE_U8 : URB_DTYPE_F8_E8M0;
    const uint64_t pc = (Cc + 1) / 2;
    if (!is2d(weight, R, pc) || weight->data_len != R * pc || scale->dtype != sdt ||
        !is2d(scale, R, blocks))
      return URB_ERR_SHAPE;
    *format = URB_FMT_MXFP4;
    *resident_bytes = weight->data_len + scale->data_len;
    return URB_OK;
  }
  return URB_ERR_ARGUMENT;  // Colibri INT4/INT8, block-FP8 and other dtypes
}

uint32_t urb_gemm_placement(urb_format format, int pair, uint32_t dense_tokens, uint32_t tiles,
                            uint32_t rows, uint32_t cols, int32_t* tile_of_block,
                            int32_t* group_of_block, uint32_t capacity) {
  if (format != URB_FMT_BF16 && format != URB_FMT_MXFP4 && format != URB_FMT_MXFP8) return 0;
  if (!urb::panel_shape_ok(rows, cols) || rows % urb::kGemmNTile || tiles == 0) return 0;
  if (capacity && (!tile_of_block || !group_of_block)) return 0;
  return (uint32_t)urb::gemm_placement((int)format, pair != 0, (int)dense_tokens, (int)tiles,
                                       (int)rows, (int)cols, tile_of_block, group_of_block,
                                       (int)capacity);
}

urb_status urb_moe_memory(const urb_moe_ctx* c, size_t* weight_bytes, size_t* workspace_bytes) {
  if (!c) return URB_ERR_ARGUMENT;
  if (weight_bytes) *weight_bytes = c->weight_bytes;
  if (workspace_bytes) *workspace_bytes = c->work_bytes;
  return URB_OK;
}

}  // extern "C"
