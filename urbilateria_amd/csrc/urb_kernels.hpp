// urb_kernels.hpp -- host-side launch interface of the MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace urb {

// Error bits written to the per-context status word (the host maps them to urb_status).
constexpr int kStatusNonFinite = 1;
constexpr int kStatusBadToken = 2;  // a token id outside the hash table

// Panel layout of a [rows, cols] weight matrix in HBM (rows % 16 == 0, cols % 128 == 0).
// The matrix is a sequence of 16-row panels, each holding exactly the bytes of its 16 rows.
// A panel is a run of 1 KiB slabs; 16-byte unit l = ln + 16 lq of slab t belongs to panel row
// ln and holds
//   BF16:  columns 32 t + 8 lq + [0, 8)                        (cols / 32 slabs)
//   MXFP4: MX block 4 t + lq, i.e. columns 128 t + 32 lq + [0, 32)  (cols / 128 slabs)
//   MXFP8: half t % 2 of MX block 4 (t / 2) + lq                (cols / 64 slabs)
// so one wavefront load instruction (64 lanes x 16 B) reads one slab, and a wavefront that
// sweeps a panel reads it front to back.  E8M0 scales: per panel, cols / 128 slabs of 64 B;
// byte l of scale slab s is the scale of row ln, block 4 s + lq.
constexpr int kPanelRows = 16;
constexpr int kPanelCols = 128;
inline bool panel_shape_ok(size_t rows, size_t cols) {
  return rows % kPanelRows == 0 && cols % kPanelCols == 0 && rows > 0 && cols > 0;
}
void launch_pack(int fmt, const uint8_t* data, const uint8_t* scales, int rows, int cols,
                 uint8_t* packed, uint8_t* packed_scales, hipStream_t s);

// One expert's three projections in HBM (gate [I,H], up [I,H], down [H,I]), panel layout.
struct ExpertMats {
  const uint8_t* data[3];
  const uint8_t* scales[3];
};

// Token -> expert permutation for one forward chunk.  Stable (expert, token) order, the
// execute_batched_moe grouping (src/models/qwen3_6/runtime.rs:1123-1132).
struct Perm {
  const int32_t* meta;        // meta[0] = active experts, meta[1] = GEMM row tiles
  const int32_t* active;      // active expert ids, ascending
  const int32_t* offsets;     // [E + 1] first permuted position of each expert
  const int32_t* counts;      // [E] tokens routed to each expert
  const int32_t* perm_token;  // [T * k] token of each permuted position
  int dense_tokens;           // > 0: one dense expert (table entry 0) over tokens 0..n-1
  const int32_t* tiles;       // [2 * tiles] (expert, first row) of each kGemmMTile-row tile
  // One token (decode): the token's ranked expert ids; slot a is expert direct[a] at permuted
  // position a.  No permutation kernel runs; the fields above are unused.
  const int32_t* direct;
  int direct_k;
};

// Epilogue of the expert projections (gate/up pair -> activation; down -> output):
//   kEpiGated     GatedMlp (src/model/mlp.rs:90-99): silu(g) * u in f32; f32 outputs.
//   kEpiQwen      Qwen38Expert (src/models/qwen3_8/expert.rs:137-207): g, u, silu(g), the
//                 product and the outputs rounded to BF16.
//   kEpiHy4       Hy4 routed expert (src/models/hy4/expert.rs:664-680): g, u rounded to BF16,
//                 bounded_swiglu with `limit` (src/models/deepseek_v4/math.rs:526-548); BF16
//                 outputs.
//   kEpiHy4Shared Hy4 shared DenseMlp (src/models/hy4/runtime.rs:1311-1321):
//                 bf16(silu(bf16(g)) * bf16(u)); BF16 outputs.
enum { kEpiGated = 0, kEpiQwen = 1, kEpiHy4 = 2, kEpiHy4Shared = 3 };
// rowexp (GatedMlp batches, MX weights): the gate/up projection also writes, per permuted row and
// panel group, the largest f32 exponent field of the row's activations (rowexp[row * groups +
// group]); the down projection then stages each row in f16 scaled by a power of two so that
// its largest value falls in [2^14, 2^15), runs one f16 MFMA per product and rescales the sums
// exactly (11 significant bits of each activation instead of the 16 of the BF16 hi + lo pair).
// no_lo: the projection's input rows are BF16-valued by construction (a Qwen38Expert's BF16
// SwiGLU output, a simulated E4M3 activation, the normalized input of a block call), so the
// grouped GEMM stages and multiplies their hi halves only.  lo_word / lo_gen: the same when the
// batched router found every lo half of this call's input zero -- it stores lo_gen into
// *lo_word when it sees a non-zero one (urb_route.hip, router_mfma_kernel).
// stream_out (down projections): the outputs are read once, by the combine at the end of the
// call, so they are stored non-temporally and do not hold L2 lines during the GEMMs between
// (the shared expert's down rows of a batch).
// wshift (the dense f16 down projection over a BF16 matrix converted to f16 times 2^wshift,
// launch_bf16_to_f16): the sums are scaled back by 2^-wshift as well.
struct Epi {
  int kind;
  float limit;
  int* rowexp = nullptr;
  int groups = 0;
  bool no_lo = false;
  const unsigned* lo_word = nullptr;
  unsigned lo_gen = 0;
  bool stream_out = false;
  int wshift = 0;
  // gate/up: the token rows as BF16 [T, K] (written by the batched MFMA router beside its own
  // staging), staged in place of the f32 rows when they are BF16-valued (no lo half: no_lo or
  // lo_word): half the activation bytes and no conversion per K step
  const uint16_t* xb = nullptr;
};
// E8M0 codes whose scale keeps every element of an MX matrix exact in f16 (MXFP4: 6 2^13 is
// the largest value and 0.5 2^-23 = 2^-24 the f16 grid; MXFP8: 448 2^7, 2^-9 2^-15).
constexpr int kF16ScaleLo[3] = {0, 104, 112};
constexpr int kF16ScaleHi[3] = {-1, 140, 134};

// Grouped GEMM (MFMA) tiling: tokens per tile, weight rows per workgroup (four panels), K per
// step.
constexpr int kGemmMTile = 32;
constexpr int kGemmNTile = 64;
constexpr int kGemmKStep = 128;
// Upper bound of row tiles for n tokens routed k ways over E experts.
inline int gemm_max_tiles(int n, int k, int E) {
  int a = n * k < E ? n * k : E;
  return a + (n * k + kGemmMTile - 1) / kGemmMTile;
}

// Workgroup placement of the grouped GEMM.  Workgroups go to the eight XCDs round robin
// (block % 8) and each XCD has its own L2.  XCD c = cx + xsplit cy takes the contiguous run cy
// (of 8 / xsplit) of the tile list and the run cx (of xsplit) of the panel groups, tile by tile:
// an expert's tiles (tiles are in expert order), which read the same weight panels, share one
// L2, and so do a tile's workgroups, which read the same activation rows.  Returns false for a
// workgroup with nothing to do.  The grid has 8 * gemm_blocks_per_xcd(...) workgroups.
__host__ __device__ inline bool gemm_place(int block, int ntiles, int groups, int xsplit,
                                           int* tile, int* group) {
  const int xcd = block & 7, local = block >> 3;
  const int cx = xcd % xsplit, cy = xcd / xsplit, ysplit = 8 / xsplit;
  const int g0 = cx * groups / xsplit, width = (cx + 1) * groups / xsplit - g0;
  if (width <= 0) return false;
  const int t1 = (cy + 1) * ntiles / ysplit;
  const int w = cy * ntiles / ysplit + local / width;
  if (w >= t1) return false;
  *tile = w;
  *group = g0 + local % width;
  return true;
}
__host__ __device__ inline int gemm_blocks_per_xcd(int max_tiles, int groups, int xsplit) {
  const int ysplit = 8 / xsplit;
  return (max_tiles + ysplit - 1) / ysplit * ((groups + xsplit - 1) / xsplit);
}
// The panel-group split across XCDs.  Routed tiles (dense_tokens == 0): 1, so each expert's
// weights come from the one XCD holding its tiles.  One dense expert over `ntiles` tiles: the
// split with the least estimated time, taking time as the HBM bytes the launch moves (weights
// once per non-empty tile run, `wbytes` each; the activations once per split, `abytes` each)
// spread over the XCDs that have work -- so a batch of one or two tiles spreads its panel
// groups over all eight XCDs instead of leaving most of them idle.
int gemm_xsplit(int dense_tokens, int ntiles, int groups, double wbytes, double abytes);
// Weight panels per wave of the grouped GEMM for a format, row count, projection (pair: gate+up)
// and dense batch size (0: routed tiles).
int gemm_panels_per_wave(int fmt, int rows, bool pair, int dense_tokens);
// Host-side replay of a launch's placement (urb_gemm_placement): the grid size, and the tile and
// panel group of each of the first `capacity` workgroups (-1 when idle).
int gemm_placement(int fmt, bool pair, int dense_tokens, int max_tiles, int rows, int K,
                   int32_t* tile_of_block, int32_t* group_of_block, int capacity);
// beside: a dense batch running on a side stream next to other work (launched at most one
// workgroup per CU at a time, so that work keeps the other slots).
void launch_gemm_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                         int I, const float* x, float* act, Epi epi, int* status,
                         hipStream_t s, bool beside = false);
void launch_gemm_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_tiles, int H,
                      int I, const float* act, float* y, Epi epi, int* status, hipStream_t s,
                      bool beside = false);

struct RouteParams {
  int router;        // 0 softmax top-k, 1 sigmoid noaux_tc, 2 sqrt-softplus
  int qwen;          // round route weights to BF16
  int n_group, topk_group, normalize;
  float scale;
  const float* bias; // [E] or nullptr
  // When set, the logits are the in-order sums of `slices` f64 partial slices
  // part[z][t][e] (z < slices, row pitch router_rows(E)); the routing kernel writes them to
  // `logits` as f32.
  const double* part;
  int slices;
  // sqrt-softplus hash experts (DeepSeek V4's first layers): the token's row of the [vocab, K]
  // table `hash` (ids validated in range and distinct per row) replaces the ranking; a token id
  // >= vocab sets kStatusBadToken and reads row 0.
  const int32_t* hash;
  const uint32_t* tokens;
  uint32_t vocab;
};


// The top-k routing of a one-token call's token 0 of `logits` with `rp` into ids / weights /
// asc, run beside another kernel's work in its launch.
struct RouteJob {
  float* logits;
  int K;
  RouteParams rp;
  int32_t* ids;
  float* weights;
  int32_t* asc;
};

// Router logits, the reference's 8-lane FP32 tree (BF16-rounded when round_bf16).
// With `xp` (T = 1 only), the kernel also writes the token's BF16 piece vector there.
// w8b / logits_b (optional): a one-row matrix in the same layout (Qwen3.6's shared-expert gate)
// computed in the same launch below 64 tokens.
// xq: the token's piece vector (xp, one token) as the hi/lo split of x (0) or as
// simulate_e4m3_activation in blocks of xq = 32 or 128 values (the MX-activation compositions).
// lo_word (optional): set to lo_gen when some value of x is not BF16 (as launch_router_mfma).
void launch_router_lane8(const uint16_t* w8, int E, int H, const float* x, int T, float* logits,
                         int round_bf16, int* status, hipStream_t s, uint16_t* xp = nullptr,
                         const uint16_t* w8b = nullptr, float* logits_b = nullptr, int xq = 0,
                         unsigned* lo_word = nullptr, unsigned lo_gen = 0);

// GLM router logits: MFMA BF16 with f64 accumulation of 32-k partials, split over K into
// f64 partial slices.  The router weight is packed in the panel layout with router_rows(E)
// rows (zero padding).
__host__ __device__ inline int router_rows(int E) { return (E + kGemmNTile - 1) / kGemmNTile * kGemmNTile; }
constexpr int kRouterMaxSlices = 16;
int router_slices(int E, int H, int T);
// lo_word (optional): set to lo_gen when some lo half of x's hi/lo BF16 split is non-zero (the
// grouped GEMMs' Epi::lo_word test).  xb (optional): x's hi halves (x as BF16 where it is
// BF16-valued), [T, H] row-major, for Epi::xb.
void launch_router_mfma(const uint8_t* wp, int E, int H, const float* x, int T, double* part,
                        int slices, int* status, hipStream_t s, unsigned* lo_word = nullptr,
                        unsigned lo_gen = 0, uint16_t* xb = nullptr);
// One token: the f64 partial slices part[z][0][e] of the row-major router [E, H] from a GEMV
// (router_gemv_slices(E) slices, exact products summed in f64).
int router_gemv_slices(int E);
void launch_router_gemv_f64(const uint16_t* w, int E, int H, const float* x, double* part,
                            int slices, int* status, hipStream_t s, uint16_t* xp = nullptr,
                            int xq = 0);
void launch_relayout_lane8(const uint16_t* w, int E, int H, uint16_t* w8, hipStream_t s);
// Top-k routing, one wavefront per token (logits is an output when p.part is set).
void launch_route(float* logits, int T, int E, int K, const RouteParams& p, int32_t* ids,
                  float* weights, int32_t* asc, int* status, hipStream_t s);
// Permutation for T <= kMaxChunkTokens tokens.
constexpr int kMaxChunkTokens = 1024;
// slot_of_pos (may be null) receives the route slot t k + j of each permuted position.
void launch_permute(const int32_t* ids, int T, int E, int K, int32_t* meta, int32_t* active,
                    int32_t* offsets, int32_t* counts, int32_t* perm_token, int32_t* pos_of_slot,
                    int32_t* tiles, int32_t* slot_of_pos, hipStream_t s);
// One-token projections on the matrix cores (urb_decode.hip).  Inputs and activations are BF16
// piece vectors (urb_panel.hpp): `xp` [H / 8 units] for the token, `act_xp` [slot][I / 8 units].
// gate_up writes the activation as f32 (`act`, may be null) and/or pieces (`act_xp`); down
// writes f32 rows y [slot][H].  The fused down + combine runs when mfma_down_combine_fits
// (otherwise it returns false and launches nothing).
void launch_gemv_mfma_gate_up(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                              int H, int I, const uint16_t* xp, float* act, uint16_t* act_xp,
                              Epi epi, int* status, hipStream_t s);
void launch_gemv_mfma_down(int fmt, const ExpertMats* mats, const Perm& perm, int max_active,
                           int H, int I, const uint16_t* act_xp, float* y, Epi epi, int* status,
                           hipStream_t s);
// The shared expert's gate_up (the dense table entry 0, as launch_gemv_mfma_gate_up) and the
// routing of the token (`job`, E <= 512 experts) in one launch (urb_route.hip).
void launch_shared_gate_up_route(int fmt, const ExpertMats* mats, int H, int I,
                                 const uint16_t* xp, float* act, uint16_t* act_xp, Epi epi,
                                 int* status, hipStream_t s, int E, const RouteJob& job);
// One token without a shared expert: the routing inside the routed gate+up GEMV (every
// workgroup routes the token; the first one writes ids, weights, asc and a sliced router's
// logits).  Returns false (nothing launched) when top_k exceeds the kernel's LDS slots.
bool launch_routed_gate_up_route(int fmt, const ExpertMats* mats, int H, int I,
                                 const uint16_t* xp, uint16_t* act_xp, Epi epi, int* status,
                                 hipStream_t s, int E, const RouteJob& job);
// The routed gate_up (as launch_gemv_mfma_gate_up, epilogue `epi`) and the shared expert's down
// projection (the dense table entry 0, f32 rows into shared_out, epilogue `shared_epi`) in one
// launch.
void launch_gemv_mfma_gate_up_and_shared_down(int fmt, const ExpertMats* mats, const Perm& perm,
                                              int max_active, int H, int I, const uint16_t* xp,
                                              float* act, uint16_t* act_xp, Epi epi,
                                              int shared_fmt, const ExpertMats* shared_mats,
                                              int Is, const uint16_t* shared_xp,
                                              float* shared_out, Epi shared_epi, int* status,
                                              hipStream_t s);
bool mfma_down_combine_fits(int K, int I);
bool launch_gemv_mfma_down_combine(int fmt, const ExpertMats* mats, const int32_t* ids,
                                   const float* weights, const int32_t* asc, int K, int H, int I,
                                   const uint16_t* act_xp, const float* shared, int comp, Epi epi,
                                   float* out, int* status, hipStream_t s,
                                   const float* residual = nullptr, const float* gate = nullptr);
void launch_split_pieces(const float* x, size_t rows, size_t cols, uint16_t* out, hipStream_t s);
constexpr int kPieceUnit = 16;  // u16 per 8-value unit of a piece vector (hi, lo)
// Combines: Qwen BF16 ascending-id, GLM f64 ranking order.  Qwen with `shared` [T, H]: the
// gated shared expert (scale bf16(sigmoid(gate[t]))) added last; with `residual` [T, H]:
// out = bf16(residual + combined).
void launch_combine_qwen(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                         const int32_t* asc, int T, int K, int H, float* out, int* status,
                         hipStream_t s, const float* residual = nullptr,
                         const float* shared = nullptr, const float* gate = nullptr);
void launch_combine_glm(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                        const float* shared, int T, int K, int H, float* out, hipStream_t s);
// MX-activation mode.  simulate_e4m3_activation (src/math/mxfp.rs:89-115) of [rows, cols] f32
// (cols % block == 0) per `block`-value block of each row (32, or DeepSeek V4's 128): the
// simulated f32 values (`values`, may alias x) and/or the E4M3 codes [rows, cols] + E8M0 scales
// [rows, cols / block] they are made of; either output may be null.
// With `round_first`, each value is first multiplied by its row's weight (row_w[row_slot[row]],
// row_w[row] when row_slot is null, none when row_w is null) and rounded to BF16 (DeepSeek
// V4.1's weighted, BF16-materialised SwiGLU output).
// `pieces` (may be null): the simulated values as BF16 piece vectors [rows][cols / 8 units]
// (exact in the first piece).
void launch_quantize(const float* x, size_t rows, size_t cols, float* values, uint8_t* codes,
                     uint8_t* scales, int* status, hipStream_t s, int round_first = 0,
                     const float* row_w = nullptr, const int32_t* row_slot = nullptr,
                     int block = 32, uint16_t* pieces = nullptr);
// Hy4 combine: ascending expert id, f32, + shared, BF16 (weights null: the plain sum of DeepSeek
// V4.1, whose experts already applied their route weight).
void launch_combine_hy4(const float* y_perm, const int32_t* pos_of_slot, const float* weights,
                        const int32_t* asc, const float* shared, int T, int K, int H,
                        float* out, int* status, hipStream_t s);
// zero_centered_rms_norm + BF16 cast of T rows [T, H] (H % 4 == 0, H <= 16384), exact to the
// reference's sequential f32 mean square; non-finite input, weight, factor or output set
// kStatusNonFinite in `status` (may be null).
void launch_rms_norm(const float* h, const float* weight, int T, int H, float eps, float* out,
                     int* status, hipStream_t s);
// Payload validation: bit 1 = non-finite BF16 / E4M3 NaN code, bit 2 = E8M0 0xFF, bit 4 (with
// f16_range) = an E8M0 code outside [kF16ScaleLo, kF16ScaleHi] of the format.
void launch_validate(int fmt, const uint8_t* data, size_t data_bytes, const uint8_t* scales,
                     size_t scale_bytes, int* flags, hipStream_t s, bool f16_range = false);
void launch_dequant(int fmt, const uint8_t* data, const uint8_t* scales, int rows, int cols,
                    int row0, int count, float* out, hipStream_t s);
void launch_fill_i32(int32_t* p, int32_t v, size_t n, hipStream_t s);

// The shared expert of a large batch (urb_dense.hip): dense BF16 GEMMs over 256 x 256 tiles
// with split K, partial sums in `part` (part_floats floats, >= T * max(2 I, H)), then the
// gate/up epilogue into act [T, I].  dense_fits: the shapes and batch it takes (T >= 256; 2 I
// and H multiples of 256).  (A BF16 down projection from f32 rows measured faster on the
// grouped GEMM's dense tiles and runs there; the f16 one runs launch_dense_down_f16.)
bool dense_fits(int T, int I, int H, size_t part_floats);
void launch_dense_gate_up(const ExpertMats& m, int T, int H, int I, const float* x, float* act,
                          Epi epi, int* status, float* part, size_t part_floats, hipStream_t s);
// The same, the SwiGLU rows as f16 at each row's scale with the row's largest exponent field in
// rowexp[T] (the input of an f16 down projection: Epi::rowexp with one group).  I <= 16384.
void launch_dense_gate_up_f16(const ExpertMats& m, int T, int H, int I, const float* x,
                              uint16_t* act16, int* rowexp, Epi epi, int* status, float* part,
                              size_t part_floats, hipStream_t s);
// The f16 down projection out[T, H] of those f16 rows (rowexp) with w16, the f16 copy of the
// BF16 down matrix times 2^epi.wshift in the panel layout: 128-token x 256-row tiles, no K
// split, the down epilogue applied (the shapes dense_fits takes).
void launch_dense_down_f16(const uint16_t* w16, int T, int H, int I, const uint16_t* act16,
                           const int* rowexp, Epi epi, float* out, int* status, hipStream_t s);
// A BF16 matrix (n values, any layout) as f16: bf16_f16_shift returns the power of two that
// makes every value exactly an f16 (the non-zero values' exponents span at most 32 binades:
// the largest lands below 2^16, every significand bit at or above 2^-24), or kNoF16Shift;
// launch_bf16_to_f16 writes the values times 2^shift, element for element.
constexpr int kNoF16Shift = -1000;
int bf16_f16_shift(const uint16_t* w, size_t n);
void launch_bf16_to_f16(const uint16_t* w, size_t n, int shift, uint16_t* out, hipStream_t s);

// The allocation-free layer call's scratch (urb_scratch.hip): kScratchBytes of device memory per
// GPU, held until the process ends; the current device's address.
constexpr size_t kScratchBytes = 32u << 20;
hipError_t scratch_region(void** out);
void launch_check_finite(const float* x, size_t n, int* status, hipStream_t s);

}  // namespace urb
