/*
 * urb_moe.h -- C ABI of the MI355X (gfx950) routed-expert MoE layer.
 *
 * Plain pointers and sizes only.  Every pointer named "device" is HBM memory on the current
 * HIP device; `stream` is a hipStream_t passed as void* (NULL = the default stream).  All calls
 * on one context are stream-ordered and must not overlap on different streams.
 *
 * Each entry point replaces a reference (inspirewind/Urbilateria 0.2.4, Rust) interface, cited
 * below as file:line.  Status codes 1..4 mirror the reference's error enums.
 */
#ifndef URB_MOE_H
#define URB_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  URB_OK = 0,
  URB_ERR_SHAPE = 1,            /* MxError::Shape, MatrixError::{InvalidShape, InputLength} */
  URB_ERR_INVALID_SCALE = 2,    /* MxError::InvalidScale (E8M0 0xFF)                         */
  URB_ERR_NONFINITE = 3,        /* MxError/MatrixError/RouteError::NonFinite                 */
  URB_ERR_INVALID_GEOMETRY = 4, /* RouteError::InvalidGeometry, Qwen38MoeError::InvalidGeometry */
  URB_ERR_DEVICE = 5,           /* HIP runtime failure                                        */
  URB_ERR_OUT_OF_MEMORY = 6,
  URB_ERR_ARGUMENT = 7          /* null pointer, unsupported option                           */
} urb_status;

/* Expert weight formats: WeightMatrix::{Bf16, MxFp4, MxFp8} (src/model/weight.rs:54-61).
 * MX formats use E8M0 scales per 32 consecutive columns of a row (MXFP8: ModelOpt 1x32). */
typedef enum { URB_FMT_BF16 = 0, URB_FMT_MXFP4 = 1, URB_FMT_MXFP8 = 2 } urb_format;

/* route_softmax_top_k (src/models/qwen3_8/moe.rs:91-159), route_noaux_tc
 * (src/math/routing.rs:38-155) or route_sqrt_softplus (src/models/deepseek_v4/math.rs:451-516;
 * not with QWEN36), with hash experts when the weights carry a tid2eid table. */
typedef enum {
  URB_ROUTER_SOFTMAX_TOPK = 0,
  URB_ROUTER_SIGMOID_NOAUX_TC = 1,
  URB_ROUTER_SQRT_SOFTPLUS = 2
} urb_router;

/* Which adapter's layer call the context reproduces:
 *  QWEN36: execute_streamed_moe / execute_batched_moe (src/models/qwen3_6/runtime.rs:1067-1243):
 *          BF16 router GEMV (FP32, 8-lane tree) + BF16 logits, BF16 route weights, BF16
 *          boundaries inside experts and in the ascending-expert-id combine; with a shared
 *          expert (BF16, shared_intermediate > 0) finish_ordered_moe (:1417-1468): the shared
 *          expert's output scaled by bf16(sigmoid(shared_expert_gate . x)) and added last, in
 *          BF16.
 *  GLM:    RuntimeMoeLayer::forward (src/models/glm/runtime/moe.rs:138-176): f64 router GEMV,
 *          GatedMlp experts, f64 combine in ranking order on top of the shared expert.
 *  HY4:    the MX-activation mode, Hy4 MoeWeights::forward (src/models/hy4/runtime.rs:
 *          1371-1447): f64 router GEMV; the token's activation quantized to E4M3 per 32 values
 *          (simulate_e4m3_activation, src/math/mxfp.rs:89-115) feeds every MX projection;
 *          routed experts Hy4Expert::forward_quantized (src/models/hy4/expert.rs:373-392,
 *          664-680: BF16 gate/up, bounded SwiGLU with swiglu_limit, re-quantized, BF16 down);
 *          shared expert DenseMlp::forward (runtime.rs:1311-1322); f32 combine in ascending
 *          expert id plus the shared expert, rounded to BF16.  MX expert and shared formats.
 *  DSV41:  the MX-activation mode of DeepSeek-V4.1 MoeWeights::forward
 *          (src/models/deepseek_v41/runtime.rs:1963-2019): FP32 8-lane router GEMV (no BF16
 *          step), E4M3 activations per 32 values, experts Expert::forward_with_mx_input
 *          (runtime.rs:2243-2261: FP32-accumulated BF16 gate/up, bounded SwiGLU with
 *          swiglu_limit, times the route weight before the BF16 step and the down projection);
 *          the shared expert is the same without a weight; f32 sum in ascending expert id plus
 *          the shared expert, BF16.  MX expert and shared formats; route_sqrt_softplus is its
 *          router.
 *  DSV4:   DeepSeek-V4 MoeWeights::forward{,_batch} (src/models/deepseek_v4/runtime.rs:
 *          2484-2828): as DSV41 but the router GEMV is the ordered f64 `linear(router)`
 *          (deepseek_v4/math.rs:106-115) and the activations are quantized per 128 values
 *          (prepare_mx_activation, math.rs:120-126) before the MX projections
 *          (DeepExpert::forward_with_mx_input, runtime.rs:3081-3155).  The first
 *          num_hash_layers layers route by a tid2eid table (urb_moe_weights.hash_experts). */
typedef enum {
  URB_COMPOSE_QWEN36 = 0,
  URB_COMPOSE_GLM = 1,
  URB_COMPOSE_HY4 = 2,
  URB_COMPOSE_DSV41 = 3,
  URB_COMPOSE_DSV4 = 4
} urb_composition;

/* Where urb_moe_create reads the weights from.  The context streams expert and shared-expert
 * matrices in the panel layout (see urb_pack_matrix); HOST and DEVICE_COPY sources are in the
 * row-major checkpoint layout below and are converted while they are copied into the context's
 * HBM arena.  DEVICE_BORROW matrices must already be in the panel layout; they are used in
 * place and must outlive the context.  The router weight and bias are always row-major and
 * always copied. */
typedef enum {
  URB_SOURCE_HOST = 0,
  URB_SOURCE_DEVICE_COPY = 1,
  URB_SOURCE_DEVICE_BORROW = 2
} urb_weight_source;

/* One matrix in its on-disk layout (row-major [rows, cols]):
 *   BF16:  little-endian u16 [rows, cols]                     (Bf16Matrix, src/model/bf16.rs:10-15)
 *   MXFP4: E2M1 nibbles [rows, cols/2], low nibble first      (MxFp4Matrix, src/math/mxfp.rs:1362-1369)
 *   MXFP8: E4M3FN bytes [rows, cols]                          (MxFp8Matrix, src/math/mxfp.rs:321-329)
 *   scales: E8M0 [rows, cols/32] for MX formats, NULL for BF16. */
typedef struct {
  const void *data;
  const uint8_t *scales;
} urb_matrix;

/* Layer geometry: MoeGeometry (src/models/glm/moe_geometry.rs:3-9) plus projection formats.
 * hidden, intermediate and shared_intermediate must be multiples of 128 and at most 12288
 * (URB_ERR_SHAPE otherwise); top_k <= 32, n_experts <= 512. */
typedef struct {
  uint32_t hidden;               /* H */
  uint32_t n_experts;            /* E */
  uint32_t top_k;                /* k */
  uint32_t intermediate;         /* I of each routed expert */
  uint32_t shared_intermediate;  /* I of the always-on shared expert, 0 = none */
  urb_format expert_format;
  urb_format shared_format;
  urb_router router;
  urb_composition composition;
  uint32_t n_group, topk_group;  /* noaux_tc group limiting; 1, 1 = none */
  int32_t normalize;             /* noaux_tc: divide by the selected gate sum */
  float routed_scaling_factor;   /* noaux_tc, sqrt_softplus */
  uint32_t max_tokens;           /* largest token count one forward call may pass */
  float swiglu_limit;            /* HY4, DSV41, DSV4: bounded SwiGLU limit (> 0) */
} urb_moe_desc;

typedef struct {
  const uint16_t *router_weight;   /* [E, H] BF16 */
  const float *correction_bias;    /* [E] f32 selection bias (noaux_tc), NULL = zeros */
  const urb_matrix *experts;       /* [E * 3]: gate [I, H], up [I, H], down [H, I] */
  const urb_matrix *shared;        /* [3] or NULL */
  /* QWEN36 with a shared expert: mlp.shared_expert_gate [1, H] BF16, the sigmoid gate of the
   * shared expert's contribution (finish_ordered_moe, src/models/qwen3_6/runtime.rs:1417-1468);
   * NULL otherwise. */
  const uint16_t *shared_expert_gate;
  /* route_sqrt_softplus hash experts: layers.N.ffn.gate.tid2eid [hash_vocab, top_k] i64, the
   * experts of each token id in table order (src/models/deepseek_v4/runtime.rs:2664-2681), in
   * the memory the source names; NULL = routing by score.  Checked at creation: every id in
   * [0, E) (URB_ERR_INVALID_GEOMETRY, the reference's "hash expert IDs must be in range",
   * math.rs:483-489) and distinct within a row (URB_ERR_ARGUMENT: the reference would run a
   * repeated expert twice; the permutation here needs distinct ids).  Layer calls then take
   * token ids (urb_moe_forward_tokens / urb_moe_route_tokens). */
  const int64_t *hash_experts;
  uint32_t hash_vocab;
} urb_moe_weights;

typedef struct urb_moe_ctx urb_moe_ctx;

/* Builds a layer: shape/geometry checks, upload (panel layout), one validation pass over every payload
 * (E8M0 0xFF -> URB_ERR_INVALID_SCALE; E4M3 0x7F/0xFF or non-finite BF16 -> URB_ERR_NONFINITE).
 * Replaces RuntimeMoeLayer::new (src/models/glm/runtime/moe.rs:78-125) together with the
 * payload checks of MxFp4Matrix::from_packed (src/math/mxfp.rs:1371-1443), MxFp8Matrix::
 * from_packed (src/math/mxfp.rs:338-457) and Bf16Matrix::from_le_bytes (src/model/bf16.rs:18-70). */
urb_status urb_moe_create(const urb_moe_desc *desc, const urb_moe_weights *weights,
                          urb_weight_source source, urb_moe_ctx **out);
void urb_moe_destroy(urb_moe_ctx *ctx);

/* One layer call over `tokens` rows x [tokens, H] (device, f32) -> y [tokens, H] (device, f32);
 * routes per token in ranking order: ids [tokens, k] (device, i32) and weights [tokens, k]
 * (device, f32), either may be NULL.  Replaces execute_streamed_moe / execute_batched_moe
 * (src/models/qwen3_6/runtime.rs:1067-1243) for QWEN36 and RuntimeMoeLayer::forward
 * (src/models/glm/runtime/moe.rs:138-176) for GLM.  1 <= tokens <= desc.max_tokens, else
 * URB_ERR_SHAPE and nothing is enqueued.  Enqueues only: numerical failures the reference
 * reports (non-finite input, activations or outputs) are latched on the device and returned by
 * urb_moe_sync. */
urb_status urb_moe_forward(urb_moe_ctx *ctx, const float *x, uint32_t tokens, float *y,
                           int32_t *ids, float *weights, void *stream);

/* urb_moe_forward with the tokens' ids [tokens] (device, u32), which hash routing needs
 * (MoeWeights::forward's `token`, src/models/deepseek_v4/runtime.rs:2484-2495, 2664-2681); an
 * id >= hash_vocab is reported by urb_moe_sync as URB_ERR_SHAPE (load_i64_matrix_row's bounds
 * check).  Without a hash table the ids are not read.  urb_moe_forward on a context with a hash
 * table returns URB_ERR_ARGUMENT. */
urb_status urb_moe_forward_tokens(urb_moe_ctx *ctx, const float *x, const uint32_t *token_ids,
                                  uint32_t tokens, float *y, int32_t *ids, float *weights,
                                  void *stream);

/* No counterpart in the reference: urb_moe_forward for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid it).  The
 * call allocates nothing: its buffers (logits, routes, permutation, activations, per-slot
 * outputs) come from a static 32 MiB scratch array each GPU holds until the process ends,
 * instead of the context's workspace.  Same kernels, results and status reporting as
 * urb_moe_forward (failures latch in the context, returned by urb_moe_sync).  Limits: 1 <=
 * tokens <= the context's max_tokens chunk, and the call's buffers must fit the scratch, else
 * URB_ERR_SHAPE: one token fits every supported shape; an H 7168, E 384, top-8, I 2048 layer
 * with a 2048-wide shared expert takes up to 88 tokens, an H 2048, E 128, top-8, I 768 one 312.
 * Contexts with a hash table return URB_ERR_ARGUMENT (use urb_moe_forward_tokens).  Every call on a GPU shares that GPU's scratch: calls that
 * overlap on one GPU (other streams, other threads, other contexts) race and must be
 * serialised by the caller. */
urb_status urb_moe_forward_noalloc(urb_moe_ctx *ctx, const float *x, uint32_t tokens, float *y,
                                   int32_t *ids, float *weights, void *stream);

/* Router only: logits [tokens, E] (device, may be NULL), ids/weights as above.  Replaces
 * `linear(router)` + route_softmax_top_k (src/models/qwen3_8/math.rs:10-26,
 * src/models/qwen3_8/moe.rs:91-159) and router.matvec + route_noaux_tc
 * (src/models/glm/runtime/moe.rs:152-161). */
urb_status urb_moe_route(urb_moe_ctx *ctx, const float *x, uint32_t tokens, float *logits,
                         int32_t *ids, float *weights, void *stream);
/* urb_moe_route with token ids, as urb_moe_forward_tokens (DeepSeek-V4 prepare_routes,
 * src/models/deepseek_v4/runtime.rs:2656-2703). */
urb_status urb_moe_route_tokens(urb_moe_ctx *ctx, const float *x, const uint32_t *token_ids,
                                uint32_t tokens, float *logits, int32_t *ids, float *weights,
                                void *stream);

/* Waits for `stream` and returns the first numerical failure latched since the previous
 * urb_moe_sync (URB_OK if none), then clears it.  The Result of the reference's layer calls. */
urb_status urb_moe_sync(urb_moe_ctx *ctx, void *stream);

/* Dequantised rows [count, cols] f32 (device) of one matrix (device): Bf16Matrix::write_row
 * (src/model/bf16.rs:92-113), MxFp4Matrix::row (src/math/mxfp.rs:1828-1846), MxFp8Matrix::row
 * (src/math/mxfp.rs:855-877).  Bit-exact: value = decode(code) * scale in f32. */
urb_status urb_dequant_rows(urb_format format, const void *data, const uint8_t *scales,
                            uint32_t rows, uint32_t cols, uint32_t row0, uint32_t count,
                            float *out, void *stream);

/* The decoder layer's FFN block around the MoE call, for the QWEN36 composition
 * (src/models/qwen3_6/runtime.rs:1053-1060 tokenwise, :1001-1019 batched):
 *   n = bf16(zero_centered_rms_norm(h, norm_weight, eps)),  out = bf16(h + moe(n))
 * h, out [tokens, H] (device, f32; out may alias h), norm_weight [H] (device, f32: the
 * checkpoint's post_attention_layernorm offset, the scale being 1 + weight); ids / weights as
 * urb_moe_forward.  The mean square is the reference's sequential f32 sum
 * (src/models/qwen3_8/norm.rs:176-186), so the MoE sees the reference's inputs bit for bit.
 * eps not finite or <= 0 -> URB_ERR_INVALID_GEOMETRY (NormError::InvalidEpsilon); non-finite
 * h, norm_weight or results -> URB_ERR_NONFINITE at urb_moe_sync (NormError::NonFinite, the
 * residual's "produced NaN or infinity"); other compositions -> URB_ERR_ARGUMENT. */
urb_status urb_moe_forward_block(urb_moe_ctx *ctx, const float *h, const float *norm_weight,
                                 float eps, uint32_t tokens, float *out, int32_t *ids,
                                 float *weights, void *stream);

/* zero_centered_rms_norm + round_runtime_bf16 of [rows, hidden] f32 rows (device; hidden % 4
 * == 0 and <= 16384): the bit-exact parity hook of urb_moe_forward_block's first step
 * (src/models/qwen3_8/norm.rs:38-52; src/models/qwen3_6/runtime.rs:1053-1057).  Inputs must be
 * finite (the block call reports non-finite ones). */
urb_status urb_zc_rms_norm_bf16(const float *x, const float *weight, uint32_t rows,
                                uint32_t hidden, float eps, float *out, void *stream);

/* simulate_e4m3_activation (src/math/mxfp.rs:82-115) of a [rows, cols] f32 matrix (device,
 * cols % 32 == 0) per 32-value block of each row, as the MX-activation mode feeds it to the
 * scaled MFMA: E4M3 codes [rows, cols] and E8M0 scales [rows, cols / 32] (device); the
 * simulated value is decode_e4m3fn(code) * 2^(scale - 127).  The bit-exact parity hook of the
 * quantizer; inputs must be finite (the layer call reports non-finite ones). */
urb_status urb_quantize_e4m3(const float *x, uint32_t rows, uint32_t cols, uint8_t *codes,
                             uint8_t *scales, void *stream);
/* urb_quantize_e4m3 per `block` values (32, or 128: DeepSeek-V4 prepare_mx_activation,
 * src/models/deepseek_v4/math.rs:120-126); cols % block == 0; scales [rows, cols / block].
 * Other block widths -> URB_ERR_ARGUMENT. */
urb_status urb_quantize_e4m3_blocks(const float *x, uint32_t rows, uint32_t cols, uint32_t block,
                                    uint8_t *codes, uint8_t *scales, void *stream);

/* Converts one row-major matrix (device, the urb_matrix layout) into the panel layout the
 * context streams (device; same byte counts: packed_data as large as data, packed_scales as
 * large as scales).  rows % 16 == 0 and cols % 128 == 0, else URB_ERR_SHAPE.  A panel is 16
 * consecutive rows; its bytes are reordered so that 1 KiB slab t holds, in 16-byte unit
 * l = ln + 16 lq, row ln's columns 32t+8lq..+8 (BF16), MX block 4t+lq (MXFP4), or half t%2 of
 * MX block 4(t/2)+lq (MXFP8); scales per panel are 64-byte slabs, byte l of slab s being row
 * ln's scale of block 4s+lq.  No reference counterpart: the reference keeps the checkpoint
 * layout (MxFp4Matrix::from_packed, src/math/mxfp.rs:1362-1443); this is the HBM layout for
 * callers that borrow pre-converted weights. */
urb_status urb_pack_matrix(urb_format format, const void *data, const uint8_t *scales,
                           uint32_t rows, uint32_t cols, void *packed_data,
                           uint8_t *packed_scales, void *stream);

/* Points expert `expert` of a URB_SOURCE_DEVICE_BORROW context at other panel-layout matrices
 * (mats[3]: gate, up, down, device, as urb_pack_matrix writes them): with
 * include/urb_residency.h this is how a caller keeps a subset of a layer's experts resident in
 * HBM slots of its own and swaps them between calls.  The payload is validated first, as
 * urb_moe_create does (E8M0 0xFF -> URB_ERR_INVALID_SCALE; E4M3 NaN codes or non-finite BF16
 * -> URB_ERR_NONFINITE, the entry unchanged); the change is ordered on `stream` and the call
 * returns once it is in place.  Other contexts -> URB_ERR_ARGUMENT.  No reference counterpart:
 * the reference's expert stores hand the layer owned matrices per access
 * (Qwen36ExpertStore::acquire / acquire_grouped, src/models/qwen3_6/expert_store.rs:291-317). */
urb_status urb_moe_set_expert(urb_moe_ctx *ctx, uint32_t expert, const urb_matrix *mats,
                              void *stream);

/* Per-expert views of consolidated checkpoint tensors, for urb_moe_weights.experts: fills
 * out[E * 3] with pointers into the tensors (no copy, no device work).  gate_up is [E, 2I, H]
 * with each expert's gate rows 0..I-1 followed by its up rows I..2I-1, down is [E, H, I], both
 * in the urb_matrix layout per expert; the scale tensors are [E, 2I, H/32] and [E, H, I/32]
 * for the MX formats and NULL for BF16 (URB_ERR_ARGUMENT otherwise); H and I multiples of 32.
 * Replaces the per-expert slicing of the Qwen3.6 packed BF16 gate_up_proj / down_proj
 * (src/models/qwen3_6/expert_store.rs:125-158) and of the Hy4 consolidated E4M3 + U8-scale
 * tensors (src/models/hy4/expert.rs:436-625, gate/up split at I as activate_gate_up,
 * src/models/hy4/expert.rs:664-680). */
urb_status urb_expert_views(urb_format format, uint32_t n_experts, uint32_t hidden,
                            uint32_t intermediate, const void *gate_up,
                            const uint8_t *gate_up_scales, const void *down,
                            const uint8_t *down_scales, urb_matrix *out);

/* Device-time spans per stage of a layer call: the counterpart of the reference's profiling
 * spans (ProfileStage, src/profiling.rs:75-136; span_with_work, src/profiling.rs:581-600).
 * While enabled, every forward call brackets each stage with HIP events on the stream the
 * stage's kernels run on and waits for them, so enable it for measurement runs only. */
typedef enum {
  URB_STAGE_ROUTER = 0,          /* router GEMV/GEMM -> logits           */
  URB_STAGE_ROUTE = 1,           /* top-k routing                        */
  URB_STAGE_PERMUTE = 2,         /* token -> expert permutation          */
  URB_STAGE_GATE_UP = 3,         /* routed gate+up projections + SwiGLU  */
  URB_STAGE_DOWN = 4,            /* routed down projections              */
  URB_STAGE_SHARED_GATE_UP = 5,  /* shared expert gate+up + SwiGLU       */
  URB_STAGE_SHARED_DOWN = 6,     /* shared expert down                   */
  URB_STAGE_COMBINE = 7,         /* weighted combine                     */
  URB_STAGE_COUNT = 8
} urb_stage;

/* Starts (enable != 0) or stops collecting; starting clears the totals. */
urb_status urb_moe_profile(urb_moe_ctx *ctx, int enable);
/* Total milliseconds and number of launches per stage since profiling was enabled
 * (arrays of URB_STAGE_COUNT). */
urb_status urb_moe_profile_read(const urb_moe_ctx *ctx, double *ms, uint64_t *launches);

/* HBM bytes the context holds for weights (own arena, plus the f16 copy of a GLM layer's BF16
 * shared down matrix that its batches of 256+ tokens multiply; 0 when borrowed) and workspace. */
urb_status urb_moe_memory(const urb_moe_ctx *ctx, size_t *weight_bytes, size_t *workspace_bytes);

const char *urb_status_string(urb_status status);

/* safetensors element types of the tensors expert matrices are stored in. */
typedef enum {
  URB_DTYPE_BF16 = 0,
  URB_DTYPE_F16 = 1,
  URB_DTYPE_F32 = 2,
  URB_DTYPE_F8_E4M3 = 3,
  URB_DTYPE_I8 = 4,
  URB_DTYPE_U8 = 5,
  URB_DTYPE_F8_E8M0 = 6,
  URB_DTYPE_OTHER = 7
} urb_dtype;

/* A tensor's safetensors header entry: dtype, shape (ndim <= 2 used) and payload bytes. */
typedef struct {
  urb_dtype dtype;
  uint32_t ndim;
  uint64_t shape[2];
  uint64_t data_len;
} urb_tensor_meta;

/* Replaces inspect_weight_matrix (src/storage/weight.rs:118-330) for the formats this layer
 * takes, from metadata only (no payload read): the format of a logical [rows, cols] matrix
 * stored as `weight` with its MX scale sidecar `scale` (NULL when the checkpoint has none;
 * the caller finds it as find_native_scale_name does, weight.rs:645-653), and `packed_name`
 * != 0 when the weight's name ends in ".weight_packed".  Selection as the reference:
 * plain BF16 [rows, cols] without a sidecar -> URB_FMT_BF16; F8_E4M3 [rows, cols] with a U8
 * [rows, ceil(cols/32)] sidecar (ModelOpt 1x32) -> URB_FMT_MXFP8; I8 (F8_E8M0 sidecar) or U8
 * ".weight_packed" (U8 sidecar) [rows, ceil(cols/2)] with a [rows, ceil(cols/32)] sidecar ->
 * URB_FMT_MXFP4.  *resident_bytes = payload + sidecar bytes.  A plain BF16 matrix stays
 * compact BF16 in this layer (its resident bytes are the payload, rows * cols * 2, as the
 * reference's inspect_compact_bf16_matrix reports, weight.rs:337-380, fixture :1237-1243);
 * this differs on purpose from inspect_weight_matrix, which widens plain matrices to F32
 * (rows * cols * 4, weight.rs:155-170, fixture :1267-1273): the GPU layer never widens.
 * Errors: rows or cols 0, or a
 * shape or sidecar that does not match the format the dtypes select -> URB_ERR_SHAPE
 * (InvalidShape); layouts the reference reads but this layer does not take -> URB_ERR_ARGUMENT
 * (F16/F32 plain matrices, E4M3 with 32x32 or 128x128 E8M0 block scales or without a sidecar,
 * Colibri INT4/INT8 and other dtypes: the reference's other formats and Unsupported). */
urb_status urb_inspect_matrix(const urb_tensor_meta *weight, const urb_tensor_meta *scale,
                              int packed_name, uint32_t rows, uint32_t cols, urb_format *format,
                              uint64_t *resident_bytes);

/* Diagnostic, host only, no reference counterpart: the grouped GEMM's workgroup placement for
 * a launch over `tiles` row tiles of a [rows, cols] projection in `format` (pair != 0: the
 * gate+up pair), with dense_tokens > 0 for one dense expert (the shared expert) over that many
 * tokens.  Writes the row tile and panel group of each of the first `capacity` workgroups (-1
 * for a workgroup with no work) and returns the grid size.  Lets a test check that every XCD
 * gets work and every (tile, group) pair is covered once. */
uint32_t urb_gemm_placement(urb_format format, int pair, uint32_t dense_tokens, uint32_t tiles,
                            uint32_t rows, uint32_t cols, int32_t *tile_of_block,
                            int32_t *group_of_block, uint32_t capacity);

#ifdef __cplusplus
}
#endif
#endif /* URB_MOE_H */
