/*
 * urb_oracle.h -- CPU restatement of the reference's routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the timed CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product
 * (urbilateria_amd/, include/urb_moe.h) never links, loads or calls it.
 *
 * Every function restates one function of inspirewind/Urbilateria 0.2.4 (Rust), cited as
 * file:line.  The reference cannot be compiled here (no Rust toolchain, crates not vendored),
 * so these are restatements, pinned by the reference's own known-answer tests and by closed
 * forms in tests/test_oracle_*.py.
 *
 * Host assumptions the reference makes at run time and this restatement fixes:
 *   - x86_64 with AVX2 + FMA: the reference then selects the 8-lane FP32-FMA BF16 GEMV
 *     (src/model/bf16.rs:249-251) and the compact 1x32 MXFP8 kernel (src/math/mxfp.rs:720-729).
 *   - Rust f32::exp is the platform libm expf (glibc on x86_64-linux-gnu).
 */
#ifndef URB_ORACLE_H
#define URB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the reference's error enums collapsed to one integer space. */
enum {
    URBO_OK = 0,
    URBO_SHAPE = 1,            /* MxError::Shape, MatrixError::{InvalidShape,InputLength} */
    URBO_INVALID_SCALE = 2,    /* MxError::InvalidScale (E8M0 0xFF) */
    URBO_NONFINITE = 3,        /* MxError::NonFinite, MatrixError::NonFinite, RouteError::NonFinite */
    URBO_INVALID_GEOMETRY = 4, /* RouteError::InvalidGeometry, Qwen38MoeError::InvalidGeometry */
};

/* F32: little-endian f32 [rows, cols], WeightMatrix::F32 (src/model/matrix.rs), the format of
 * DeepSeek V4's reference fixtures. */
enum { URBO_FMT_BF16 = 0, URBO_FMT_MXFP4 = 1, URBO_FMT_MXFP8 = 2, URBO_FMT_F32 = 3 };
enum { URBO_ROUTER_SOFTMAX_TOPK = 0, URBO_ROUTER_SIGMOID_NOAUX_TC = 1, URBO_ROUTER_SQRT_SOFTPLUS = 2 };
/* QWEN36: execute_streamed_moe / execute_batched_moe (src/models/qwen3_6/runtime.rs:1067-1243).
 * GLM:    RuntimeMoeLayer::forward (src/models/glm/runtime/moe.rs:138-176).
 * HY4:    Hy4 MoeWeights::forward (src/models/hy4/runtime.rs:1371-1447).
 * DSV41:  DeepSeek-V4.1 MoeWeights::forward (src/models/deepseek_v41/runtime.rs:1963-2019).
 * DSV4:   DeepSeek-V4 MoeWeights::forward{,_batch} (src/models/deepseek_v4/runtime.rs:2484-2828). */
enum { URBO_COMPOSE_QWEN36 = 0, URBO_COMPOSE_GLM = 1, URBO_COMPOSE_HY4 = 2, URBO_COMPOSE_DSV41 = 3,
       URBO_COMPOSE_DSV4 = 4 };

/* ---- element decoders (src/math/mxfp.rs, src/model/bf16.rs, src/models/qwen3_8/math.rs) ---- */
int urbo_decode_e8m0(uint8_t code, float *out);
float urbo_decode_e2m1(uint8_t code);
float urbo_decode_e4m3fn(uint8_t code);
uint8_t urbo_encode_e4m3fn_finite(float value);
float urbo_power_of_two_ceiling(float value);
int urbo_simulate_e4m3_activation(float *values, size_t n, size_t block);
int urbo_round_to_bf16(float value, float *out);
int urbo_round_to_bf16_in_place(float *values, size_t n);

/* ---- matrices: row-major [rows, cols] in the reference's packed layouts ---- */
int urbo_validate(int format, const uint8_t *data, const uint8_t *scales, size_t rows, size_t cols);
int urbo_row(int format, const uint8_t *data, const uint8_t *scales, size_t rows, size_t cols,
             size_t row, float *out);
/* WeightMatrix::matvec_rows for the format (BF16 and MXFP4: ordered f64; MXFP8 1x32: compact FMA). */
int urbo_matvec_rows(int format, const uint8_t *data, const uint8_t *scales, size_t rows,
                     size_t cols, size_t start, size_t count, const float *x, float *out);
/* Bf16Matrix::matvec_rows_fp32 (8-lane FMA tree). */
int urbo_bf16_matvec_rows_fp32(const uint16_t *data, size_t rows, size_t cols, size_t start,
                               size_t count, const float *x, float *out);
/* MxFp4Matrix::matvec_rows_fp32 (sequential fp32, no FMA). */
int urbo_mxfp4_matvec_rows_fp32(const uint8_t *packed, const uint8_t *scales, size_t rows,
                                size_t cols, size_t start, size_t count, const float *x,
                                float *out);
/* MxFp8Matrix::matvec_rows with the ordered-f64 kernel (non-AVX2 hosts / block layouts). */
int urbo_mxfp8_matvec_rows_f64(const uint8_t *codes, const uint8_t *scales, size_t rows,
                               size_t cols, size_t start, size_t count, const float *x,
                               float *out);

/* ---- routers ---- */
int urbo_route_softmax_top_k(const float *logits, size_t n, size_t top_k, int32_t *ids,
                             float *weights);
int urbo_route_noaux_tc(const float *logits, const float *bias, size_t n, size_t top_k,
                        size_t n_group, size_t topk_group, int normalize, float scale,
                        int32_t *ids, float *weights, float *selection);
/* route_sqrt_softplus (src/models/deepseek_v4/math.rs:451-516), no hash experts. */
int urbo_route_sqrt_softplus(const float *logits, const float *bias, size_t n, size_t top_k,
                             float scale, int32_t *ids, float *weights, float *selection_out);
/* The same with hash_experts = hash[0..top_k) (NULL: none); ids out of range ->
 * URBO_INVALID_GEOMETRY (DeepseekMathError::Invalid). */
int urbo_route_sqrt_softplus_hashed(const float *logits, const float *bias, const int64_t *hash,
                                    size_t n, size_t top_k, float scale, int32_t *ids,
                                    float *weights, float *selection_out);
float urbo_silu(float value);
/* The reference's execution contract (src/execution.rs:254-394): the number of physical cores
 * in the allowed CPU set (recommended_worker_threads), and the allowed logical CPUs in
 * physical-core-first order (room for `capacity`; returns the count).  With pinning on, worker i
 * of the row-parallel pool runs pinned to the i-th CPU of that order; returns the previous
 * setting.  Default off. */
int urbo_physical_cores(void);
size_t urbo_cpu_order(int *cpus, size_t capacity);
int urbo_set_pinning(int enable);
/* Selects MxFp8Matrix::matvec_rows's host kernel for layer calls (src/math/mxfp.rs:720-765):
 * 1 = compact 8-lane FMA (AVX2+FMA hosts, the default), 0 = ordered f64.  Returns the previous. */
int urbo_set_mxfp8_fma_host(int fma_host);
/* bounded_swiglu (src/models/deepseek_v4/math.rs:526-548): out = min(g, L) / (1 + exp(-min(g, L)))
 * * clamp(u, -L, L). */
int urbo_bounded_swiglu(const float *gate, const float *up, size_t n, float limit, float *out);

/* ---- the decoder layer's steps either side of the MoE call (Qwen3.6) ---- */
/* zero_centered_rms_norm (src/models/qwen3_8/norm.rs:38-52, 142-193) of each of n rows [n, H],
 * followed (round_bf16 != 0) by round_runtime_bf16 (src/models/qwen3_6/runtime.rs:1053-1057):
 * mean square as the sequential f32 sum of x*x divided by H, inverse = 1 / sqrt(mean_square +
 * eps), out = x * inverse * (1 + weight).  eps must be finite and > 0 (URBO_INVALID_GEOMETRY
 * otherwise); non-finite input, weight, factor or output -> URBO_NONFINITE. */
int urbo_zc_rms_norm(const float *x, const float *weight, size_t n, size_t hidden, float eps,
                     int round_bf16, float *out);
/* add_residual with BF16 activations (src/models/qwen3_6/runtime.rs:1470-1494): residual +=
 * update in f32, rounded to BF16; non-finite -> URBO_NONFINITE. */
int urbo_add_residual_bf16(float *residual, const float *update, size_t n);

/* ---- one MoE layer ---- */
typedef struct {
    const uint8_t *data;   /* BF16 LE bytes, packed E2M1 nibbles, or E4M3 bytes */
    const uint8_t *scales; /* E8M0 [rows, cols/32]; NULL for BF16 */
} urbo_matrix;

typedef struct {
    uint32_t hidden, n_experts, top_k, intermediate, shared_intermediate;
    int32_t expert_format, shared_format, router, composition;
    uint32_t n_group, topk_group;
    int32_t normalize;
    float routed_scaling_factor;
    const uint16_t *router_weight; /* [E, H] BF16 */
    const float *correction_bias;  /* [E] or NULL (zeros) */
    const urbo_matrix *experts;    /* [E][3] = gate [I,H], up [I,H], down [H,I] */
    const urbo_matrix *shared;     /* [3] or NULL */
    float swiglu_limit;            /* HY4, DSV41, DSV4: bounded SwiGLU limit */
    const uint16_t *shared_expert_gate; /* QWEN36 with a shared expert: [H] BF16 gate row */
    /* DeepSeek hash routing: layers.N.ffn.gate.tid2eid [hash_vocab, top_k] (NULL = none); the
     * layer call then needs token ids (urbo_moe_forward_tokens). */
    const int64_t *hash_experts;
    uint32_t hash_vocab;
    const float *router_weight_f32; /* DSV4: an F32 [E, H] router instead of router_weight */
} urbo_layer;

/* Hy4 MX-activation experts over n tokens [n, H] -> [n, H] (x is quantized here):
 * routed Hy4Expert::forward_quantized (src/models/hy4/expert.rs:373-392, 664-680) when
 * swiglu_limit > 0, else the shared DenseMlp::forward (src/models/hy4/runtime.rs:1311-1322). */
int urbo_hy4_expert(int format, const urbo_matrix *gate_up_down, uint32_t hidden,
                    uint32_t intermediate, const float *x, uint32_t n, float swiglu_limit,
                    float *y, int threads);
/* DeepSeek-V4.1 Expert::forward_with_mx_input (src/models/deepseek_v41/runtime.rs:2243-2261)
 * over n tokens [n, H] (x quantized here); route_weights [n] or NULL (the shared expert). */
int urbo_dsv41_expert(int format, const urbo_matrix *gate_up_down, uint32_t hidden,
                      uint32_t intermediate, const float *x, uint32_t n, float swiglu_limit,
                      const float *route_weights, float *y, int threads);
/* DeepSeek-V4 DeepExpert::forward_with_mx_input{,_batch} (src/models/deepseek_v4/runtime.rs:
 * 3081-3155) over n tokens [n, H]: MX weights read x quantized per 128 values (here) and round
 * their outputs to BF16; BF16 and F32 weights read x as it is. */
int urbo_dsv4_expert(int format, const urbo_matrix *gate_up_down, uint32_t hidden,
                     uint32_t intermediate, const float *x, uint32_t n, float swiglu_limit,
                     const float *route_weights, float *y, int threads);
/* GatedMlp::forward (src/model/mlp.rs:90-99) over n tokens [n, H] -> [n, H]. */
int urbo_gated_mlp(int format, const urbo_matrix *gate_up_down, uint32_t hidden,
                   uint32_t intermediate, const float *x, uint32_t n, float *y, int threads);
/* Qwen38Expert::forward_projections_batch with BF16 weights (src/models/qwen3_8/expert.rs:209-312). */
int urbo_qwen_expert(const urbo_matrix *gate_up_down, uint32_t hidden, uint32_t intermediate,
                     const float *x, uint32_t n, float *y, int threads);

/* Forward T tokens [T, H] -> y [T, H]; routes per token in ranking order (ids, weights [T, k]);
 * router logits [T, E] (may be NULL).  threads >= 1 selects the row-parallel pool width; every
 * row keeps its scalar reduction order so results are identical for any thread count.
 * Returns the first error in token order. */
int urbo_moe_forward(const urbo_layer *layer, const float *x, uint32_t tokens, float *y,
                     int32_t *ids, float *weights, float *logits, int threads);
/* The same with the tokens' ids [tokens] (hash routing reads the layer's tid2eid row of each;
 * an id >= hash_vocab -> URBO_SHAPE). */
int urbo_moe_forward_tokens(const urbo_layer *layer, const float *x, const uint32_t *token_ids,
                            uint32_t tokens, float *y, int32_t *ids, float *weights,
                            float *logits, int threads);

/* Bytes of one expert matrix for a format. */
size_t urbo_matrix_bytes(int format, size_t rows, size_t cols, size_t *scale_bytes);

#ifdef __cplusplus
}
#endif
#endif
