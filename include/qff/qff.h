/*
 * qff.h -- C ABI of the MI355X (gfx950) attention hot path of QwenFieldfare.
 *
 * Drop-in boundary: each entry point replaces one encoder block that the
 * reference's per-layer scheduler records into a Metal command buffer inside
 * QwenQ4ActiveExpertStreamingRunner.forwardToken. Paths below are relative
 * to Sources/QwenFieldfareCore/ of the reference.
 *
 * Conventions
 *   - The caller owns every tensor; all tensor arguments are device pointers
 *     (hipMalloc'd) unless stated otherwise. The context owns only scratch
 *     workspace, allocated once in qff_ctx_create.
 *   - Calls are asynchronous on the caller's stream (a hipStream_t; NULL is
 *     the default stream). No hot call allocates, frees or synchronises.
 *   - Every call returns QFF_OK (0) or a negative qff_status. Nothing aborts
 *     and nothing throws across this boundary. Shapes are validated on the
 *     host before any kernel is launched.
 *   - A context may be used from one stream at a time. Distinct contexts are
 *     independent and may run concurrently.
 *   - Element types are selected per argument with qff_dtype. bf16 and f16
 *     tensors are 16-bit IEEE/bfloat16 bit patterns.
 *   - Model geometry is fixed as in the reference kernels: DeltaNet 16 key
 *     heads / 32 value heads of dim 128 over 8192 conv channels; full
 *     attention 16 q heads / 2 kv heads of dim 256.
 */
#ifndef QFF_QFF_H
#define QFF_QFF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same underlying type as hipStream_t, without pulling in HIP headers. */
typedef struct ihipStream_t* qff_stream_t;

typedef enum qff_status {
    QFF_OK = 0,
    QFF_ERR_INVALID_ARG = -1,   /* null pointer, bad dtype, negative size      */
    QFF_ERR_UNSUPPORTED = -2,   /* shape outside what the kernels implement    */
    QFF_ERR_HIP = -3,           /* a HIP runtime call failed                   */
    QFF_ERR_WORKSPACE = -4,     /* request exceeds the context's configuration */
    QFF_ERR_OUT_OF_MEMORY = -5  /* qff_ctx_create could not allocate           */
} qff_status;

typedef enum qff_dtype {
    QFF_F32 = 0,
    QFF_BF16 = 1,
    QFF_F16 = 2
} qff_dtype;

typedef struct qff_ctx qff_ctx;

/* Workspace limits of a context. Zero fields take the defaults
 * (max_batch 32, max_ctx 65536, max_prefill_tokens 8192). */
typedef struct qff_ctx_cfg {
    int max_batch;           /* largest decode batch                        */
    int max_ctx;             /* largest KV context a decode call may attend,
                                and the largest start_pos + T of a prefill
                                (the workspace holds the copies of the cache
                                that the prefill attention reads: V
                                transposed, and the fp16 K of a bf16 cache;
                                2 KB per position)                          */
    int max_prefill_tokens;  /* largest T of a prefill call                 */
} qff_ctx_cfg;

/* ---------------------------------------------------------------- context */

/* Replaces MetalContext() + Attention(context:) set-up
 * (Infrastructure/Metal/MetalContext.swift:65-107,
 * Kernels/Attention/Attention.swift:63-127): binds `device`, checks it is a
 * gfx950 part, and allocates the workspace the configuration needs. */
int qff_ctx_create(qff_ctx** out, int device, const qff_ctx_cfg* cfg);
int qff_ctx_destroy(qff_ctx* ctx);

/* Bytes of device workspace a context with `cfg` holds. */
int qff_workspace_size(const qff_ctx_cfg* cfg, size_t* bytes);

const char* qff_status_string(int status);

/* ABI version, (major << 16) | minor. */
int qff_version(void);

/* Kernel timing, the counterpart of the reference's --subcomponent-profile
 * (QwenQ4ActiveExpertStreamingRunner.swift:1602-1912), which brackets each
 * kernel family with GPU timestamps. While enabled, every kernel a hot call
 * launches is bracketed by hipEvents on the call's stream (the first 4096
 * kernels after enabling or reading are kept; events are created by
 * qff_profile_enable, never by a hot call). qff_profile_read waits for the
 * recorded kernels, writes up to `capacity` (name, milliseconds) pairs in
 * launch order, sets *count to the number written and clears the record. */
int qff_profile_enable(qff_ctx* ctx, int enable);
int qff_profile_read(qff_ctx* ctx, const char** names, float* ms, int capacity,
                     int* count);

/* --------------------------------------------------------------- affine Q4 */

/* MLX affine Q4, group 64: element c of row r is nibble (c % 8) (lowest
 * first) of uint32 word w[r*(cols/8) + c/8]; value = nibble * scale + bias
 * with scale/bias [rows, cols/64] of sb_dtype (QFF_F16 or QFF_BF16).
 * Test hook: writes the dequantized fp32 matrix [rows, cols], bit-exact with
 * the closed form of Runtime/Generation/QwenQ4ActiveExpertStreamingRunner
 * .swift:899-922 (CPU) and Metal/LinearAttention/deltanet.metal:809-814. */
int qff_q4_dequant(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w,
                   const void* scales, const void* biases, qff_dtype sb_dtype,
                   float* out, int rows, int cols);

/* y[m, r] = sum_c W[r, c] * x[m, c] for m < batch, with W affine-Q4 as above.
 * x [batch, cols] of x_dtype (F32 or BF16), y [batch, rows] of y_dtype.
 * cols must be a multiple of 64. Replaces qwen_gemv_q4_affine_simd_f32
 * (deltanet.metal:1897-1919) and qwen_gemv_q4_affine (deltanet.metal:816-861)
 * as dispatched for the q/k/v and out projections
 * (QwenQ4ActiveExpertStreamingRunner.swift:1024-1032, 1051-1074, 1152-1160);
 * batch > 1 covers batched decode and prefill projections. Up to 32 tokens
 * the nibbles and x enter exactly (fp32 x as a bf16 hi + lo pair: fp32-class
 * products); from 33 tokens the product runs on fp16 operands, W rounded
 * once to fp16 and x to fp16 after a per-token power-of-two shift (relative
 * error ~3e-4 of the exact product; x of any fp32 magnitude, dequantized
 * weights of magnitude 2^-22 .. 255). */
int qff_q4_matmul(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w,
                  const void* scales, const void* biases, qff_dtype sb_dtype,
                  const void* x, qff_dtype x_dtype, void* y, qff_dtype y_dtype,
                  int rows, int cols, int batch);

/* One part of a grouped product: W [rows, cols] affine-Q4 as above (its own
 * scales/biases, sb_dtype of the call) and its output y [batch, rows] of
 * y_dtype. residual, when not NULL, is [batch, rows] of y_dtype and the part
 * writes y = residual + x W^T: the out-projection's residual add
 * (qwen_residual_add_f32, deltanet.metal:454-463, dispatched after the out
 * projection at QwenQ4ActiveExpertStreamingRunner.swift:1034-1040 and
 * 1162-1166) folded into the product's store. residual may be y itself;
 * any other overlap of residual and y is undefined. */
typedef struct qff_q4_part {
    const uint32_t* w;
    const void* scales;
    const void* biases;
    int rows;
    void* y;
    qff_dtype y_dtype;
    const void* residual;
} qff_q4_part;

#define QFF_Q4_MAX_PARTS 8

/* y_p = x W_p^T for every part p (1 <= nparts <= QFF_Q4_MAX_PARTS), all
 * sharing x [batch, cols]: one launch over the parts' rows laid end to end
 * for decode batches. Replaces the fused four-part DeltaNet in-projection
 * qwen_fused_linear_attn_in_proj_q4_simd_f32 (deltanet.metal:1921-1983:
 * qkv 8192, z 4096, b 32, a 32 rows, separate weights and outputs, one
 * global row index), dispatched at QwenQ4ActiveExpertStreamingRunner
 * .swift:982-997, and serves the q/k/v projections of a full-attention
 * layer (.swift:1056-1074, three dispatches there) the same way. */
int qff_q4_matmul_parts(qff_ctx* ctx, qff_stream_t stream, const qff_q4_part* parts,
                        int nparts, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                        int cols, int batch);

/* The layer's decode/prefill front-end: RMSNorm of each token of x, then
 * the grouped product of qff_q4_matmul_parts on the normalised rows,
 *   xn[m, c] = x[m, c] * rsqrt(mean_c x[m, c]^2 + eps) * norm_w[c],
 *   y_p = xn W_p^T (+ residual_p),
 * without writing a normalised copy of x: in one pass over the weights up
 * to 16 tokens (two for 17-32, one per 16-token half; many-token batches
 * fold the norm into the pass that forms their fp16 activations).
 * Replaces qwen_rmsnorm_f32 (deltanet.metal:18-53, weight used as is, mean
 * over the row) followed by the in-projections, as dispatched at
 * QwenQ4ActiveExpertStreamingRunner.swift:973-997 (DeltaNet layer) and
 * 1043-1074 (full-attention layer). norm_w [cols] of norm_dtype (F32 or
 * BF16). The product takes x[m, c] * norm_w[c] (exact as a bf16 hi + lo
 * pair up to 32 tokens, as fp16 from 33 as in qff_q4_matmul) and applies the
 * per-token inverse RMS to the fp32 row sums. */
int qff_q4_norm_matmul_parts(qff_ctx* ctx, qff_stream_t stream, const qff_q4_part* parts,
                             int nparts, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                             const void* norm_w, qff_dtype norm_dtype, float eps,
                             int cols, int batch);

/* ------------------------------------------------------------- MoE router */

/* MLX affine Q8, group 64: element c of row r is byte c % 4 (lowest first)
 * of uint32 word w[r*(cols/4) + c/4], i.e. byte c of the row; value = byte *
 * scale + bias with scale/bias [rows, cols/64] of sb_dtype (QFF_BF16 or
 * QFF_F16). Test hook: writes the dequantized fp32 matrix [rows, cols],
 * bit-exact with the closed form of deltanet.metal:863-900 (byte * scale is
 * exact in fp32, so each value is one rounding). */
int qff_q8_dequant(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w,
                   const void* scales, const void* biases, qff_dtype sb_dtype,
                   float* out, int rows, int cols);

/* The MoE router of `batch` tokens: logits[m, e] = sum_c W[e, c] x[m, c]
 * with W [experts, cols] affine-Q8 as above, accumulated in fp32 in the
 * factored form scale * sum(q x) + bias * sum(x) per group; then per token
 * the eight largest logits in descending order (equal logits: lower expert
 * index first) into indices [batch, 8], and their routing weights into
 * scores [batch, 8]: softmax over all `experts` logits shifted by the
 * largest, the eight probabilities divided by their sum. x [batch, cols] of
 * x_dtype (F32 or BF16), logits [batch, experts] fp32 (written). Replaces
 * qwen_router_q8_logits_simd_f32 + qwen_router_top8_logits_f32
 * (deltanet.metal:2229-2329) as dispatched at
 * QwenQ4ActiveExpertStreamingRunner.swift:1177-1190 (experts 256, cols
 * 2048). Requires 8 <= experts <= 256 and cols a multiple of 64, <= 4096. */
int qff_router_top8(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w,
                    const void* scales, const void* biases, qff_dtype sb_dtype,
                    const void* x, qff_dtype x_dtype, float* logits,
                    int32_t* indices, float* scores, int experts, int cols, int batch);

/* ---------------------------------------------------------------- DeltaNet */

/* Per-layer constants of a Gated DeltaNet layer (fp32, device pointers),
 * decoded from the checkpoint as QwenQ4ActiveExpertStreamingRunner
 * .swift:561-572 does. */
typedef struct qff_deltanet_params {
    const float* a_log;    /* [32]                                     */
    const float* dt_bias;  /* [32]                                     */
    const float* conv_w;   /* [8192][4], tap 3 multiplies the newest   */
    const float* norm_w;   /* [128], gated RMSNorm weight              */
    float eps;             /* gated RMSNorm epsilon (1e-6)             */
} qff_deltanet_params;

/* One decode step of `batch` independent sequences through the DeltaNet
 * layer core: causal conv1d (k=4) + SiLU over the 8192 qkv channels, L2
 * normalisation of q (then / sqrt(128)) and k per key head, the gated delta
 * rule S = g*S; S += beta*(v - S k) k^T; o = S q on the fp32 128x128 state of
 * each of the 32 value heads (value head h reads key head h/2), and the gated
 * RMSNorm o * rsqrt(mean(o^2) + eps) * norm_w * silu(z).
 * Replaces the encoder blocks qwen_conv1d_f32 + qwen_fused_deltanet_step_f32
 * (QwenQ4ActiveExpertStreamingRunner.swift:1001-1022; kernels
 * deltanet.metal:112-138, 250-356).
 *   qkv        [batch, 8192] pre-conv projection (F32 or BF16)
 *   z          [batch, 4096] gate projection (F32 or BF16)
 *   a, b       [batch, 32] fp32 (g from a, beta = sigmoid(b))
 *   conv_state [batch, 8192, 4] fp32, updated in place (slot 3 newest)
 *   ssm_state  [batch, 32, 128, 128] fp32, row = v index, updated in place
 *   out        [batch, 4096] of out_dtype (F32 or BF16) */
int qff_deltanet_decode(qff_ctx* ctx, qff_stream_t stream,
                        const qff_deltanet_params* p, const void* qkv,
                        const void* z, qff_dtype in_dtype, const float* a,
                        const float* b, float* conv_state, float* ssm_state,
                        void* out, qff_dtype out_dtype, int batch);

/* T consecutive tokens of one sequence through the same layer core, starting
 * from conv_state / ssm_state (updated in place to the state after token
 * T-1). The reference feeds prompts token by token through the decode path
 * (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561); this computes the same
 * result with the chunked WY form, chunk = 64 (the only value accepted).
 *   qkv [T, 8192], z [T, 4096] (in_dtype), a, b [T, 32] fp32,
 *   out [T, 4096] of out_dtype. */
int qff_deltanet_prefill(qff_ctx* ctx, qff_stream_t stream,
                         const qff_deltanet_params* p, const void* qkv,
                         const void* z, qff_dtype in_dtype, const float* a,
                         const float* b, float* conv_state, float* ssm_state,
                         void* out, qff_dtype out_dtype, int T, int chunk);

/* ---------------------------------------------------------- full attention */

typedef struct qff_gqa_params {
    const float* q_norm_w;  /* [256] per-head q RMSNorm weight              */
    const float* k_norm_w;  /* [256] per-head k RMSNorm weight              */
    float rope_theta;       /* 1e7                                          */
    int rotary_dim;         /* 64: rotate-half on pairs (i, i+32), i < 32   */
    float scale;            /* softmax scale, 1/16                          */
    float eps;              /* head RMSNorm epsilon (1e-6)                  */
    int kv_f16;             /* KV cache element type: 0 bf16 (the default a
                               zeroed struct gets), 1 fp16 (the runner's
                               Float16 caches, Runner:731-732)             */
} qff_gqa_params;

/* One decode token for each of `batch` sequences: split the per-head
 * interleaved q|gate projection, RMSNorm q and k per head, partial RoPE at
 * the sequence's position, append k and v at that position of the
 * token-major cache (bf16, or fp16 with p->kv_f16; the reference's cache is
 * fp16, written by qwen_update_kv_cache_f16), attend over positions 0..pos
 * with 16 q heads on 2 kv
 * heads (q head h uses kv head h/8), and gate: out = attn * sigmoid(gate).
 * Replaces QwenQ4ActiveExpertStreamingRunner.swift:1076-1150, i.e.
 * qwen_split_q_gate_f32, qwen_head_rmsnorm_f32, host RoPE tables +
 * qwen_rope_partial_f32, qwen_update_kv_cache_f16, qwen_f32_to_f16,
 * Attention.encodeFull and qwen_apply_attention_gate_f16_f32
 * (deltanet.metal:599-708; attention.metal:134-377; Attention.swift:195-299).
 *   q_gate    [batch, 16, 512]: q = [..., :256], gate = [..., 256:] (in_dtype)
 *   k_new     [batch, 2, 256], v_new [batch, 2, 256] (in_dtype)
 *   k_cache, v_cache [batch, max_ctx, 2, 256] bf16 (fp16 with p->kv_f16),
 *             updated at pos
 *   positions [batch] int32 device array, 0 <= pos < max_ctx
 *   out       [batch, 16, 256] of out_dtype (F32 or BF16) */
int qff_gqa_decode(qff_ctx* ctx, qff_stream_t stream, const qff_gqa_params* p,
                   const void* q_gate, const void* k_new, const void* v_new,
                   qff_dtype in_dtype, void* k_cache, void* v_cache,
                   const int32_t* positions, void* out, qff_dtype out_dtype,
                   int batch, int max_ctx);

/* qff_gqa_decode without a context, for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. No counterpart in the reference (its split-KV scratch is
 * allocated with the Attention object, Kernels/Attention/Attention.swift
 * :117-126). Same arguments, kernels and results as qff_gqa_decode on the
 * current device; the split-KV partials live in a fixed device array of the
 * library (4096 slots, 33.8 MB, one per GPU, held until the process ends),
 * so batch is limited to 64 (QFF_ERR_WORKSPACE above). The first call on a
 * device looks up that array's address (make it before a capture that must
 * not see runtime queries; a failed look-up returns its status and is tried
 * again by the next call); no call allocates or frees. Calls that overlap on
 * one GPU (other streams or threads) race on the array. */
int qff_gqa_decode_static(qff_stream_t stream, const qff_gqa_params* p, const void* q_gate,
                          const void* k_new, const void* v_new, qff_dtype in_dtype, void* k_cache,
                          void* v_cache, const int32_t* positions, void* out, qff_dtype out_dtype,
                          int batch, int max_ctx);

/* T consecutive tokens of one sequence at positions start_pos .. start_pos+T-1
 * (causal): the same per-token steps as qff_gqa_decode, with all T keys and
 * values appended to the cache. The reference runs prompts token by token
 * through the decode path (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561).
 *   q_gate [T, 16, 512], k, v [T, 2, 256] (in_dtype);
 *   k_cache, v_cache [max_ctx, 2, 256] bf16 (fp16 with p->kv_f16);
 *   out [T, 16, 256] (out_dtype).
 * QFF_ERR_INVALID_ARG when start_pos + T > max_ctx; QFF_ERR_WORKSPACE when T
 * exceeds the context's max_prefill_tokens or start_pos + T exceeds the
 * context's max_ctx (the attention reads copies of the cache kept in the
 * workspace: V transposed, and the fp16 K of a bf16 cache). */
int qff_gqa_prefill(qff_ctx* ctx, qff_stream_t stream, const qff_gqa_params* p,
                    const void* q_gate, const void* k, const void* v,
                    qff_dtype in_dtype, void* k_cache, void* v_cache,
                    int start_pos, void* out, qff_dtype out_dtype, int T,
                    int max_ctx);

/* Raw KV append, token-major: cache[(pos*2 + kv_head)*256 + d] = k[kv_head*256
 * + d] rounded to cache_dtype (QFF_BF16 or QFF_F16), same for v. No-op when
 * pos >= max_seq. Replaces qwen_update_kv_cache_f16 (deltanet.metal:670-689)
 * for callers that append without the fused decode path.
 *   k, v [2, 256] fp32; caches [max_seq, 2, 256]. */
int qff_kv_append(qff_ctx* ctx, qff_stream_t stream, const float* k,
                  const float* v, void* k_cache, void* v_cache,
                  qff_dtype cache_dtype, int pos, int max_seq);

/* out[i] = float(attn[i]) * sigmoid(gate[i]) for an f16 attention output.
 * Replaces qwen_apply_attention_gate_f16_f32 (deltanet.metal:700-708). */
int qff_attention_gate(qff_ctx* ctx, qff_stream_t stream, const uint16_t* attn_f16,
                       const float* gate, float* out, int count);

#ifdef __cplusplus
}
#endif

#endif /* QFF_QFF_H */
