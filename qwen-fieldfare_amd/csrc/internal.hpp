// internal.hpp -- host-side context and the launchers each kernel file
// provides. Not part of the public ABI (include/qff/qff.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "qff/qff.h"

struct qff_prof_record {
    const char* name;
    hipEvent_t start, stop;
};

// Chunked DeltaNet prefill intermediates, one block per (chunk, value head),
// each array split into bf16 hi / lo halves.
struct qff_dn_bufs {
    uint16_t* kimg;   // per (chunk, key head): K hi, lo [64][128] in the state pass's LDS image order
    uint16_t* qop;    // per (chunk, key head): Q hi, lo, 16 MFMA operand blocks each
    uint16_t* top;    // per (chunk, value head): T = (I + A)^-1 hi, lo, 6 operand blocks each
    uint16_t* pop;    // per (chunk, value head): P hi, lo, 6 operand blocks each
    float* gates;     // per (chunk, value head): beta, beta e^G, e^{G_C - G}, e^G [4][64]
    float* bv;        // per (chunk, value head): beta V [64][128] in the state pass's lane order
};

struct qff_ctx {
    int device = 0;
    qff_ctx_cfg cfg{};
    // One device allocation, carved into the regions below.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Full-attention decode: split-KV partials per (sequence, kv head, chunk).
    float* gqa_m = nullptr;       // [gqa_slots(cfg) * 8]
    float* gqa_d = nullptr;       // same
    float* gqa_o = nullptr;       // [gqa_slots(cfg) * 8 * 256]
    // Full-attention prefill: normed, rotated q as bf16 [T][16][256].
    uint16_t* gqa_qb = nullptr;
    uint16_t* gqa_kv16 = nullptr;   // fp16 copy of a bf16 K cache for prefill: [max_ctx][2][256]
    uint16_t* gqa_vt = nullptr;     // transposed fp16 copy of the V cache for prefill: [2][max_ctx / 64][256][64]
    // Many-token Q4 products, per slice of q4_xs_tokens tokens: the fp16
    // activations x16 [q4_xs_tokens][<= 4096] and each token's output factor.
    uint16_t* q4_x16 = nullptr;
    float* q4_fm = nullptr;
    int q4_xs_tokens = 0;
    // Decode-batch Q4 products split over 512-column slices: per (row tile,
    // slice) the partial [16 tokens][64 rows], kQ4SkSlots of them.
    float* q4_sk_part = nullptr;
    // DeltaNet prefill: pre-norm outputs [T rounded up to 64][32][128] fp32
    // and chunk intermediates.
    float* pf_o = nullptr;
    qff_dn_bufs dn{};
    // DeltaNet decode: per (sequence, key head) arrival counters [max_batch][16],
    // zero between launches (the second arrival resets its counter).
    unsigned* dn_arrive = nullptr;
    // Work-queue counters of the persistent kernels, zero between launches
    // (each launch's last workgroup resets its pair); kSchedSlots pairs.
    unsigned* sched = nullptr;
    int num_cu = 0;
    // Kernel timing (qff_profile_enable): a pool of event pairs.
    bool prof = false;
    std::vector<qff_prof_record> prof_pool;
    int prof_n = 0;
};

namespace qff {

constexpr int kGqaMaxChunks = 512;     // split-KV chunks per (sequence, kv head), any call
constexpr int kGqaSeqChunks = 128;     // partial slots per (sequence, kv head) at max_batch
// (sequence, kv head, chunk) partial slots of the workspace: a call with a
// smaller batch spreads them over more chunks per sequence.
inline int gqa_slots(const qff_ctx_cfg& cfg) { return 2 * (cfg.max_batch > 4 ? cfg.max_batch : 4) * kGqaSeqChunks; }
constexpr int kSchedSlots = 8;         // work-queue counter pairs in the context
constexpr int kQ4SkSlots = 4096;       // (row tile, slice) partials of the split decode-batch Q4 product
constexpr int kSchedChunkLocal = 0;    // slot of the DeltaNet chunk-local pass

struct WorkspaceLayout {
    size_t gqa_m, gqa_d, gqa_o;
    size_t gqa_qb, gqa_kv16, gqa_vt, q4_x16, q4_fm, q4_sk_part, pf_o, dn_arrive, sched, kimg, qop, top, pop, gates, bv;
    size_t total;
};
WorkspaceLayout workspace_layout(const qff_ctx_cfg& cfg);
int q4_xs_tokens(const qff_ctx_cfg& cfg);

// Brackets the kernels launched in its scope with the context's profiling
// events when profiling is on; costs one branch otherwise.
struct ProfScope {
    qff_ctx* ctx;
    hipStream_t stream;
    int idx = -1;
    ProfScope(qff_ctx* c, hipStream_t s, const char* name) : ctx(c), stream(s) {
        if (c && c->prof && c->prof_n < static_cast<int>(c->prof_pool.size())) {
            idx = c->prof_n++;
            c->prof_pool[idx].name = name;
            (void)hipEventRecord(c->prof_pool[idx].start, s);
        }
    }
    ~ProfScope() {
        if (idx >= 0) (void)hipEventRecord(ctx->prof_pool[idx].stop, stream);
    }
};

// Inverse RoPE frequencies 1 / theta^(2i/64), i < 32, computed on the host
// in fp32 as the reference does (QwenQ4ActiveExpertStreamingRunner.swift
// :1090-1099) and passed to kernels by value; kernels form pos * f[i] and
// its cos / sin themselves, so no table travels per token.
struct RopeFreqs {
    float f[32];
};
RopeFreqs rope_freqs(float theta);

// Status of a full-attention parameter block: the norm weights present, a
// finite positive softmax scale, RoPE theta and eps, a cache type flag of 0
// or 1 (invalid argument otherwise); rotary_dim 64 is the only rotation
// built (unsupported otherwise).
inline int gqa_params_status(const qff_gqa_params* p) {
    if (!p || !p->q_norm_w || !p->k_norm_w) return QFF_ERR_INVALID_ARG;
    if (p->kv_f16 != 0 && p->kv_f16 != 1) return QFF_ERR_INVALID_ARG;
    if (!(p->scale > 0.0f) || !(p->scale < __builtin_huge_valf())) return QFF_ERR_INVALID_ARG;
    if (!(p->rope_theta > 0.0f) || !(p->rope_theta < __builtin_huge_valf()) || !(p->eps >= 0.0f))
        return QFF_ERR_INVALID_ARG;
    if (p->rotary_dim != 64) return QFF_ERR_UNSUPPORTED;
    return QFF_OK;
}

inline bool dtype_ok(qff_dtype d, bool allow_f16 = false) {
    return d == QFF_F32 || d == QFF_BF16 || (allow_f16 && d == QFF_F16);
}

// Launchers: validate nothing (qff_api.cpp does), enqueue on `stream`,
// return the HIP status of the launch.
hipError_t launch_deltanet_decode(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                  const void* qkv, const void* z, qff_dtype in_dtype,
                                  const float* a, const float* b, float* conv_state,
                                  float* ssm_state, void* out, qff_dtype out_dtype, int batch);
hipError_t launch_deltanet_prefill(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, const void* z, qff_dtype in_dtype,
                                   const float* a, const float* b, float* conv_state,
                                   float* ssm_state, void* out, qff_dtype out_dtype, int T);
hipError_t launch_deltanet_chunked(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, qff_dtype in_dtype, const float* a, const float* b,
                                   const float* conv_state, float* ssm_state, int T);
hipError_t launch_gqa_decode(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                             const void* q_gate, const void* k_new, const void* v_new,
                             qff_dtype in_dtype, void* k_cache, void* v_cache,
                             const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                             int max_ctx);
// Split-KV partial slots (m, d [slots][8], o [slots][8][256] fp32) and the
// chunk cap per (sequence, kv head) they allow for a call's batch.
struct GqaPartials {
    float* m;
    float* d;
    float* o;
    int cap;
    int num_cu;
};
// The decode kernels on caller-chosen partial slots; ctx only for profiling
// (may be null).
hipError_t launch_gqa_decode_into(qff_ctx* ctx, const GqaPartials& ws, hipStream_t stream,
                                  const qff_gqa_params* p, const void* q_gate, const void* k_new,
                                  const void* v_new, qff_dtype in_dtype, void* k_cache, void* v_cache,
                                  const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                                  int max_ctx);
hipError_t launch_gqa_prefill(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                              const void* q_gate, const void* k, const void* v, qff_dtype in_dtype,
                              void* k_cache, void* v_cache, int start_pos, void* out,
                              qff_dtype out_dtype, int T, int max_ctx);
hipError_t launch_q4_dequant(hipStream_t stream, const uint32_t* w, const void* scales,
                             const void* biases, qff_dtype sb_dtype, float* out, int rows, int cols);
hipError_t launch_q4_matmul(qff_ctx* ctx, hipStream_t stream, const uint32_t* w, const void* scales,
                            const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                            void* y, qff_dtype y_dtype, int rows, int cols, int batch);
// RMSNorm of each token of x folded into a Q4 product:
// xn = x * rsqrt(mean(x^2) + eps) * w; w == nullptr means no norm.
struct Q4Norm {
    const void* w = nullptr;
    int wbf16 = 0;
    float eps = 0.0f;
};
// Product over up to QFF_Q4_MAX_PARTS parts sharing x: one launch for decode
// batches, one group-sum pass plus one tiled launch over all parts for many
// tokens.
hipError_t launch_q4_parts(qff_ctx* ctx, hipStream_t stream, const qff_q4_part* parts, int nparts,
                           qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, const Q4Norm& norm, int cols,
                           int batch);
hipError_t launch_q8_dequant(hipStream_t stream, const uint32_t* w, const void* scales, const void* biases,
                             qff_dtype sb_dtype, float* out, int rows, int cols);
hipError_t launch_router_top8(qff_ctx* ctx, hipStream_t stream, const uint32_t* w, const void* scales,
                              const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                              float* logits, int32_t* indices, float* scores, int experts, int cols, int batch);
constexpr int kQ4GemmMinBatch = 33;   // batches at least this large take the tiled GEMM
hipError_t launch_kv_append(hipStream_t stream, const float* k, const float* v, void* k_cache,
                            void* v_cache, qff_dtype cache_dtype, int pos, int max_seq);
hipError_t launch_attention_gate(hipStream_t stream, const uint16_t* attn, const float* gate,
                                 float* out, int count);

}  // namespace qff
