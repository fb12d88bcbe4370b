/*
 * cpu_baseline.c -- the reference's CPU algorithms as a timed baseline.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by bench.py's cpu_baseline leg (and by
 * tests/ to check it against the oracle), never by the product.
 *
 * It instantiates the oracle's fp32 functions (qff_oracle_impl.h, the
 * reference's loop order) and adds two drivers that spread independent work
 * over OpenMP threads without changing any arithmetic:
 *
 *   qffb_deltanet_prefill  the DeltaNet layer core over T tokens of one
 *       sequence, as the reference's QwenLinearAttentionMath applies it token
 *       by token (Kernels/LinearAttention/QwenDeltaNetKernel.swift:39-151,
 *       fed per token at Runtime/Generation/QwenQ4ActiveExpertStreamingRunner
 *       .swift:1545-1561). The conv1d of each channel runs over all tokens
 *       (channels in parallel), L2 norms per (token, head) in parallel, then
 *       each value head's recurrence over the T tokens (heads in parallel:
 *       a head's state depends on no other head), then the gated RMSNorm per
 *       (token, head). Every value is computed by the same operations in the
 *       same order as qffo_deltanet_sequence_f32, so the outputs are equal
 *       bit for bit (checked in tests/test_oracle_deltanet.py).
 *   qffb_attention_decode  split-KV decode attention of a batch of
 *       sequences (Metal/Attention/attention.metal:134-224, 342-377 with the
 *       geometry of Kernels/Attention/Attention.swift:129-157), (sequence,
 *       q head) pairs in parallel.
 *   qffb_gqa_prefill_tokens  the full-attention layer core over tokens
 *       t0 .. t1-1 of one sequence the way the reference prefills, token by
 *       token through its decode path (Runtime/Generation/
 *       QwenQ4ActiveExpertStreamingRunner.swift:1545-1561, full-attention
 *       branch :1041-1150): the affine-Q4 q|gate, k and v products of the
 *       token (rows in parallel), head RMSNorm + RoPE of k appended to the
 *       cache, head RMSNorm + RoPE of q, split-KV attention over positions
 *       0..t (q heads in parallel), sigmoid gate.
 *   qffb_dn_layer_decode / qffb_gqa_layer_decode  one decoder layer's
 *       attention block for a batch of decode tokens in the reference's
 *       encoder order (Runner:972-1040 and :1041-1167): input RMSNorm, the
 *       Q4 in-projection, the layer core, the Q4 out-projection added into
 *       the residual stream. Sequences run one after the other, each with
 *       its products' rows, its DeltaNet channels and heads, or its q heads
 *       spread over the threads.
 * Caches are fp32 here (the reference keeps fp16, a rounding that does not
 * change the work), and q is not rounded to fp16 before attention.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define R float
#define SFX(name) name##_f32
#define EXP expf
#define LOG1P log1pf
#define SQRT sqrtf
#define FMA fmaf
#define COS cosf
#define SIN sinf
#define POW powf
#include "qff_oracle_impl.h"
#undef R
#undef SFX

static void set_threads(int threads) {
#ifdef _OPENMP
    omp_set_num_threads(threads > 0 ? threads : 1);
#else
    (void)threads;
#endif
}

int qffb_openmp(void) {
#ifdef _OPENMP
    return 1;
#else
    return 0;
#endif
}

/* qkv [T][8192] pre-conv, z [T][4096], a, b [T][32]; conv_state [8192][4]
 * and ssm [32][128][128] updated in place; out [T][4096]; work [T][12288]
 * floats of scratch (conv outputs, then q, k per value head... see below). */
void qffb_deltanet_prefill(int T, const float* qkv, const float* z, const float* a,
                           const float* b, const float* a_log, const float* dt_bias,
                           const float* conv_w, const float* norm_w, float eps,
                           float* conv_state, float* ssm, float* out, float* conv_out,
                           int threads) {
    set_threads(threads);
    const float q_scale = 1.0f / sqrtf(128.0f);
    /* conv1d + SiLU of every channel over the tokens (LA:39-59): conv_out
     * [T][8192], then the L2 norms in place (LA:61-71, q scaled at LA:210) */
    #pragma omp parallel for schedule(static)
    for (int c = 0; c < 8192; ++c) {
        float* s = conv_state + (size_t)c * 4;
        const float* w = conv_w + (size_t)c * 4;
        for (int t = 0; t < T; ++t) {
            s[0] = s[1]; s[1] = s[2]; s[2] = s[3]; s[3] = qkv[(size_t)t * 8192 + c];
            float acc = s[0] * w[0] + s[1] * w[1] + s[2] * w[2] + s[3] * w[3];
            conv_out[(size_t)t * 8192 + c] = silu__f32(acc);
        }
    }
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < T * 32; ++i) {
        const int t = i / 32, kh = i % 32;   /* kh < 16: q head, else k head */
        float* x = conv_out + (size_t)t * 8192 + (size_t)kh * 128;
        float tmp[128];
        qffo_l2norm_f32(x, 128, 1e-6f, tmp);
        for (int e = 0; e < 128; ++e) x[e] = kh < 16 ? tmp[e] * q_scale : tmp[e];
    }
    /* each value head's recurrence over the tokens (LA:73-125) */
    #pragma omp parallel for schedule(dynamic, 1)
    for (int h = 0; h < 32; ++h) {
        float core[128];
        for (int t = 0; t < T; ++t) {
            const float* row = conv_out + (size_t)t * 8192;
            qffo_deltanet_head_step_f32(row + (h / 2) * 128, row + 2048 + (h / 2) * 128,
                                        row + 4096 + h * 128, a[(size_t)t * 32 + h], b[(size_t)t * 32 + h],
                                        a_log[h], dt_bias[h], ssm + (size_t)h * 128 * 128, core);
            /* gated RMSNorm of this head's output (LA:127-151) */
            float ss = 0;
            for (int r = 0; r < 128; ++r) ss += core[r] * core[r];
            float inv = 1.0f / sqrtf(ss / 128.0f + eps);
            const float* zz = z + (size_t)t * 4096 + h * 128;
            for (int r = 0; r < 128; ++r)
                out[(size_t)t * 4096 + h * 128 + r] = core[r] * inv * norm_w[r] * silu__f32(zz[r]);
        }
    }
}

/* B sequences: q [B][16][256] (already normed, rotated and rounded as the
 * caller wants), K, V [B][max_ctx][2][256] fp32, lengths [B] -> out
 * [B][16][256]. */
void qffb_attention_decode(int B, const float* q, const float* K, const float* V,
                           const int32_t* lengths, int max_ctx, float scale, float* out,
                           int threads) {
    set_threads(threads);
    #pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < B * 16; ++i) {
        const int s = i / 16, h = i % 16;
        const size_t base = (size_t)s * max_ctx * 512;
        qffo_attention_decode_head_f32(q + (size_t)i * 256, K + base, V + base, lengths[s], 2, h / 8, 256,
                                       scale, 0, out + (size_t)i * 256);
    }
}

/* One token's affine-Q4 product over `rows` rows (blocks of 64 rows over
 * the threads): the oracle's factored order (deltanet.metal:1838-1895). */
static void q4_rows(const uint32_t* w, const float* sc, const float* bi, const float* x, int rows, int cols,
                    float* y) {
    const int blocks = (rows + 63) / 64;
    #pragma omp parallel for schedule(static)
    for (int blk = 0; blk < blocks; ++blk) {
        const int r0 = blk * 64, n = rows - r0 < 64 ? rows - r0 : 64;
        qffo_q4_matvec_f32(w + (size_t)r0 * (cols / 8), sc + (size_t)r0 * (cols / 64),
                           bi + (size_t)r0 * (cols / 64), x, n, cols, y + r0);
    }
}

/* x [T][2048]; the three projections stacked as one weight of 9216 rows
 * (q|gate 8192, k 512, v 512: w [9216][256] u32, scales / biases
 * [9216][32] fp32); K, V [max_ctx][2][256] fp32 caches (positions < t0
 * filled by the caller); out [T][16][256]. */
void qffb_gqa_prefill_tokens(int t0, int t1, const float* x, const uint32_t* w, const float* sc, const float* bi,
                             const float* q_norm_w, const float* k_norm_w, float theta, float scale, float eps,
                             float* K, float* V, float* out, int threads) {
    set_threads(threads);
    float* y = (float*)malloc(sizeof(float) * 9216);
    for (int t = t0; t < t1; ++t) {
        q4_rows(w, sc, bi, x + (size_t)t * 2048, 9216, 2048, y);
        float cs[64], sn[64], q[16 * 256];
        qffo_rope_tables_f32(t, theta, 64, cs, sn);
        float* kt = K + (size_t)t * 512;
        memcpy(kt, y + 8192, sizeof(float) * 512);
        memcpy(V + (size_t)t * 512, y + 8704, sizeof(float) * 512);
        qffo_head_rmsnorm_f32(kt, k_norm_w, 2, 256, eps);
        qffo_rope_partial_f32(kt, cs, sn, 2, 256, 64);
        for (int h = 0; h < 16; ++h) memcpy(q + h * 256, y + h * 512, sizeof(float) * 256);
        qffo_head_rmsnorm_f32(q, q_norm_w, 16, 256, eps);
        qffo_rope_partial_f32(q, cs, sn, 16, 256, 64);
        #pragma omp parallel for schedule(dynamic, 1)
        for (int h = 0; h < 16; ++h) {
            float* o = out + ((size_t)t * 16 + h) * 256;
            qffo_attention_decode_head_f32(q + h * 256, K, V, t + 1, 2, h / 8, 256, scale, 0, o);
            for (int i = 0; i < 256; ++i) o[i] *= sigmoid__f32(y[h * 512 + 256 + i]);
        }
    }
    free(y);
}

/* B decode tokens through one Gated DeltaNet layer's attention block:
 * x [B][2048] updated in place; in-projection stacked as 12352 rows (qkv
 * 8192, z 4096, b 32, a 32) of 2048 columns, out-projection 2048 rows of
 * 4096 columns; conv_state [B][8192][4], ssm [B][32][128][128]. */
void qffb_dn_layer_decode(int B, float* x, const float* in_norm_w, const uint32_t* w_in, const float* s_in,
                          const float* b_in, const uint32_t* w_out, const float* s_out, const float* b_out,
                          const float* a_log, const float* dt_bias, const float* conv_w, const float* norm_w,
                          float eps, float* conv_state, float* ssm, int threads) {
    set_threads(threads);
    float xn[2048], y[12352], core[4096], r[2048], conv_out[8192];
    for (int s = 0; s < B; ++s) {
        float* xs = x + (size_t)s * 2048;
        qffo_rmsnorm_f32(xs, in_norm_w, 2048, eps, 0, xn);
        q4_rows(w_in, s_in, b_in, xn, 12352, 2048, y);
        qffb_deltanet_prefill(1, y, y + 8192, y + 12320, y + 12288, a_log, dt_bias, conv_w, norm_w, eps,
                              conv_state + (size_t)s * 8192 * 4, ssm + (size_t)s * 32 * 128 * 128, core,
                              conv_out, threads);
        q4_rows(w_out, s_out, b_out, core, 2048, 4096, r);
        for (int i = 0; i < 2048; ++i) xs[i] += r[i];
    }
}

/* B decode tokens through one full-attention layer's attention block:
 * in-projection stacked as 9216 rows (q|gate 8192, k 512, v 512),
 * out-projection 2048 x 4096; K, V [B][max_ctx][2][256] fp32, token b at
 * positions[b]. */
void qffb_gqa_layer_decode(int B, float* x, const float* in_norm_w, const uint32_t* w_in, const float* s_in,
                           const float* b_in, const uint32_t* w_out, const float* s_out, const float* b_out,
                           const float* q_norm_w, const float* k_norm_w, float theta, float scale, float eps,
                           float* K, float* V, const int32_t* positions, int max_ctx, int threads) {
    set_threads(threads);
    float xn[2048], y[9216], att[4096], r[2048], q[4096], cs[64], sn[64];
    for (int s = 0; s < B; ++s) {
        float* xs = x + (size_t)s * 2048;
        const int pos = positions[s];
        float* Ks = K + (size_t)s * max_ctx * 512;
        float* Vs = V + (size_t)s * max_ctx * 512;
        qffo_rmsnorm_f32(xs, in_norm_w, 2048, eps, 0, xn);
        q4_rows(w_in, s_in, b_in, xn, 9216, 2048, y);
        qffo_rope_tables_f32(pos, theta, 64, cs, sn);
        float* kt = Ks + (size_t)pos * 512;
        memcpy(kt, y + 8192, sizeof(float) * 512);
        memcpy(Vs + (size_t)pos * 512, y + 8704, sizeof(float) * 512);
        qffo_head_rmsnorm_f32(kt, k_norm_w, 2, 256, eps);
        qffo_rope_partial_f32(kt, cs, sn, 2, 256, 64);
        for (int h = 0; h < 16; ++h) memcpy(q + h * 256, y + h * 512, sizeof(float) * 256);
        qffo_head_rmsnorm_f32(q, q_norm_w, 16, 256, eps);
        qffo_rope_partial_f32(q, cs, sn, 16, 256, 64);
        #pragma omp parallel for schedule(dynamic, 1)
        for (int h = 0; h < 16; ++h) {
            float* o = att + h * 256;
            qffo_attention_decode_head_f32(q + h * 256, Ks, Vs, pos + 1, 2, h / 8, 256, scale, 0, o);
            for (int i = 0; i < 256; ++i) o[i] *= sigmoid__f32(y[h * 512 + 256 + i]);
        }
        q4_rows(w_out, s_out, b_out, att, 2048, 4096, r);
        for (int i = 0; i < 2048; ++i) xs[i] += r[i];
    }
}
