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
