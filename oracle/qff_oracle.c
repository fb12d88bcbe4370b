/*
 * qff_oracle.c -- CPU restatement of QwenFieldfare's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. Nothing in the product library links or calls it.
 *
 * The reference (Swift + Metal, Apple-only) cannot be compiled or run on
 * Linux, so this file restates its arithmetic from source, in the same loop
 * order, in plain C. Build flags keep that order: -O2 -ffp-contract=off and
 * no fast-math, so a*b+c is never fused unless the reference wrote fma().
 *
 * What pins each function (tests/test_oracle_*.py): the reference's own
 * known-answer tests, closed forms, invariants and brute force on tiny
 * inputs. The header of each function names the reference lines it follows.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp32 instantiation: the reference's own precision and loop order.   */
#define R float
#define SFX(n) n##_f32
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
#undef EXP
#undef LOG1P
#undef SQRT
#undef FMA
#undef COS
#undef SIN
#undef POW

/* fp64 instantiation: same algorithm, used as the accuracy yardstick. */
#define R double
#define SFX(n) n##_f64
#define EXP exp
#define LOG1P log1p
#define SQRT sqrt
#define FMA fma
#define COS cos
#define SIN sin
#define POW pow
#include "qff_oracle_impl.h"

/* ------------------------------------------------------------------ */
/* Storage conversions (IEEE 754 binary16 / bfloat16, round to nearest  */
/* even). Metal's half(x) and the build's bf16 stores both round RNE.   */

uint16_t qffo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))  /* NaN */
        return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float qffo_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t qffo_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x007fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);           /* overflow -> inf */
    if (e <= 0) {                                              /* subnormal / zero */
        if (e < -10) return (uint16_t)sign;
        man |= 0x00800000u;
        int shift = 14 - e;                                    /* 14..24 */
        uint32_t half_man = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_man & 1u))) half_man++;
        return (uint16_t)(sign | half_man);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* carries into exp ok */
    return (uint16_t)h;
}

float qffo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {                                               /* subnormal */
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400u));
            man &= 0x3ffu;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1fu) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* dtype codes shared with include/qff/qff.h: 0 f32, 1 bf16, 2 f16 */
static float load_elem(const void* p, int dtype, size_t i) {
    if (dtype == 1) return qffo_bf16_to_f32(((const uint16_t*)p)[i]);
    if (dtype == 2) return qffo_f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static void store_elem(void* p, int dtype, size_t i, float v) {
    if (dtype == 1) ((uint16_t*)p)[i] = qffo_f32_to_bf16(v);
    else if (dtype == 2) ((uint16_t*)p)[i] = qffo_f32_to_f16(v);
    else ((float*)p)[i] = v;
}

float qffo_round_to(float v, int dtype) {
    if (dtype == 1) return qffo_bf16_to_f32(qffo_f32_to_bf16(v));
    if (dtype == 2) return qffo_f16_to_f32(qffo_f32_to_f16(v));
    return v;
}

/* ------------------------------------------------------------------ */
/* Q4 unpack + dequant, closed form: RUN:899-922 (CPU embedding) and    */
/* DN:809-814 (bf16 scales). Element c of row r lives in word           */
/* w[r*(cols/8) + c/8], nibble (c % 8), lowest nibble first;            */
/* W = nibble * scale + bias in fp32. nibble*scale is exact (<= 15      */
/* significant bits), so the single rounding of "+ bias" makes the      */
/* result identical with or without FMA contraction.                    */
void qffo_q4_dequant(const uint32_t* w, const void* scales, const void* biases,
                     int sb_dtype, int rows, int cols, float* out) {
    int groups = cols / 64;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            uint32_t word = w[(size_t)r * (cols / 8) + c / 8];
            float nib = (float)((word >> (4 * (c % 8))) & 0xFu);
            float s = load_elem(scales, sb_dtype, (size_t)r * groups + c / 64);
            float b = load_elem(biases, sb_dtype, (size_t)r * groups + c / 64);
            out[(size_t)r * cols + c] = nib * s + b;
        }
}

/* ------------------------------------------------------------------ */
/* MLX affine Q8, group 64 (deltanet.metal:863-900, 2229-2259): element  */
/* c of row r is byte c of the row (byte c % 4 of little-endian word     */
/* c / 4); value = byte * scale + bias. byte (8 bits) x scale (<= 11     */
/* significant bits) is exact in fp32, so the value is one rounding.     */
void qffo_q8_dequant(const uint32_t* w, const void* scales, const void* biases,
                     int sb_dtype, int rows, int cols, float* out) {
    int groups = cols / 64;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            uint32_t word = w[(size_t)r * (cols / 4) + c / 4];
            float q = (float)((word >> (8 * (c % 4))) & 0xFFu);
            float s = load_elem(scales, sb_dtype, (size_t)r * groups + c / 64);
            float b = load_elem(biases, sb_dtype, (size_t)r * groups + c / 64);
            out[(size_t)r * cols + c] = q * s + b;
        }
}

/* Router logits, the factored order of qwen_q8_row_simd_f32            */
/* (deltanet.metal:2229-2259) without its cross-lane split: per group    */
/* dot = sum q x, sum = sum x, acc = fma(scale, dot, acc) then           */
/* acc = fma(bias, sum, acc). x [cols] f32 -> logits [rows].            */
void qffo_router_logits(const uint32_t* w, const void* scales, const void* biases, int sb_dtype,
                        const float* x, int rows, int cols, float* logits) {
    int groups = cols / 64;
    for (int r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (int g = 0; g < groups; ++g) {
            float s = load_elem(scales, sb_dtype, (size_t)r * groups + g);
            float b = load_elem(biases, sb_dtype, (size_t)r * groups + g);
            float dot = 0.0f, sum = 0.0f;
            for (int i = 0; i < 64; ++i) {
                int c = 64 * g + i;
                uint32_t word = w[(size_t)r * (cols / 4) + c / 4];
                float xv = x[c];
                dot = fmaf((float)((word >> (8 * (c % 4))) & 0xFFu), xv, dot);
                sum += xv;
            }
            acc = fmaf(s, dot, acc);
            acc = fmaf(b, sum, acc);
        }
        logits[r] = acc;
    }
}

/* Top-8 routing, qwen_router_top8_logits_f32 (deltanet.metal:2283-2329): */
/* insertion of each logit into a descending list of eight (a later     */
/* logit enters only if strictly larger than the eighth, and moves up   */
/* only past strictly smaller ones, so ties keep the lower index first), */
/* softmax over all `n` logits with the top value as the shift, and the */
/* eight probabilities renormalised to sum to one.                       */
void qffo_router_top8(const float* logits, int n, int32_t* idx, float* scores) {
    int top_idx[8];
    float top_val[8];
    for (int k = 0; k < 8; ++k) {
        top_idx[k] = 0;
        top_val[k] = -INFINITY;
    }
    for (int i = 0; i < n; ++i) {
        float v = logits[i];
        if (v > top_val[7]) {
            top_val[7] = v;
            top_idx[7] = i;
            for (int k = 6; k >= 0; --k) {
                if (top_val[k + 1] <= top_val[k]) break;
                float tv = top_val[k];
                top_val[k] = top_val[k + 1];
                top_val[k + 1] = tv;
                int ti = top_idx[k];
                top_idx[k] = top_idx[k + 1];
                top_idx[k + 1] = ti;
            }
        }
    }
    float mx = top_val[0], den = 0.0f;
    for (int i = 0; i < n; ++i) den += expf(logits[i] - mx);
    float p[8], tot = 0.0f;
    for (int k = 0; k < 8; ++k) {
        p[k] = expf(top_val[k] - mx) / den;
        tot += p[k];
    }
    for (int k = 0; k < 8; ++k) {
        idx[k] = top_idx[k];
        scores[k] = p[k] / tot;
    }
}

/* ------------------------------------------------------------------ */
/* KV append, token-major: DN:670-689. offset = (pos*nkv + kvh)*hd + d,  */
/* value rounded to the cache dtype (reference: half; build: bf16).      */
void qffo_kv_append(const float* k_in, const float* v_in, void* k_cache,
                    void* v_cache, int cache_dtype, int pos, int max_seq,
                    int nkv, int hd) {
    if (pos >= max_seq) return;
    for (int i = 0; i < nkv * hd; ++i) {
        size_t off = (size_t)pos * nkv * hd + i;
        store_elem(k_cache, cache_dtype, off, k_in[i]);
        store_elem(v_cache, cache_dtype, off, v_in[i]);
    }
}

/* Attention gate: DN:700-708, out = float(attn_half) * sigmoid(gate). */
void qffo_attention_gate(const uint16_t* attn_half, const float* gate, int n,
                         float* out) {
    for (int i = 0; i < n; ++i)
        out[i] = qffo_f16_to_f32(attn_half[i]) * qffo_sigmoid_f32(gate[i]);
}

/* ------------------------------------------------------------------ */
/* Full-attention decode, reference order (RUN:1041-1167), in two       */
/* halves so a prefill row can be checked on its own:                   */
/*   qffo_gqa_append_kv: head RMSNorm of k (DN:614-632), host fp32 RoPE  */
/*     tables (RUN:1090-1099) + RoPE (DN:634-651), KV append             */
/*     (DN:670-689) of k and the raw v;                                  */
/*   qffo_gqa_attend: split q/gate (DN:599-612), head RMSNorm + RoPE of  */
/*     q, q rounded to half (RUN:1119-1126), split-KV attention over     */
/*     pos+1 entries (ATT:134-377), half(out), gate (DN:700-708).        */
/* q_gate [16][512] per-head interleaved, k_new/v_new [2][256], caches   */
/* [max_seq][2][256] of cache_dtype, out [16][256] f32.                  */
/* q_dtype / attn_dtype: rounding of q before attention and of the       */
/* attention output before the gate (2 = half as the reference does,     */
/* 0 = keep fp32).                                                       */
void qffo_gqa_append_kv(const float* k_new, const float* v_new,
                        const float* k_norm_w, float theta, int rot, float eps,
                        void* k_cache, void* v_cache, int cache_dtype, int pos,
                        int max_seq) {
    float k[2 * 256], cs[256], sn[256];
    memcpy(k, k_new, sizeof(k));
    qffo_head_rmsnorm_f32(k, k_norm_w, 2, 256, eps);
    qffo_rope_tables_f32(pos, theta, rot, cs, sn);
    qffo_rope_partial_f32(k, cs, sn, 2, 256, rot);
    qffo_kv_append(k, v_new, k_cache, v_cache, cache_dtype, pos, max_seq, 2, 256);
}

/* T consecutive tokens starting at start_pos: k, v are [T][2][256]. */
void qffo_gqa_append_kv_seq(int T, int start_pos, const float* k, const float* v,
                            const float* k_norm_w, float theta, int rot, float eps,
                            void* k_cache, void* v_cache, int cache_dtype,
                            int max_seq) {
    for (int t = 0; t < T; ++t)
        qffo_gqa_append_kv(k + (size_t)t * 512, v + (size_t)t * 512, k_norm_w,
                           theta, rot, eps, k_cache, v_cache, cache_dtype,
                           start_pos + t, max_seq);
}

void qffo_gqa_attend(const float* q_gate, const float* q_norm_w, float theta,
                     int rot, float scale, float eps, const void* k_cache,
                     const void* v_cache, int cache_dtype, int pos, int q_dtype,
                     int attn_dtype, int num_chunks, float* out) {
    const int NQ = 16, NKV = 2, HD = 256;
    float q[16 * 256], gate[16 * 256], cs[256], sn[256];
    for (int h = 0; h < NQ; ++h)
        for (int i = 0; i < HD; ++i) {
            q[h * HD + i] = q_gate[h * 512 + i];
            gate[h * HD + i] = q_gate[h * 512 + 256 + i];
        }
    qffo_head_rmsnorm_f32(q, q_norm_w, NQ, HD, eps);
    qffo_rope_tables_f32(pos, theta, rot, cs, sn);
    qffo_rope_partial_f32(q, cs, sn, NQ, HD, rot);
    for (int i = 0; i < NQ * HD; ++i) q[i] = qffo_round_to(q[i], q_dtype);
    int L = pos + 1;
    float* Kf = (float*)malloc(sizeof(float) * (size_t)L * NKV * HD);
    float* Vf = (float*)malloc(sizeof(float) * (size_t)L * NKV * HD);
    for (size_t i = 0; i < (size_t)L * NKV * HD; ++i) {
        Kf[i] = load_elem(k_cache, cache_dtype, i);
        Vf[i] = load_elem(v_cache, cache_dtype, i);
    }
    float att[16 * 256];
    qffo_attention_decode_f32(q, Kf, Vf, L, NQ, NKV, HD, scale, num_chunks, att);
    for (int i = 0; i < NQ * HD; ++i)
        out[i] = qffo_round_to(att[i], attn_dtype) * qffo_sigmoid_f32(gate[i]);
    free(Kf);
    free(Vf);
}

/* fp64 yardstick for qffo_gqa_attend: same steps, single-pass softmax,
 * no rounding of q or of the attention output. The caches hold whatever
 * the fp32 path appended (their dtype is part of the layer's semantics). */
void qffo_gqa_attend_f64(const double* q_gate, const double* q_norm_w,
                         double theta, int rot, double scale, double eps,
                         const void* k_cache, const void* v_cache,
                         int cache_dtype, int pos, double* out) {
    const int NQ = 16, NKV = 2, HD = 256;
    double q[16 * 256], gate[16 * 256], cs[256], sn[256];
    for (int h = 0; h < NQ; ++h)
        for (int i = 0; i < HD; ++i) {
            q[h * HD + i] = q_gate[h * 512 + i];
            gate[h * HD + i] = q_gate[h * 512 + 256 + i];
        }
    qffo_head_rmsnorm_f64(q, q_norm_w, NQ, HD, eps);
    qffo_rope_tables_f64(pos, theta, rot, cs, sn);
    qffo_rope_partial_f64(q, cs, sn, NQ, HD, rot);
    int L = pos + 1;
    double* Kd = (double*)malloc(sizeof(double) * (size_t)L * NKV * HD);
    double* Vd = (double*)malloc(sizeof(double) * (size_t)L * NKV * HD);
    for (size_t i = 0; i < (size_t)L * NKV * HD; ++i) {
        Kd[i] = load_elem(k_cache, cache_dtype, i);
        Vd[i] = load_elem(v_cache, cache_dtype, i);
    }
    double att[16 * 256];
    qffo_attention_decode_f64(q, Kd, Vd, L, NQ, NKV, HD, scale, 1, att);
    for (int i = 0; i < NQ * HD; ++i) out[i] = att[i] * qffo_sigmoid_f64(gate[i]);
    free(Kd);
    free(Vd);
}
