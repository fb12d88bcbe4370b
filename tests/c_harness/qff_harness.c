/*
 * qff_harness.c -- a plain C caller of libqff_hip.so through include/qff/qff.h
 * only, as the Swift runner would be (a C module map over the same header):
 * no C++, no torch, device memory from the HIP runtime's C API.
 *
 * TEST PROGRAM. It checks, against the CPU oracle (oracle/build/
 * libqff_oracle.so, test infrastructure), on seeded inputs:
 *   1. qff_deltanet_decode, batch 2, bf16 activations, fp32 outputs, three
 *      steps in a row: outputs max-abs <= 2e-2, the conv state bit for bit,
 *      the fp32 state per-head relative Frobenius error <= 1e-4;
 *   2. qff_gqa_decode, batch 2 at positions 37 and 300 of a 512-position
 *      cache: outputs max-abs <= 2e-2 against the reference's order (q and
 *      the attention output rounded to fp16);
 *   3. the error paths: null pointers return QFF_ERR_INVALID_ARG, a batch
 *      above the context's max_batch QFF_ERR_WORKSPACE, and
 *      qff_status_string names them.
 * Exit status 0 when every check passes; each failure prints one line.
 *
 * Build (tests/c_harness/Makefile): gcc -std=c99 against include/, linked to
 * qwen-fieldfare_amd/lib/libqff_hip.so, oracle/build/libqff_oracle.so and
 * libamdhip64.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qff/qff.h"

/* ---- oracle entry points (oracle/qff_oracle.c, fp32 reference order) ---- */
uint16_t qffo_f32_to_bf16(float f);
float qffo_bf16_to_f32(uint16_t h);
void qffo_deltanet_token_f32(const float* qkv, const float* z, const float* a, const float* b,
                             const float* a_log, const float* dt_bias, const float* conv_w,
                             const float* norm_w, float eps, float* conv_state, float* ssm, float* out);
void qffo_gqa_append_kv(const float* k_new, const float* v_new, const float* k_norm_w, float theta, int rot,
                        float eps, void* k_cache, void* v_cache, int cache_dtype, int pos, int max_seq);
void qffo_gqa_attend(const float* q_gate, const float* q_norm_w, float theta, int rot, float scale, float eps,
                     const void* k_cache, const void* v_cache, int cache_dtype, int pos, int q_dtype,
                     int attn_dtype, int num_chunks, float* out);

static int failures = 0;

#define HIP_OK(call)                                                               \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) {                                                    \
            fprintf(stderr, "qff_harness: %s failed: %s\n", #call, hipGetErrorString(e_)); \
            exit(2);                                                               \
        }                                                                          \
    } while (0)

#define QFF_OK_CALL(call)                                                          \
    do {                                                                           \
        int s_ = (call);                                                           \
        if (s_ != QFF_OK) {                                                        \
            fprintf(stderr, "qff_harness: %s -> %d (%s)\n", #call, s_, qff_status_string(s_)); \
            exit(3);                                                               \
        }                                                                          \
    } while (0)

static void check(int ok, const char* what, double value, double bar) {
    printf("  %-44s %.3g (bar %.3g) %s\n", what, value, bar, ok ? "ok" : "FAIL");
    if (!ok) ++failures;
}

/* splitmix64 stream, then Box-Muller: seeded normal samples */
static uint64_t rng_state;
static uint64_t next_u64(void) {
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static float uniform01(void) { return (float)((next_u64() >> 11) * (1.0 / 9007199254740992.0)); }
static float normal(void) {
    float u1 = uniform01(), u2 = uniform01();
    if (u1 < 1e-12f) u1 = 1e-12f;
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
}
static void fill_normal(float* x, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) x[i] = normal() * scale;
}
/* bf16 bits of x, and x replaced by the value those bits hold */
static void to_bf16(float* x, uint16_t* bits, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        bits[i] = qffo_f32_to_bf16(x[i]);
        x[i] = qffo_bf16_to_f32(bits[i]);
    }
}
static void* dev_copy(const void* host, size_t bytes) {
    void* d = NULL;
    HIP_OK(hipMalloc(&d, bytes));
    HIP_OK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
    return d;
}
static void host_copy(void* host, const void* dev, size_t bytes) {
    HIP_OK(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
}
static double max_abs_diff(const float* a, const float* b, size_t n) {
    double m = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double d = fabs((double)a[i] - (double)b[i]);
        if (d > m || d != d) m = d;
    }
    return m;
}

/* ---- 1. DeltaNet decode ----------------------------------------------------- */
static void run_deltanet(qff_ctx* ctx) {
    enum { B = 2, STEPS = 3 };
    const size_t nconv = (size_t)8192 * 4, nssm = (size_t)32 * 128 * 128;
    float a_log[32], dt_bias[32], norm_w[128];
    float* conv_w = malloc(sizeof(float) * nconv);
    for (int h = 0; h < 32; ++h) {
        a_log[h] = logf(1.0f + 15.0f * uniform01());
        dt_bias[h] = 0.5f * normal();
    }
    for (int i = 0; i < 128; ++i) norm_w[i] = 1.0f + 0.1f * normal();
    fill_normal(conv_w, nconv, 0.5f);

    float* conv = malloc(sizeof(float) * B * nconv);
    float* ssm = malloc(sizeof(float) * B * nssm);
    fill_normal(conv, B * nconv, 1.0f);
    fill_normal(ssm, B * nssm, 0.02f);

    float* d_alog = dev_copy(a_log, sizeof a_log);
    float* d_dtb = dev_copy(dt_bias, sizeof dt_bias);
    float* d_convw = dev_copy(conv_w, sizeof(float) * nconv);
    float* d_normw = dev_copy(norm_w, sizeof norm_w);
    float* d_conv = dev_copy(conv, sizeof(float) * B * nconv);
    float* d_ssm = dev_copy(ssm, sizeof(float) * B * nssm);
    qff_deltanet_params prm = {d_alog, d_dtb, d_convw, d_normw, 1e-6f};

    float* qkv = malloc(sizeof(float) * B * 8192);
    float* z = malloc(sizeof(float) * B * 4096);
    uint16_t* qkv_b = malloc(sizeof(uint16_t) * B * 8192);
    uint16_t* z_b = malloc(sizeof(uint16_t) * B * 4096);
    float a[B * 32], b[B * 32];
    float* ref = malloc(sizeof(float) * B * 4096);
    float* got = malloc(sizeof(float) * B * 4096);
    float* got_conv = malloc(sizeof(float) * B * nconv);
    float* got_ssm = malloc(sizeof(float) * B * nssm);
    void *d_qkv = NULL, *d_z = NULL, *d_a = NULL, *d_b = NULL, *d_out = NULL;
    HIP_OK(hipMalloc(&d_qkv, sizeof(uint16_t) * B * 8192));
    HIP_OK(hipMalloc(&d_z, sizeof(uint16_t) * B * 4096));
    HIP_OK(hipMalloc(&d_a, sizeof a));
    HIP_OK(hipMalloc(&d_b, sizeof b));
    HIP_OK(hipMalloc(&d_out, sizeof(float) * B * 4096));

    double worst_out = 0.0, worst_rel = 0.0;
    int conv_exact = 1;
    for (int step = 0; step < STEPS; ++step) {
        fill_normal(qkv, B * 8192, 1.0f);
        fill_normal(z, B * 4096, 1.0f);
        fill_normal(a, B * 32, 1.0f);
        fill_normal(b, B * 32, 1.0f);
        to_bf16(qkv, qkv_b, B * 8192);
        to_bf16(z, z_b, B * 4096);
        HIP_OK(hipMemcpy(d_qkv, qkv_b, sizeof(uint16_t) * B * 8192, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(d_z, z_b, sizeof(uint16_t) * B * 4096, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(d_a, a, sizeof a, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(d_b, b, sizeof b, hipMemcpyHostToDevice));
        QFF_OK_CALL(qff_deltanet_decode(ctx, NULL, &prm, d_qkv, d_z, QFF_BF16, d_a, d_b, d_conv, d_ssm, d_out,
                                        QFF_F32, B));
        HIP_OK(hipDeviceSynchronize());
        for (int s = 0; s < B; ++s)
            qffo_deltanet_token_f32(qkv + s * 8192, z + s * 4096, a + s * 32, b + s * 32, a_log, dt_bias, conv_w,
                                    norm_w, 1e-6f, conv + s * nconv, ssm + s * nssm, ref + s * 4096);
        host_copy(got, d_out, sizeof(float) * B * 4096);
        host_copy(got_conv, d_conv, sizeof(float) * B * nconv);
        host_copy(got_ssm, d_ssm, sizeof(float) * B * nssm);
        double e = max_abs_diff(got, ref, (size_t)B * 4096);
        if (e > worst_out || e != e) worst_out = e;
        if (memcmp(got_conv, conv, sizeof(float) * B * nconv) != 0) conv_exact = 0;
        for (int hd = 0; hd < B * 32; ++hd) {
            double num = 0.0, den = 0.0;
            for (int i = 0; i < 128 * 128; ++i) {
                double r = ssm[(size_t)hd * 128 * 128 + i], g = got_ssm[(size_t)hd * 128 * 128 + i];
                num += (g - r) * (g - r);
                den += r * r;
            }
            double rel = sqrt(num) / (den > 0.0 ? sqrt(den) : 1e-30);
            if (rel > worst_rel || rel != rel) worst_rel = rel;
        }
    }
    printf("qff_deltanet_decode: batch %d, %d steps\n", B, STEPS);
    check(worst_out <= 2e-2, "outputs max-abs vs oracle", worst_out, 2e-2);
    check(conv_exact, "conv state bit-exact (1 = yes)", conv_exact, 1);
    check(worst_rel <= 1e-4, "state per-head rel Frobenius", worst_rel, 1e-4);

    hipFree(d_alog); hipFree(d_dtb); hipFree(d_convw); hipFree(d_normw); hipFree(d_conv); hipFree(d_ssm);
    hipFree(d_qkv); hipFree(d_z); hipFree(d_a); hipFree(d_b); hipFree(d_out);
    free(conv_w); free(conv); free(ssm); free(qkv); free(z); free(qkv_b); free(z_b);
    free(ref); free(got); free(got_conv); free(got_ssm);
}

/* ---- 2. GQA decode ------------------------------------------------------------ */
static void run_gqa(qff_ctx* ctx) {
    enum { B = 2, L = 512 };
    const int pos[B] = {37, 300};
    const size_t cache_n = (size_t)L * 512;   /* per sequence: [L][2][256] */
    float q_norm_w[256], k_norm_w[256];
    for (int i = 0; i < 256; ++i) {
        q_norm_w[i] = 1.0f + 0.1f * normal();
        k_norm_w[i] = 1.0f + 0.1f * normal();
    }
    float* cache_f = malloc(sizeof(float) * cache_n);
    uint16_t* kc = malloc(sizeof(uint16_t) * B * cache_n);
    uint16_t* vc = malloc(sizeof(uint16_t) * B * cache_n);
    fill_normal(cache_f, cache_n, 1.0f);
    to_bf16(cache_f, kc, cache_n);
    fill_normal(cache_f, cache_n, 1.0f);
    to_bf16(cache_f, vc, cache_n);
    memcpy(kc + cache_n, kc, sizeof(uint16_t) * cache_n);
    memcpy(vc + cache_n, vc, sizeof(uint16_t) * cache_n);

    float* qg = malloc(sizeof(float) * B * 16 * 512);
    float kn[B * 512], vn[B * 512];
    uint16_t* qg_b = malloc(sizeof(uint16_t) * B * 16 * 512);
    uint16_t kn_b[B * 512], vn_b[B * 512];
    fill_normal(qg, B * 16 * 512, 1.0f);
    fill_normal(kn, B * 512, 1.0f);
    fill_normal(vn, B * 512, 1.0f);
    to_bf16(qg, qg_b, B * 16 * 512);
    to_bf16(kn, kn_b, B * 512);
    to_bf16(vn, vn_b, B * 512);

    float* d_qn = dev_copy(q_norm_w, sizeof q_norm_w);
    float* d_kn = dev_copy(k_norm_w, sizeof k_norm_w);
    void* d_kc = dev_copy(kc, sizeof(uint16_t) * B * cache_n);
    void* d_vc = dev_copy(vc, sizeof(uint16_t) * B * cache_n);
    void* d_qg = dev_copy(qg_b, sizeof(uint16_t) * B * 16 * 512);
    void* d_knew = dev_copy(kn_b, sizeof kn_b);
    void* d_vnew = dev_copy(vn_b, sizeof vn_b);
    int32_t* d_pos = dev_copy(pos, sizeof pos);
    void* d_out = NULL;
    HIP_OK(hipMalloc(&d_out, sizeof(float) * B * 16 * 256));
    qff_gqa_params prm = {d_qn, d_kn, 1e7f, 64, 1.0f / 16.0f, 1e-6f, 0};   /* bf16 cache */
    QFF_OK_CALL(qff_gqa_decode(ctx, NULL, &prm, d_qg, d_knew, d_vnew, QFF_BF16, d_kc, d_vc, d_pos, d_out, QFF_F32,
                               B, L));
    HIP_OK(hipDeviceSynchronize());
    float* got = malloc(sizeof(float) * B * 16 * 256);
    host_copy(got, d_out, sizeof(float) * B * 16 * 256);

    double worst = 0.0;
    float ref[16 * 256];
    for (int s = 0; s < B; ++s) {
        /* the reference's order: append (bf16 cache), q and attention output
         * rounded to fp16 (QFF_F16 = 2), single pass over the chunks */
        qffo_gqa_append_kv(kn + s * 512, vn + s * 512, k_norm_w, 1e7f, 64, 1e-6f, kc + s * cache_n,
                           vc + s * cache_n, QFF_BF16, pos[s], L);
        qffo_gqa_attend(qg + (size_t)s * 16 * 512, q_norm_w, 1e7f, 64, 1.0f / 16.0f, 1e-6f, kc + s * cache_n,
                        vc + s * cache_n, QFF_BF16, pos[s], QFF_F16, QFF_F16, 1, ref);
        double e = max_abs_diff(got + (size_t)s * 16 * 256, ref, 16 * 256);
        if (e > worst || e != e) worst = e;
    }
    printf("qff_gqa_decode: batch %d at positions %d, %d\n", B, pos[0], pos[1]);
    check(worst <= 2e-2, "outputs max-abs vs oracle", worst, 2e-2);

    hipFree(d_qn); hipFree(d_kn); hipFree(d_kc); hipFree(d_vc); hipFree(d_qg); hipFree(d_knew); hipFree(d_vnew);
    hipFree(d_pos); hipFree(d_out);
    free(cache_f); free(kc); free(vc); free(qg); free(qg_b); free(got);
}

int main(void) {
    rng_state = 20260101ull;
    printf("qff_harness: library version %d\n", qff_version());
    qff_ctx* ctx = NULL;
    qff_ctx_cfg cfg = {4, 512, 64};
    QFF_OK_CALL(qff_ctx_create(&ctx, 0, &cfg));
    run_deltanet(ctx);
    run_gqa(ctx);

    /* 3. error paths: null pointers, then batch 8 on a max_batch 4 context
     * (buffers sized for batch 8, so nothing could run out of bounds) */
    int s = qff_deltanet_decode(ctx, NULL, NULL, NULL, NULL, QFF_BF16, NULL, NULL, NULL, NULL, NULL, QFF_F32, 2);
    printf("error path: null pointers -> %d (%s)\n", s, qff_status_string(s));
    if (s != QFF_ERR_INVALID_ARG) ++failures;
    {
        enum { B8 = 8 };
        void *w = NULL, *qkv = NULL, *z = NULL, *ab = NULL, *conv = NULL, *ssm = NULL, *out = NULL;
        HIP_OK(hipMalloc(&w, sizeof(float) * 8192 * 4));
        HIP_OK(hipMalloc(&qkv, sizeof(uint16_t) * B8 * 8192));
        HIP_OK(hipMalloc(&z, sizeof(uint16_t) * B8 * 4096));
        HIP_OK(hipMalloc(&ab, sizeof(float) * B8 * 64));
        HIP_OK(hipMalloc(&conv, sizeof(float) * B8 * 8192 * 4));
        HIP_OK(hipMalloc(&ssm, sizeof(float) * B8 * 32 * 128 * 128));
        HIP_OK(hipMalloc(&out, sizeof(float) * B8 * 4096));
        qff_deltanet_params prm = {(const float*)w, (const float*)w, (const float*)w, (const float*)w, 1e-6f};
        s = qff_deltanet_decode(ctx, NULL, &prm, qkv, z, QFF_BF16, (const float*)ab, (const float*)ab + B8 * 32,
                                (float*)conv, (float*)ssm, out, QFF_F32, B8);
        printf("error path: batch %d on max_batch 4 -> %d (%s)\n", B8, s, qff_status_string(s));
        if (s != QFF_ERR_WORKSPACE) ++failures;
        HIP_OK(hipDeviceSynchronize());
        hipFree(w); hipFree(qkv); hipFree(z); hipFree(ab); hipFree(conv); hipFree(ssm); hipFree(out);
    }
    QFF_OK_CALL(qff_ctx_destroy(ctx));
    printf("qff_harness: %s\n", failures ? "FAILED" : "OK");
    return failures ? 1 : 0;
}
