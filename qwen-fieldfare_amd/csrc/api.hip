// api.hip -- the extern "C" entry points of include/qff/qff.h: argument
// validation, the context and its workspace, and the two small kernels
// (raw KV append, f16 attention gate) that do not belong to a larger file.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "common.hpp"
#include "internal.hpp"

namespace qff {

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static qff_ctx_cfg resolve(const qff_ctx_cfg* cfg) {
    qff_ctx_cfg c{};
    if (cfg) c = *cfg;
    if (c.max_batch <= 0) c.max_batch = 32;
    if (c.max_ctx <= 0) c.max_ctx = 65536;
    if (c.max_prefill_tokens <= 0) c.max_prefill_tokens = 8192;
    return c;
}

// Tokens per slice of a many-token Q4 product (fp16 activations in workspace).
int q4_xs_tokens(const qff_ctx_cfg& cfg) { return std::max(std::max(cfg.max_batch, cfg.max_prefill_tokens), 1024); }

WorkspaceLayout workspace_layout(const qff_ctx_cfg& cfg) {
    WorkspaceLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
    const size_t B = static_cast<size_t>(cfg.max_batch);
    const size_t T = static_cast<size_t>(cfg.max_prefill_tokens);
    const size_t S = static_cast<size_t>(gqa_slots(cfg));
    L.gqa_m = take(S * 8 * sizeof(float));
    L.gqa_d = take(S * 8 * sizeof(float));
    L.gqa_o = take(S * 8 * 256 * sizeof(float));
    L.gqa_qb = take(T * 16 * 256 * sizeof(uint16_t));
    L.gqa_kv16 = take(static_cast<size_t>(cfg.max_ctx) * 512 * sizeof(uint16_t));
    L.gqa_vt = take(static_cast<size_t>((cfg.max_ctx + 63) / 64) * 64 * 512 * sizeof(uint16_t));
    L.q4_x16 = take(static_cast<size_t>(q4_xs_tokens(cfg)) * 4096 * sizeof(uint16_t));
    L.q4_fm = take(static_cast<size_t>(q4_xs_tokens(cfg)) * sizeof(float));
    L.q4_sk_part = take(static_cast<size_t>(kQ4SkSlots) * 16 * 64 * sizeof(float));
    const size_t TC = (T + 63) / 64 * 64;   // tokens rounded up to whole chunks
    L.pf_o = take(TC * 4096 * sizeof(float));   // pre-norm DeltaNet prefill output, fp32
    L.sched = take(2 * kSchedSlots * sizeof(unsigned));
    L.dn_arrive = take(B * 16 * sizeof(unsigned));
    // DeltaNet prefill chunk records (deltanet_chunked.hip): per chunk and key
    // head the K image and Q blocks (hi, lo), per chunk and value head the T
    // and P blocks (hi, lo), gate factors and beta V
    const size_t NC = TC / 64;
    L.kimg = take(NC * 16 * 2 * 64 * 128 * sizeof(uint16_t));
    L.qop = take(NC * 16 * 2 * 16 * 512 * sizeof(uint16_t));
    L.top = take(NC * 32 * 2 * 6 * 512 * sizeof(uint16_t));
    L.pop = take(NC * 32 * 2 * 6 * 512 * sizeof(uint16_t));
    L.gates = take(NC * 32 * 4 * 64 * sizeof(float));
    L.bv = take(NC * 32 * 64 * 128 * sizeof(float));
    L.total = off;
    return L;
}

RopeFreqs rope_freqs(float theta) {
    RopeFreqs r;
    for (int i = 0; i < 32; ++i) r.f[i] = 1.0f / powf(theta, static_cast<float>(2 * i) / 64.0f);
    return r;
}

// out = float(attn_f16) * sigmoid(gate): deltanet.metal:700-708.
__global__ void attention_gate_kernel(const uint16_t* __restrict__ attn, const float* __restrict__ gate,
                                      float* __restrict__ out, int count) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = f16_to_f32(attn[i]) * sigmoid(gate[i]);
}

// Token-major append: deltanet.metal:670-689.
template <int DT>
__global__ void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                 void* __restrict__ kc, void* __restrict__ vc, int pos) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;  // 0..511 = kv_head*256 + d
    if (i >= 512) return;
    size_t off = static_cast<size_t>(pos) * 512 + i;
    elem<DT>::store(kc, off, k[i]);
    elem<DT>::store(vc, off, v[i]);
}

hipError_t launch_attention_gate(hipStream_t stream, const uint16_t* attn, const float* gate,
                                 float* out, int count) {
    attention_gate_kernel<<<(count + 255) / 256, 256, 0, stream>>>(attn, gate, out, count);
    return hipGetLastError();
}

hipError_t launch_kv_append(hipStream_t stream, const float* k, const float* v, void* k_cache,
                            void* v_cache, qff_dtype cache_dtype, int pos, int max_seq) {
    if (pos >= max_seq) return hipSuccess;
    if (cache_dtype == QFF_BF16)
        kv_append_kernel<1><<<2, 256, 0, stream>>>(k, v, k_cache, v_cache, pos);
    else
        kv_append_kernel<2><<<2, 256, 0, stream>>>(k, v, k_cache, v_cache, pos);
    return hipGetLastError();
}

}  // namespace qff

using namespace qff;

#define QFF_CHECK_HIP(expr)                       \
    do {                                          \
        if ((expr) != hipSuccess) return QFF_ERR_HIP; \
    } while (0)

extern "C" {

int qff_version(void) { return (0 << 16) | 1; }

const char* qff_status_string(int status) {
    switch (status) {
        case QFF_OK: return "ok";
        case QFF_ERR_INVALID_ARG: return "invalid argument";
        case QFF_ERR_UNSUPPORTED: return "unsupported shape";
        case QFF_ERR_HIP: return "HIP runtime error";
        case QFF_ERR_WORKSPACE: return "request exceeds the context workspace";
        case QFF_ERR_OUT_OF_MEMORY: return "out of device memory";
        default: return "unknown status";
    }
}

int qff_workspace_size(const qff_ctx_cfg* cfg, size_t* bytes) {
    if (!bytes) return QFF_ERR_INVALID_ARG;
    if (cfg && (cfg->max_batch < 0 || cfg->max_ctx < 0 || cfg->max_prefill_tokens < 0))
        return QFF_ERR_INVALID_ARG;
    *bytes = workspace_layout(resolve(cfg)).total;
    return QFF_OK;
}

int qff_ctx_create(qff_ctx** out, int device, const qff_ctx_cfg* cfg) {
    if (!out) return QFF_ERR_INVALID_ARG;
    *out = nullptr;
    if (cfg && (cfg->max_batch < 0 || cfg->max_ctx < 0 || cfg->max_prefill_tokens < 0))
        return QFF_ERR_INVALID_ARG;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return QFF_ERR_INVALID_ARG;
    hipDeviceProp_t prop;
    QFF_CHECK_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return QFF_ERR_UNSUPPORTED;
    int prev = 0;
    QFF_CHECK_HIP(hipGetDevice(&prev));
    QFF_CHECK_HIP(hipSetDevice(device));
    qff_ctx* c = new (std::nothrow) qff_ctx();
    if (!c) return QFF_ERR_OUT_OF_MEMORY;
    c->device = device;
    c->cfg = resolve(cfg);
    WorkspaceLayout L = workspace_layout(c->cfg);
    if (hipMalloc(&c->ws, L.total) != hipSuccess) {
        delete c;
        (void)hipSetDevice(prev);
        return QFF_ERR_OUT_OF_MEMORY;
    }
    c->ws_bytes = L.total;
    char* base = static_cast<char*>(c->ws);
    c->gqa_m = reinterpret_cast<float*>(base + L.gqa_m);
    c->gqa_d = reinterpret_cast<float*>(base + L.gqa_d);
    c->gqa_o = reinterpret_cast<float*>(base + L.gqa_o);
    auto u16 = [&](size_t off) { return reinterpret_cast<uint16_t*>(base + off); };
    c->gqa_qb = u16(L.gqa_qb);
    c->gqa_kv16 = u16(L.gqa_kv16);
    c->gqa_vt = u16(L.gqa_vt);
    c->q4_x16 = reinterpret_cast<uint16_t*>(base + L.q4_x16);
    c->q4_fm = reinterpret_cast<float*>(base + L.q4_fm);
    c->q4_xs_tokens = q4_xs_tokens(c->cfg);
    c->q4_sk_part = reinterpret_cast<float*>(base + L.q4_sk_part);
    c->pf_o = reinterpret_cast<float*>(base + L.pf_o);
    c->sched = reinterpret_cast<unsigned*>(base + L.sched);
    c->num_cu = prop.multiProcessorCount;
    c->dn_arrive = reinterpret_cast<unsigned*>(base + L.dn_arrive);
    if (hipMemset(c->sched, 0, 2 * kSchedSlots * sizeof(unsigned)) != hipSuccess ||
        hipMemset(c->dn_arrive, 0, static_cast<size_t>(c->cfg.max_batch) * 16 * sizeof(unsigned)) != hipSuccess) {
        (void)hipFree(c->ws);
        delete c;
        (void)hipSetDevice(prev);
        return QFF_ERR_HIP;
    }
    c->dn = qff_dn_bufs{u16(L.kimg), u16(L.qop), u16(L.top), u16(L.pop), reinterpret_cast<float*>(base + L.gates),
                        reinterpret_cast<float*>(base + L.bv)};
    (void)hipSetDevice(prev);
    *out = c;
    return QFF_OK;
}

static void prof_release(qff_ctx* ctx) {
    for (auto& r : ctx->prof_pool) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    ctx->prof_pool.clear();
    ctx->prof_n = 0;
    ctx->prof = false;
}

int qff_profile_enable(qff_ctx* ctx, int enable) {
    if (!ctx) return QFF_ERR_INVALID_ARG;
    if (!enable) {
        prof_release(ctx);
        return QFF_OK;
    }
    if (ctx->prof_pool.empty()) {
        constexpr int kPool = 4096;
        ctx->prof_pool.resize(kPool);
        for (int i = 0; i < kPool; ++i) {
            if (hipEventCreate(&ctx->prof_pool[i].start) != hipSuccess ||
                hipEventCreate(&ctx->prof_pool[i].stop) != hipSuccess) {
                ctx->prof_pool.resize(i);
                prof_release(ctx);
                return QFF_ERR_HIP;
            }
            ctx->prof_pool[i].name = "";
        }
    }
    ctx->prof_n = 0;
    ctx->prof = true;
    return QFF_OK;
}

int qff_profile_read(qff_ctx* ctx, const char** names, float* ms, int capacity, int* count) {
    if (!ctx || !count || capacity < 0 || (capacity > 0 && (!names || !ms))) return QFF_ERR_INVALID_ARG;
    int n = 0;
    for (int i = 0; i < ctx->prof_n && n < capacity; ++i, ++n) {
        if (hipEventSynchronize(ctx->prof_pool[i].stop) != hipSuccess) return QFF_ERR_HIP;
        float t = 0.0f;
        if (hipEventElapsedTime(&t, ctx->prof_pool[i].start, ctx->prof_pool[i].stop) != hipSuccess)
            return QFF_ERR_HIP;
        names[n] = ctx->prof_pool[i].name;
        ms[n] = t;
    }
    *count = n;
    ctx->prof_n = 0;
    return QFF_OK;
}

int qff_ctx_destroy(qff_ctx* ctx) {
    if (!ctx) return QFF_ERR_INVALID_ARG;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ctx->device);
    prof_release(ctx);
    hipError_t e = hipSuccess;
    if (ctx->ws) e = hipFree(ctx->ws);
    (void)hipSetDevice(prev);
    delete ctx;
    return e == hipSuccess ? QFF_OK : QFF_ERR_HIP;
}

int qff_q4_dequant(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w, const void* scales,
                   const void* biases, qff_dtype sb_dtype, float* out, int rows, int cols) {
    if (!ctx || !w || !scales || !biases || !out) return QFF_ERR_INVALID_ARG;
    if (sb_dtype != QFF_F16 && sb_dtype != QFF_BF16) return QFF_ERR_INVALID_ARG;
    if (rows <= 0 || cols <= 0) return QFF_ERR_INVALID_ARG;
    if (cols % 64 != 0) return QFF_ERR_UNSUPPORTED;
    QFF_CHECK_HIP(launch_q4_dequant(stream, w, scales, biases, sb_dtype, out, rows, cols));
    return QFF_OK;
}

int qff_q4_matmul(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w, const void* scales,
                  const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, void* y,
                  qff_dtype y_dtype, int rows, int cols, int batch) {
    if (!ctx || !w || !scales || !biases || !x || !y) return QFF_ERR_INVALID_ARG;
    if (sb_dtype != QFF_F16 && sb_dtype != QFF_BF16) return QFF_ERR_INVALID_ARG;
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return QFF_ERR_INVALID_ARG;
    if (rows <= 0 || cols <= 0 || batch <= 0) return QFF_ERR_INVALID_ARG;
    if (cols % 64 != 0 || cols > 4096) return QFF_ERR_UNSUPPORTED;
    QFF_CHECK_HIP(launch_q4_matmul(ctx, stream, w, scales, biases, sb_dtype, x, x_dtype, y, y_dtype,
                                   rows, cols, batch));
    return QFF_OK;
}

int qff_q8_dequant(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w, const void* scales,
                   const void* biases, qff_dtype sb_dtype, float* out, int rows, int cols) {
    if (!ctx || !w || !scales || !biases || !out) return QFF_ERR_INVALID_ARG;
    if (sb_dtype != QFF_F16 && sb_dtype != QFF_BF16) return QFF_ERR_INVALID_ARG;
    if (rows <= 0 || cols <= 0) return QFF_ERR_INVALID_ARG;
    if (cols % 64 != 0) return QFF_ERR_UNSUPPORTED;
    QFF_CHECK_HIP(launch_q8_dequant(stream, w, scales, biases, sb_dtype, out, rows, cols));
    return QFF_OK;
}

int qff_router_top8(qff_ctx* ctx, qff_stream_t stream, const uint32_t* w, const void* scales,
                    const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, float* logits,
                    int32_t* indices, float* scores, int experts, int cols, int batch) {
    if (!ctx || !w || !scales || !biases || !x || !logits || !indices || !scores) return QFF_ERR_INVALID_ARG;
    if (sb_dtype != QFF_F16 && sb_dtype != QFF_BF16) return QFF_ERR_INVALID_ARG;
    if (!dtype_ok(x_dtype) || experts <= 0 || cols <= 0 || batch <= 0) return QFF_ERR_INVALID_ARG;
    if (experts < 8 || experts > 256 || cols % 64 != 0 || cols > 4096) return QFF_ERR_UNSUPPORTED;
    QFF_CHECK_HIP(launch_router_top8(ctx, stream, w, scales, biases, sb_dtype, x, x_dtype, logits, indices, scores,
                                     experts, cols, batch));
    return QFF_OK;
}

static int check_q4_parts(const qff_ctx* ctx, const qff_q4_part* parts, int nparts, qff_dtype sb_dtype,
                          const void* x, qff_dtype x_dtype, int cols, int batch) {
    if (!ctx || !parts || !x || nparts < 1 || nparts > QFF_Q4_MAX_PARTS) return QFF_ERR_INVALID_ARG;
    if (sb_dtype != QFF_F16 && sb_dtype != QFF_BF16) return QFF_ERR_INVALID_ARG;
    if (!dtype_ok(x_dtype) || cols <= 0 || batch <= 0) return QFF_ERR_INVALID_ARG;
    for (int i = 0; i < nparts; ++i) {
        const qff_q4_part& q = parts[i];
        if (!q.w || !q.scales || !q.biases || !q.y || q.rows <= 0 || !dtype_ok(q.y_dtype))
            return QFF_ERR_INVALID_ARG;
    }
    if (cols % 64 != 0 || cols > 4096) return QFF_ERR_UNSUPPORTED;
    return QFF_OK;
}

int qff_q4_matmul_parts(qff_ctx* ctx, qff_stream_t stream, const qff_q4_part* parts, int nparts,
                        qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, int cols, int batch) {
    const int st = check_q4_parts(ctx, parts, nparts, sb_dtype, x, x_dtype, cols, batch);
    if (st != QFF_OK) return st;
    QFF_CHECK_HIP(launch_q4_parts(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, Q4Norm{}, cols, batch));
    return QFF_OK;
}

int qff_q4_norm_matmul_parts(qff_ctx* ctx, qff_stream_t stream, const qff_q4_part* parts, int nparts,
                             qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, const void* norm_w,
                             qff_dtype norm_dtype, float eps, int cols, int batch) {
    const int st = check_q4_parts(ctx, parts, nparts, sb_dtype, x, x_dtype, cols, batch);
    if (st != QFF_OK) return st;
    if (!norm_w || !dtype_ok(norm_dtype) || !(eps >= 0.0f)) return QFF_ERR_INVALID_ARG;
    Q4Norm norm;
    norm.w = norm_w;
    norm.wbf16 = norm_dtype == QFF_BF16;
    norm.eps = eps;
    QFF_CHECK_HIP(launch_q4_parts(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, batch));
    return QFF_OK;
}

static bool dn_params_ok(const qff_deltanet_params* p) {
    return p && p->a_log && p->dt_bias && p->conv_w && p->norm_w && p->eps >= 0.0f;
}

int qff_deltanet_decode(qff_ctx* ctx, qff_stream_t stream, const qff_deltanet_params* p,
                        const void* qkv, const void* z, qff_dtype in_dtype, const float* a,
                        const float* b, float* conv_state, float* ssm_state, void* out,
                        qff_dtype out_dtype, int batch) {
    if (!ctx || !dn_params_ok(p) || !qkv || !z || !a || !b || !conv_state || !ssm_state || !out)
        return QFF_ERR_INVALID_ARG;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return QFF_ERR_INVALID_ARG;
    if (batch <= 0) return QFF_ERR_INVALID_ARG;
    if (batch > ctx->cfg.max_batch) return QFF_ERR_WORKSPACE;
    QFF_CHECK_HIP(launch_deltanet_decode(ctx, stream, p, qkv, z, in_dtype, a, b, conv_state, ssm_state,
                                         out, out_dtype, batch));
    return QFF_OK;
}

int qff_deltanet_prefill(qff_ctx* ctx, qff_stream_t stream, const qff_deltanet_params* p,
                         const void* qkv, const void* z, qff_dtype in_dtype, const float* a,
                         const float* b, float* conv_state, float* ssm_state, void* out,
                         qff_dtype out_dtype, int T, int chunk) {
    if (!ctx || !dn_params_ok(p) || !qkv || !z || !a || !b || !conv_state || !ssm_state || !out)
        return QFF_ERR_INVALID_ARG;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return QFF_ERR_INVALID_ARG;
    if (T <= 0) return QFF_ERR_INVALID_ARG;
    if (chunk != 64) return QFF_ERR_UNSUPPORTED;
    if (T > ctx->cfg.max_prefill_tokens) return QFF_ERR_WORKSPACE;
    QFF_CHECK_HIP(launch_deltanet_prefill(ctx, stream, p, qkv, z, in_dtype, a, b, conv_state, ssm_state,
                                          out, out_dtype, T));
    return QFF_OK;
}

int qff_gqa_decode(qff_ctx* ctx, qff_stream_t stream, const qff_gqa_params* p, const void* q_gate,
                   const void* k_new, const void* v_new, qff_dtype in_dtype, void* k_cache,
                   void* v_cache, const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                   int max_ctx) {
    if (!ctx || !q_gate || !k_new || !v_new || !k_cache || !v_cache || !positions || !out)
        return QFF_ERR_INVALID_ARG;
    if (const int st = gqa_params_status(p)) return st;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return QFF_ERR_INVALID_ARG;
    if (batch <= 0 || max_ctx <= 0) return QFF_ERR_INVALID_ARG;
    if (batch > ctx->cfg.max_batch || max_ctx > ctx->cfg.max_ctx) return QFF_ERR_WORKSPACE;
    QFF_CHECK_HIP(launch_gqa_decode(ctx, stream, p, q_gate, k_new, v_new, in_dtype, k_cache, v_cache,
                                    positions, out, out_dtype, batch, max_ctx));
    return QFF_OK;
}

int qff_gqa_prefill(qff_ctx* ctx, qff_stream_t stream, const qff_gqa_params* p, const void* q_gate,
                    const void* k, const void* v, qff_dtype in_dtype, void* k_cache, void* v_cache,
                    int start_pos, void* out, qff_dtype out_dtype, int T, int max_ctx) {
    if (!ctx || !q_gate || !k || !v || !k_cache || !v_cache || !out) return QFF_ERR_INVALID_ARG;
    if (const int st = gqa_params_status(p)) return st;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return QFF_ERR_INVALID_ARG;
    if (T <= 0 || start_pos < 0 || max_ctx <= 0) return QFF_ERR_INVALID_ARG;
    if (static_cast<long long>(start_pos) + T > max_ctx) return QFF_ERR_INVALID_ARG;
    if (T > ctx->cfg.max_prefill_tokens) return QFF_ERR_WORKSPACE;   // the staged q rows hold that many tokens
    // the cache copies the attention reads (fp16 K of a bf16 cache, V
    // transposed) hold the context's max_ctx rows
    if (static_cast<long long>(start_pos) + T > ctx->cfg.max_ctx) return QFF_ERR_WORKSPACE;
    QFF_CHECK_HIP(launch_gqa_prefill(ctx, stream, p, q_gate, k, v, in_dtype, k_cache, v_cache, start_pos,
                                     out, out_dtype, T, max_ctx));
    return QFF_OK;
}

int qff_kv_append(qff_ctx* ctx, qff_stream_t stream, const float* k, const float* v, void* k_cache,
                  void* v_cache, qff_dtype cache_dtype, int pos, int max_seq) {
    if (!ctx || !k || !v || !k_cache || !v_cache) return QFF_ERR_INVALID_ARG;
    if (cache_dtype != QFF_BF16 && cache_dtype != QFF_F16) return QFF_ERR_INVALID_ARG;
    if (pos < 0 || max_seq <= 0) return QFF_ERR_INVALID_ARG;
    QFF_CHECK_HIP(launch_kv_append(stream, k, v, k_cache, v_cache, cache_dtype, pos, max_seq));
    return QFF_OK;
}

int qff_attention_gate(qff_ctx* ctx, qff_stream_t stream, const uint16_t* attn_f16, const float* gate,
                       float* out, int count) {
    if (!ctx || !attn_f16 || !gate || !out) return QFF_ERR_INVALID_ARG;
    if (count < 0) return QFF_ERR_INVALID_ARG;
    if (count == 0) return QFF_OK;
    QFF_CHECK_HIP(launch_attention_gate(stream, attn_f16, gate, out, count));
    return QFF_OK;
}

}  // extern "C"
