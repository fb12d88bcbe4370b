// gqa_decode.hip -- full-attention decode (16 q heads on 2 kv heads, head dim
// 256, bf16 token-major KV cache) for a batch of sequences on gfx950.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1076-1150 runs split
// q/gate, head RMSNorm, host RoPE tables + RoPE, the f16 KV append, a cast of
// q to half, Attention.encodeFull (split-KV partial + combine,
// attention.metal:134-224, 342-377; geometry Attention.swift:129-157) and the
// gate (deltanet.metal:700-708), one q head per threadgroup.
//
// Here the eight q heads that share a kv head run in the same workgroup, so
// every K/V byte is read from HBM once, and both products run on the matrix
// cores:
//   partial  grid (chunk, kv head, sequence), 4 waves. Each workgroup
//            normalises and rotates its 8 q heads into LDS (bf16, softmax
//            scale folded in); the workgroup whose chunk holds the new token
//            also normalises/rotates k, appends k and v to the cache and
//            fences them before the chunk is read. Each wave then walks
//            16-position tiles: S^T = K Q^T with 8 MFMA 16x16x32 (K rows
//            straight from HBM, 16 B per lane), online softmax per head in
//            registers, V transposed through a per-wave LDS tile, and
//            O += P V with 16 MFMA 16x16x16. The 4 waves merge in LDS and the
//            workgroup writes one (m, d, o[8][256]) partial.
//   combine  grid (q head, sequence): merges the chunk partials and applies
//            out = attn * sigmoid(gate).
// Lengths come from the device `positions` array, so no host sync is needed;
// workgroups past a sequence's last chunk exit at once.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kVtStride = 20;  // bf16 per transposed V row: 16 positions + pad

template <int IN_DT>
__global__ __launch_bounds__(256) void gqa_decode_partial_kernel(
    const void* __restrict__ q_gate, const void* __restrict__ k_new, const void* __restrict__ v_new,
    const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w, RopeFreqs rf, float scale,
    float eps, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ positions, int max_ctx, int chunk_len, float* __restrict__ pm,
    float* __restrict__ pd, float* __restrict__ po) {
    const int c = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = positions[seq];
    // a position outside the cache is the caller's error: skip the sequence
    // (the combine writes NaN for it) rather than touch memory past the cache
    if (pos < 0 || pos >= max_ctx) return;
    const int L = pos + 1;
    if (c * chunk_len >= L) return;
    const int p_start = c * chunk_len;
    const int p_end = min(L, p_start + chunk_len);

    __shared__ float qf[8][256];
    __shared__ __attribute__((aligned(16))) uint16_t qb[8][256];
    __shared__ __attribute__((aligned(16))) uint16_t vt[4][256 * kVtStride];
    __shared__ float rcos[32], rsin[32], kf[256], red[4];
    __shared__ float wm[4][8], wd[4][8];

    // RoPE table for this position: QwenQ4ActiveExpertStreamingRunner.swift:1090-1099
    // (the inverse frequencies come from the host, computed there in fp32)
    if (t < 32) {
        const float ang = static_cast<float>(pos) * rf.f[t];
        rcos[t] = cosf(ang);
        rsin[t] = sinf(ang);
    }
    // head RMSNorm of the 8 q heads: thread -> head t/32, dims 8*(t%32)..+7
    // (deltanet.metal:599-632)
    {
        const int hl = t >> 5, j = t & 31;
        const size_t qbase = (static_cast<size_t>(seq) * 16 + kvh * 8 + hl) * 512 + 8 * j;
        float x[8], ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[i] = elem<IN_DT>::load(q_gate, qbase + i);
            ss += x[i] * x[i];
        }
        ss = group_sum<32>(ss);
        const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[hl][8 * j + i] = x[i] * inv * q_norm_w[8 * j + i];
    }
    __syncthreads();
    // partial RoPE (deltanet.metal:634-651), softmax scale, bf16
    {
        const int hl = t >> 5, j = t & 31;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = 8 * j + i;
            float v = qf[hl][d];
            if (d < 32) v = v * rcos[d] + (-qf[hl][d + 32]) * rsin[d];
            else if (d < 64) v = v * rcos[d - 32] + qf[hl][d - 32] * rsin[d - 32];
            qb[hl][d] = f32_to_bf16(v * scale);
        }
    }
    const size_t seq_base = static_cast<size_t>(seq) * max_ctx * 512 + kvh * 256;
    // the new token: k norm + RoPE, append k and v (deltanet.metal:670-689)
    if (pos >= p_start && pos < p_end) {
        const size_t kb0 = (static_cast<size_t>(seq) * 2 + kvh) * 256;
        const float kx = elem<IN_DT>::load(k_new, kb0 + t);
        const float kss = group_sum<64>(kx * kx);
        if (lane == 0) red[wave] = kss;
        __syncthreads();
        const float kinv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / 256.0f + eps);
        kf[t] = kx * kinv * k_norm_w[t];
        __syncthreads();
        float kr = kf[t];
        if (t < 32) kr = kr * rcos[t] + (-kf[t + 32]) * rsin[t];
        else if (t < 64) kr = kr * rcos[t - 32] + kf[t - 32] * rsin[t - 32];
        const size_t off = seq_base + static_cast<size_t>(pos) * 512 + t;
        k_cache[off] = f32_to_bf16(kr);
        v_cache[off] = f32_to_bf16(elem<IN_DT>::load(v_new, kb0 + t));
        __threadfence();
    }
    __syncthreads();

    // q^T operands (B of 16x16x32): col = head n (< 8 real), k = dims
    const int n = lane & 15, kb = lane >> 4;
    u32x4_t qreg[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        if (n < 8) qreg[jj] = *reinterpret_cast<const u32x4_t*>(&qb[n][32 * jj + 8 * kb]);
        else qreg[jj] = u32x4_t{0u, 0u, 0u, 0u};
    }

    float m_run = -INFINITY, d_run = 0.0f;
    f32x4_t oacc[16];
#pragma unroll
    for (int jd = 0; jd < 16; ++jd) oacc[jd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint16_t* vtw = vt[wave];
    const uint16_t* Kb = k_cache + seq_base;
    const uint16_t* Vb = v_cache + seq_base;

    // K operand rows (A of 16x16x32: position p0 + n, dims 32jj + 8kb .. +7)
    // and V rows (positions p0 + 4kb + i, dims 8(n + 16it) .. +7) of one tile.
    // K rows past the chunk end re-read its last row (masked below) and V
    // rows past it read as zero (their probability is 0, and the cache
    // beyond the sequence may hold any bit pattern, NaN included), so no
    // lane reads outside the chunk.
    auto load_tile = [&](int p0, u32x4_t (&ka)[8], u32x4_t (&va)[2][4]) {
        const uint16_t* krow = Kb + static_cast<size_t>(min(p0 + n, p_end - 1)) * 512;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) ka[jj] = *reinterpret_cast<const u32x4_t*>(krow + 32 * jj + 8 * kb);
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int pp = p0 + 4 * kb + i;
                va[it][i] = pp < p_end
                    ? *reinterpret_cast<const u32x4_t*>(Vb + static_cast<size_t>(pp) * 512 + 8 * (n + 16 * it))
                    : u32x4_t{0u, 0u, 0u, 0u};
            }
    };
    u32x4_t kn[8], vn[2][4];
    if (p_start + wave * 16 < p_end) load_tile(p_start + wave * 16, kn, vn);
    for (int p0 = p_start + wave * 16; p0 < p_end; p0 += 64) {
        u32x4_t kcur[8], vr[2][4];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) kcur[jj] = kn[jj];
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i) vr[it][i] = vn[it][i];
        if (p0 + 64 < p_end) load_tile(p0 + 64, kn, vn);   // next tile in flight
        // S^T = K Q^T
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) s = mfma_16x16x32_bf16(kcur[jj], qreg[jj], s);
        // online softmax: lane holds head n, positions p0 + 4kb + i
        float sv[4], tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = (p0 + 4 * kb + i < p_end) ? s[i] : -INFINITY;
            tmax = fmaxf(tmax, sv[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = expf(m_run - m_new);
        float pe[4], psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pe[i] = expf(sv[i] - m_new);
            psum += pe[i];
        }
        d_run = d_run * alpha + psum;
        m_run = m_new;
        if (__any(alpha != 1.0f)) {
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
            for (int jd = 0; jd < 16; ++jd)
#pragma unroll
                for (int i = 0; i < 4; ++i) oacc[jd][i] *= al[i];
        }
        const u32x2_t pa = u32x2_t{pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3])};
        // transpose V (4 positions x 8 dims per lane) into vt[dim][position]
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int dg = n + 16 * it;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int w = e >> 1;
                uint32_t lo, hi;
                if (e & 1) {
                    lo = (vr[it][0][w] >> 16) | (vr[it][1][w] & 0xffff0000u);
                    hi = (vr[it][2][w] >> 16) | (vr[it][3][w] & 0xffff0000u);
                } else {
                    lo = (vr[it][0][w] & 0xffffu) | (vr[it][1][w] << 16);
                    hi = (vr[it][2][w] & 0xffffu) | (vr[it][3][w] << 16);
                }
                *reinterpret_cast<u32x2_t*>(&vtw[(8 * dg + e) * kVtStride + 4 * kb]) = u32x2_t{lo, hi};
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O += P V: A = P (head n, positions 4kb..), B = V^T tile (dim 16jd + n)
#pragma unroll
        for (int jd = 0; jd < 16; ++jd) {
            const u32x2_t vb = *reinterpret_cast<const u32x2_t*>(&vtw[(16 * jd + n) * kVtStride + 4 * kb]);
            oacc[jd] = mfma_16x16x16_bf16(pa, vb, oacc[jd]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    d_run += __shfl_xor(d_run, 16, 64);
    d_run += __shfl_xor(d_run, 32, 64);
    if (lane < 8) {
        wm[wave][lane] = m_run;
        wd[wave][lane] = d_run;
    }
    __syncthreads();
    // merge the 4 waves (the vt tiles are free now): om[wave][head][dim]
    float* om = reinterpret_cast<float*>(&vt[0][0]);
    if (kb < 2) {
#pragma unroll
        for (int jd = 0; jd < 16; ++jd)
#pragma unroll
            for (int i = 0; i < 4; ++i) om[(wave * 8 + 4 * kb + i) * 256 + 16 * jd + n] = oacc[jd][i];
    }
    __syncthreads();
    const size_t pbase = (static_cast<size_t>(seq) * 2 + kvh) * kGqaMaxChunks + c;
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][h]);
        float D = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float e = expf(wm[w][h] - M);
            D += wd[w][h] * e;
            O += om[(w * 8 + h) * 256 + t] * e;
        }
        po[(pbase * 8 + h) * 256 + t] = O;
        if (t == 0) {
            pm[pbase * 8 + h] = M;
            pd[pbase * 8 + h] = D;
        }
    }
}

// grid (16 q heads, batch), 256 threads: attention.metal:342-377 merge, then
// the gate of deltanet.metal:700-708. Chunk weights are formed in parallel
// (one thread per chunk) and the dim loop issues 8 independent loads at a
// time.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void gqa_decode_combine_kernel(
    const void* __restrict__ q_gate, const int32_t* __restrict__ positions, int max_ctx, int chunk_len,
    const float* __restrict__ pm, const float* __restrict__ pd, const float* __restrict__ po,
    void* __restrict__ out) {
    __shared__ float es[kGqaMaxChunks], red[8];
    const int h = blockIdx.x, seq = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int kvh = h >> 3, hl = h & 7;
    const size_t qi = (static_cast<size_t>(seq) * 16 + h);
    const int pos = positions[seq];
    if (pos < 0 || pos >= max_ctx) {
        elem<OUT_DT>::store(out, qi * 256 + t, __builtin_nanf(""));
        return;
    }
    const int L = pos + 1;
    const int nc = (L + chunk_len - 1) / chunk_len;
    const size_t base = (static_cast<size_t>(seq) * 2 + kvh) * kGqaMaxChunks;
    const float m = t < nc ? pm[(base + t) * 8 + hl] : -INFINITY;
    const float d = t < nc ? pd[(base + t) * 8 + hl] : 0.0f;
    const float wmax = group_max<64>(m);
    if (lane == 0) red[wave] = wmax;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = t < nc ? expf(m - M) : 0.0f;
    if (t < kGqaMaxChunks) es[t] = e;
    const float wd = group_sum<64>(d * e);
    if (lane == 0) red[4 + wave] = wd;
    __syncthreads();
    const float D = red[4] + red[5] + red[6] + red[7];
    const float* pr = po + (base * 8 + hl) * 256 + t;   // chunk c at pr[c * 8 * 256]
    float O = 0.0f;
    int c = 0;
    for (; c + 8 <= nc; c += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = pr[static_cast<size_t>(c + u) * 2048];
#pragma unroll
        for (int u = 0; u < 8; ++u) O += v[u] * es[c + u];
    }
    for (; c < nc; ++c) O += pr[static_cast<size_t>(c) * 2048] * es[c];
    const float gate = elem<IN_DT>::load(q_gate, qi * 512 + 256 + t);
    elem<OUT_DT>::store(out, qi * 256 + t, (O / D) * sigmoid(gate));
}

// Chunk length: aim for ~2048 partial workgroups over the batch (8 per CU),
// at most kGqaMaxChunks chunks per sequence, multiples of 64 positions.
int gqa_chunk_len(int max_ctx, int batch) {
    int target = 2048 / (2 * batch);
    if (target < 1) target = 1;
    if (target > kGqaMaxChunks) target = kGqaMaxChunks;
    const int per = (max_ctx + target - 1) / target;
    const int ch = ((per + 63) / 64) * 64;
    return ch < 64 ? 64 : ch;
}

hipError_t launch_gqa_decode(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                             const void* q_gate, const void* k_new, const void* v_new,
                             qff_dtype in_dtype, void* k_cache, void* v_cache,
                             const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                             int max_ctx) {
    const int ch = gqa_chunk_len(max_ctx, batch);
    const int nc = (max_ctx + ch - 1) / ch;
    const RopeFreqs rf = rope_freqs(p->rope_theta);
    const dim3 pgrid(nc, 2, batch);
    uint16_t* kc = static_cast<uint16_t*>(k_cache);
    uint16_t* vc = static_cast<uint16_t*>(v_cache);
    {
    ProfScope prof(ctx, stream, "gqa_decode_partial");
    if (in_dtype == QFF_BF16)
        gqa_decode_partial_kernel<1><<<pgrid, 256, 0, stream>>>(q_gate, k_new, v_new, p->q_norm_w, p->k_norm_w,
                                                                rf, p->scale, p->eps, kc, vc, positions,
                                                                max_ctx, ch, ctx->gqa_m, ctx->gqa_d, ctx->gqa_o);
    else
        gqa_decode_partial_kernel<0><<<pgrid, 256, 0, stream>>>(q_gate, k_new, v_new, p->q_norm_w, p->k_norm_w,
                                                                rf, p->scale, p->eps, kc, vc, positions,
                                                                max_ctx, ch, ctx->gqa_m, ctx->gqa_d, ctx->gqa_o);
    }
    const dim3 cgrid(16, batch);
    ProfScope prof(ctx, stream, "gqa_decode_combine");
#define QFF_COMB(I, O) \
    gqa_decode_combine_kernel<I, O><<<cgrid, 256, 0, stream>>>(q_gate, positions, max_ctx, ch, ctx->gqa_m, ctx->gqa_d, ctx->gqa_o, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_COMB(1, 1); else QFF_COMB(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_COMB(0, 1); else QFF_COMB(0, 0);
    }
#undef QFF_COMB
    return hipGetLastError();
}

}  // namespace qff
