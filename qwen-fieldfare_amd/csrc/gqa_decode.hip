// gqa_decode.hip -- full-attention decode (16 q heads on 2 kv heads, head dim
// 256, bf16 token-major KV cache) for a batch of sequences on gfx950.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1076-1150 runs split
// q/gate, head RMSNorm, host RoPE tables + RoPE, the f16 KV append, a cast of
// q to half, Attention.encodeFull (split-KV partial + combine,
// attention.metal:134-224, 342-377; geometry Attention.swift:129-157) and the
// gate (deltanet.metal:700-708), one q head per threadgroup.
//
// Here the eight q heads that share a kv head run in the same wave, so every
// K/V byte is read from HBM once, and both products run on the matrix cores:
//   partial  grid (chunk group, kv head, sequence), four waves, one chunk
//            each. The workgroup normalises and rotates the 8 q heads into
//            LDS once (bf16, softmax scale and log2 e folded in); the wave
//            whose chunk holds the new token also normalises/rotates k,
//            appends k and v to the cache and keeps both in LDS for its own
//            use. Each wave then walks 16-position tiles with the next tile's
//            K and V rows already in flight (two register stages): S^T = K Q^T
//            with 8 MFMA 16x16x32 (K rows straight from HBM, 16 B per lane),
//            base-2 online softmax per head whose running max is raised only
//            past 2^8 (so O is rarely rescaled), the V tile copied row-major
//            into LDS and read back as MFMA B operands with the gfx950
//            transpose read (ds_read_b64_tr_b16), O += P V with 16 MFMA
//            16x16x16, and one (m, d, o[8][256]) partial per chunk (m in
//            base-2 units).
//   combine  grid (q head, sequence): merges the chunk partials and applies
//            out = attn * sigmoid(gate).
// Lengths come from the device `positions` array, so no host sync is needed;
// waves past a sequence's last chunk exit at once.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kDecTile = 16;          // positions per MFMA tile
constexpr int kVRowStride = 264;      // bf16 per V row in LDS: 256 + 8 pad (528 B)


struct DecTile {
    u32x4_t k[8], v[8];
};

// grid (2 kv heads x ceil(chunks / NW), 1, batch), 64 NW threads: the kv
// head is the fastest-varying block index, so the two heads' workgroups of a
// chunk group are dispatched together and stream the interleaved halves of
// the same cache records at the same time; wave w takes chunk NW * group + w. NW = 4 (long chunks) shares one q preparation
// between four chunks and keeps the next tile's loads in flight (two register
// stages, two waves per SIMD); NW = 1 (short chunks, small batches) loads
// each tile as it goes and keeps three or more single-wave workgroups per
// SIMD resident instead.
template <int IN_DT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 2 : 3)))
void gqa_decode_partial_kernel(
    const void* __restrict__ q_gate, const void* __restrict__ k_new, const void* __restrict__ v_new,
    const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w, RopeFreqs rf, float scale,
    float eps, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ positions, int max_ctx, int chunk_len, int cstride, float* __restrict__ pm,
    float* __restrict__ pd, float* __restrict__ po) {
    const int kvh = blockIdx.x & 1, grp = blockIdx.x >> 1, seq = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = NW * grp + wave;
    const int pos = positions[seq];
    // a position outside the cache is the caller's error: skip the sequence
    // (the combine writes NaN for it) rather than touch memory past the cache
    if (pos < 0 || pos >= max_ctx) return;
    const int L = pos + 1;
    if (NW * grp * chunk_len >= L) return;   // the whole group is past the end
    const int p_start = c * chunk_len;
    const int p_end = min(L, p_start + chunk_len);

    __shared__ __attribute__((aligned(16))) uint16_t qs[8][256];                           // 4 KB
    __shared__ __attribute__((aligned(16))) uint16_t vs[NW][kDecTile * kVRowStride];  // NW x 8.25 KB
    __shared__ __attribute__((aligned(16))) uint16_t knew[256], vnew[256];
    __shared__ float2 rcs[32];   // (cos, sin) of pos * f[i]

    if (t < 32) {
        const float ang = static_cast<float>(pos) * rf.f[t];
        rcs[t] = make_float2(cosf(ang), sinf(ang));
    }
    __syncthreads();

    // ---- q: head RMSNorm + partial RoPE + scale, bf16 into LDS ---------------
    // (deltanet.metal:599-651; RoPE angles as QwenQ4ActiveExpertStreamingRunner
    // .swift:1090-1099 with host-computed inverse frequencies). Thread -> head
    // u/32, dims 8*(u%32) .. +7 for u = t, t + 64 NW, ...; the RoPE pair
    // (d, d^32) of dims < 64 sits in threads 4 apart.
    for (int u = t; u < 256; u += 64 * NW) {
        const int hl = u >> 5, j = u & 31;
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
        for (int i = 0; i < 8; ++i) x[i] = x[i] * inv * q_norm_w[8 * j + i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = 8 * j + i;
            const float partner = __shfl_xor(x[i], 4, 64);   // d +- 32 (used when d < 64)
            if (d < 64) {
                const float2 r = rcs[d & 31];
                x[i] = (d < 32) ? x[i] * r.x + (-partner) * r.y : x[i] * r.x + partner * r.y;
            }
        }
        const float qscale = scale * 1.44269504088896341f;
#pragma unroll
        for (int i = 0; i < 8; i += 2)
            *reinterpret_cast<uint32_t*>(&qs[hl][8 * j + i]) = pack_bf16x2(x[i] * qscale, x[i + 1] * qscale);
    }
    // ---- the new token (only the wave whose chunk holds it): k norm + RoPE,
    // append k and v to the cache (deltanet.metal:670-689), keep both in LDS
    // so the wave never reads back its own global stores.
    const bool has_new = pos >= p_start && pos < p_end;
    const size_t seq_base = static_cast<size_t>(seq) * max_ctx * 512 + kvh * 256;
    if (has_new) {
        const size_t kb0 = (static_cast<size_t>(seq) * 2 + kvh) * 256 + 4 * lane;
        float kx[4], vx[4], ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kx[i] = elem<IN_DT>::load(k_new, kb0 + i);
            vx[i] = elem<IN_DT>::load(v_new, kb0 + i);
            ss += kx[i] * kx[i];
        }
        ss = group_sum<64>(ss);
        const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
        for (int i = 0; i < 4; ++i) kx[i] = kx[i] * inv * k_norm_w[4 * lane + i];
        // dims 4*lane .. +3; RoPE partner of dim d < 32 is d + 32 = lane + 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float up = __shfl_down(kx[i], 8, 64), dn = __shfl_up(kx[i], 8, 64);
            const int d = 4 * lane + i;
            if (d < 64) {
                const float2 r = rcs[d & 31];
                kx[i] = (d < 32) ? kx[i] * r.x + (-up) * r.y : kx[i] * r.x + dn * r.y;
            }
        }
        const uint32_t k01 = pack_bf16x2(kx[0], kx[1]), k23 = pack_bf16x2(kx[2], kx[3]);
        const uint32_t v01 = pack_bf16x2(vx[0], vx[1]), v23 = pack_bf16x2(vx[2], vx[3]);
        *reinterpret_cast<u32x2_t*>(&knew[4 * lane]) = u32x2_t{k01, k23};
        *reinterpret_cast<u32x2_t*>(&vnew[4 * lane]) = u32x2_t{v01, v23};
        const size_t off = seq_base + static_cast<size_t>(pos) * 512 + 4 * lane;
        *reinterpret_cast<u32x2_t*>(k_cache + off) = u32x2_t{k01, k23};
        *reinterpret_cast<u32x2_t*>(v_cache + off) = u32x2_t{v01, v23};
    }
    __syncthreads();
    if (p_start >= L) return;

    const int n = lane & 15, kb = lane >> 4;
    // q^T (B of 16x16x32): col = head n (< 8 real), k = dims 32jj + 8kb .. +7,
    // read from LDS per tile (registers are kept for the two tile stages)
    const uint16_t* qrow = &qs[n & 7][8 * kb];
    uint16_t* vsw = vs[wave];
    constexpr float kLazy = 8.0f;   // raise the running max only past 2^8

    float m_run = -INFINITY, d_run = 0.0f;
    f32x4_t oacc[16];
#pragma unroll
    for (int jd = 0; jd < 16; ++jd) oacc[jd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint16_t* Kb = k_cache + seq_base;
    const uint16_t* Vb = v_cache + seq_base;

    // K rows p0 + n (A of 16x16x32) and V rows p0 + 2i + lane/32 (dims
    // 8*(lane%32) .. +7). Rows past the chunk end re-read its last row: their
    // scores are masked to -inf, so they enter P V with probability 0 times
    // finite data (the cache past the sequence may hold any bit pattern, NaN
    // included, and is never read). The loads are unconditional so the
    // compiler's vmcnt bookkeeping stays exact across the two stages.
    auto load = [&](DecTile& tl, int p0) {
        const uint16_t* krow = Kb + static_cast<size_t>(min(p0 + n, p_end - 1)) * 512;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) tl.k[jj] = *reinterpret_cast<const u32x4_t*>(krow + 32 * jj + 8 * kb);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int vp = min(p0 + 2 * i + (lane >> 5), p_end - 1);
            tl.v[i] = *reinterpret_cast<const u32x4_t*>(Vb + static_cast<size_t>(vp) * 512 + 8 * (lane & 31));
        }
    };
    auto compute = [&](DecTile& tl, int p0) {
        if (has_new && min(p0 + n, p_end - 1) == pos) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) tl.k[jj] = *reinterpret_cast<const u32x4_t*>(&knew[32 * jj + 8 * kb]);
        }
        // S^T = K Q^T
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const u32x4_t qv = n < 8 ? *reinterpret_cast<const u32x4_t*>(qrow + 32 * jj) : u32x4_t{0u, 0u, 0u, 0u};
            s = mfma_16x16x32_bf16(tl.k[jj], qv, s);
        }
        // V tile row-major into LDS (the new token's row from LDS as well)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 2 * i + (lane >> 5);
            u32x4_t v = tl.v[i];
            if (has_new && p0 + r == pos) v = *reinterpret_cast<const u32x4_t*>(&vnew[8 * (lane & 31)]);
            *reinterpret_cast<u32x4_t*>(&vsw[r * kVRowStride + 8 * (lane & 31)]) = v;
        }
        // online softmax (base 2); lane holds head n, positions p0 + 4kb + i
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (p0 + 4 * kb + i >= p_end) s[i] = -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        if (__any(tmax > m_run + kLazy)) {
            const float m_new = tmax > m_run + kLazy ? tmax : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            d_run *= alpha;
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
            for (int jd = 0; jd < 16; ++jd)
#pragma unroll
                for (int i = 0; i < 4; ++i) oacc[jd][i] *= al[i];
        }
        float pe[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pe[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
            d_run += pe[i];
        }
        // A of O += P V (16x16x16): row = head n, k = positions 4kb .. +3
        const u32x2_t pa = u32x2_t{pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3])};
        // B = V^T block straight from the row-major tile with a transpose read:
        // source lane (group kb, s = n) points at row 4kb + n/4, dims
        // 16jd + 4(n%4) .. +3, and receives V[4kb + k][16jd + n], k = 0..3.
        __builtin_amdgcn_wave_barrier();
        const uint16_t* vsrc = &vsw[(4 * kb + (n >> 2)) * kVRowStride + 4 * (n & 3)];
#pragma unroll
        for (int jd = 0; jd < 16; ++jd) oacc[jd] = mfma_16x16x16_bf16(pa, lds_read_tr16(vsrc + 16 * jd), oacc[jd]);
        __builtin_amdgcn_wave_barrier();
    };
    if (NW == 4) {
        DecTile ta, tb;
        load(ta, p_start);
        int p0 = p_start;
        for (; p0 + kDecTile < p_end; p0 += 2 * kDecTile) {
            load(tb, p0 + kDecTile);
            compute(ta, p0);
            load(ta, p0 + 2 * kDecTile);
            compute(tb, p0 + kDecTile);
        }
        if (p0 < p_end) compute(ta, p0);
    } else {
        for (int p0 = p_start; p0 < p_end; p0 += kDecTile) {
            DecTile ta;
            load(ta, p0);
            compute(ta, p0);
        }
    }
    // ---- partial (m, d, o) of this chunk; oacc[jd][i] = O[head 4kb+i][dim 16jd+n]
    d_run += __shfl_xor(d_run, 16, 64);
    d_run += __shfl_xor(d_run, 32, 64);
    const size_t pbase = (static_cast<size_t>(seq) * 2 + kvh) * cstride + c;
    if (lane < 8) {
        pm[pbase * 8 + lane] = m_run;
        pd[pbase * 8 + lane] = d_run;
    }
    if (kb < 2) {
        float* orow = po + pbase * 8 * 256;
#pragma unroll
        for (int jd = 0; jd < 16; ++jd)
#pragma unroll
            for (int i = 0; i < 4; ++i) orow[(4 * kb + i) * 256 + 16 * jd + n] = oacc[jd][i];
    }
}

// grid (16 q heads, batch), 512 threads: attention.metal:342-377 merge, then
// the gate of deltanet.metal:700-708. Chunk weights are formed one thread per
// chunk; then wave w sums chunks w, w+8, ... for all 256 dims (a float4 per
// lane) so each lane has few dependent loads in flight, and the 8 wave sums
// are added in LDS in a fixed order.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(512) void gqa_decode_combine_kernel(
    const void* __restrict__ q_gate, const int32_t* __restrict__ positions, int max_ctx, int chunk_len,
    int cstride, const float* __restrict__ pm, const float* __restrict__ pd, const float* __restrict__ po,
    void* __restrict__ out) {
    __shared__ float es[kGqaMaxChunks], red[16];
    __shared__ __attribute__((aligned(16))) float osum[8][256];
    const int h = blockIdx.x, seq = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int kvh = h >> 3, hl = h & 7;
    const size_t qi = (static_cast<size_t>(seq) * 16 + h);
    const int pos = positions[seq];
    if (pos < 0 || pos >= max_ctx) {
        if (t < 256) elem<OUT_DT>::store(out, qi * 256 + t, __builtin_nanf(""));
        return;
    }
    const int L = pos + 1;
    const int nc = (L + chunk_len - 1) / chunk_len;
    const size_t base = (static_cast<size_t>(seq) * 2 + kvh) * cstride;
    const float m = t < nc ? pm[(base + t) * 8 + hl] : -INFINITY;
    const float d = t < nc ? pd[(base + t) * 8 + hl] : 0.0f;
    const float wmax = group_max<64>(m);
    if (lane == 0) red[wave] = wmax;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) M = fmaxf(M, red[w]);
    const float e = t < nc ? __builtin_amdgcn_exp2f(m - M) : 0.0f;   // m are base-2 maxima
    if (t < kGqaMaxChunks) es[t] = e;
    const float wd = group_sum<64>(d * e);
    if (lane == 0) red[8 + wave] = wd;
    __syncthreads();
    const float4* pr = reinterpret_cast<const float4*>(po + (base * 8 + hl) * 256) + lane;  // chunk c at pr[c*512]
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int c = wave;
    for (; c + 24 < nc; c += 32) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = pr[static_cast<size_t>(c + 8 * u) * 512];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float w = es[c + 8 * u];
            acc.x += v[u].x * w; acc.y += v[u].y * w; acc.z += v[u].z * w; acc.w += v[u].w * w;
        }
    }
    for (; c < nc; c += 8) {
        const float4 v = pr[static_cast<size_t>(c) * 512];
        const float w = es[c];
        acc.x += v.x * w; acc.y += v.y * w; acc.z += v.z * w; acc.w += v.w * w;
    }
    reinterpret_cast<float4*>(osum[wave])[lane] = acc;
    __syncthreads();
    if (t < 256) {
        float D = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            D += red[8 + w];
            O += osum[w][t];
        }
        const float gate = elem<IN_DT>::load(q_gate, qi * 512 + 256 + t);
        elem<OUT_DT>::store(out, qi * 256 + t, (O / D) * sigmoid(gate));
    }
}

// Chunks per (sequence, kv head) available to a call of this batch: the
// workspace's partial slots spread over the batch, at most kGqaMaxChunks.
int gqa_chunk_cap(const qff_ctx_cfg& cfg, int batch) {
    const int cap = gqa_slots(cfg) / (2 * batch);
    return cap < kGqaMaxChunks ? cap : kGqaMaxChunks;
}

// Chunk length: aim for ~4096 one-wave partial workgroups over the batch
// (16 per CU), at most `cap` chunks per sequence, multiples of 64 positions
// (4 MFMA tiles).
int gqa_chunk_len(int max_ctx, int batch, int cap) {
    int target = 4096 / (2 * batch);
    if (target < 1) target = 1;
    if (target > cap) target = cap;
    const int per = (max_ctx + target - 1) / target;
    const int ch = ((per + 63) / 64) * 64;
    return ch < 64 ? 64 : ch;
}

hipError_t launch_gqa_decode(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                             const void* q_gate, const void* k_new, const void* v_new,
                             qff_dtype in_dtype, void* k_cache, void* v_cache,
                             const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                             int max_ctx) {
    const int cap = gqa_chunk_cap(ctx->cfg, batch);
    const int ch = gqa_chunk_len(max_ctx, batch, cap);
    const int nc = (max_ctx + ch - 1) / ch;
    const RopeFreqs rf = rope_freqs(p->rope_theta);
    uint16_t* kc = static_cast<uint16_t*>(k_cache);
    uint16_t* vc = static_cast<uint16_t*>(v_cache);
    {
        ProfScope prof(ctx, stream, "gqa_decode_partial");
        const bool grouped = ch >= 256;
#define QFF_PART(I, W)                                                                                     \
    gqa_decode_partial_kernel<I, W><<<dim3(2 * ((nc + W - 1) / W), 1, batch), 64 * W, 0, stream>>>(              \
        q_gate, k_new, v_new, p->q_norm_w, p->k_norm_w, rf, p->scale, p->eps, kc, vc, positions, max_ctx, ch, cap, \
        ctx->gqa_m, ctx->gqa_d, ctx->gqa_o)
        if (in_dtype == QFF_BF16) {
            if (grouped) QFF_PART(1, 4); else QFF_PART(1, 1);
        } else {
            if (grouped) QFF_PART(0, 4); else QFF_PART(0, 1);
        }
#undef QFF_PART
    }
    const dim3 cgrid(16, batch);
    ProfScope prof(ctx, stream, "gqa_decode_combine");
#define QFF_COMB(I, O) \
    gqa_decode_combine_kernel<I, O><<<cgrid, 512, 0, stream>>>(q_gate, positions, max_ctx, ch, cap, ctx->gqa_m, ctx->gqa_d, ctx->gqa_o, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_COMB(1, 1); else QFF_COMB(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_COMB(0, 1); else QFF_COMB(0, 0);
    }
#undef QFF_COMB
    return hipGetLastError();
}

}  // namespace qff
