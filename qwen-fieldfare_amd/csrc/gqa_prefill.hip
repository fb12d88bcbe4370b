// gqa_prefill.hip -- causal full-attention prefill (16 q heads on 2 kv heads,
// head dim 256) for T consecutive tokens of one sequence on gfx950.
//
// The reference has no prefill kernel: each prompt token runs the decode
// path at its position (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561,
// 1076-1150), so token t attends to positions 0 .. start+t. This file
// computes all T rows at once:
//   prep   grid (token, 18 heads): head RMSNorm + partial RoPE of the 16 q
//          heads (bf16, softmax scale folded in, to workspace) and of the 2 k
//          heads (appended to the bf16 cache together with v).
//   attn   flash attention. A workgroup owns 16 query tokens x the 8 q heads
//          of one kv head (128 rows; each wave 32 rows = 2 MFMA row tiles of
//          2 tokens x 8 heads) and walks 32-position K/V tiles staged in LDS
//          (double-buffered; the next tile's global loads are in flight while
//          the current one computes). S^T = K Q^T on 16x16x32 bf16 MFMAs (one
//          K operand read feeds both row tiles), online softmax in fp32
//          registers, then O += P V with 16x16x32 MFMAs whose 32-deep k runs
//          over the tile's positions in the order the S^T registers hold them.
//          Query blocks are issued last-first so the longest rows start
//          earliest. The epilogue divides by the row sums and applies the
//          sigmoid gate.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kPfQB = 16;       // query tokens per workgroup
constexpr int kPfKT = 32;       // K/V positions per tile
constexpr int kKStride = 264;   // bf16 per K row in LDS: 256 + 8 pad (528 B)
constexpr int kVStride = 36;    // bf16 per transposed V row: 32 + 4 pad (72 B)

// grid (T, 18): y < 16 -> q head y, else kv head y - 16. 256 threads (dims).
template <int IN_DT>
__global__ __launch_bounds__(256) void gqa_prefill_prep_kernel(
    const void* __restrict__ q_gate, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w, RopeFreqs rf, float scale,
    float eps, int start, uint16_t* __restrict__ qb, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
    __shared__ float xs[256], red[4];
    const int tok = blockIdx.x, hs = blockIdx.y, t = threadIdx.x;
    const int pos = start + tok;
    const bool is_q = hs < 16;
    const float x = is_q ? elem<IN_DT>::load(q_gate, (static_cast<size_t>(tok) * 16 + hs) * 512 + t)
                         : elem<IN_DT>::load(k, (static_cast<size_t>(tok) * 2 + (hs - 16)) * 256 + t);
    const float ss = group_sum<64>(x * x);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / 256.0f + eps);
    xs[t] = x * inv * (is_q ? q_norm_w[t] : k_norm_w[t]);
    __syncthreads();
    float r = xs[t];
    if (t < 64) {
        const int i = t & 31;
        const float ang = static_cast<float>(pos) * rf.f[i];
        const float c = cosf(ang), s = sinf(ang);
        r = (t < 32) ? r * c + (-xs[t + 32]) * s : r * c + xs[t - 32] * s;
    }
    if (is_q) {
        qb[(static_cast<size_t>(tok) * 16 + hs) * 256 + t] = f32_to_bf16(r * scale);
    } else {
        const int kvh = hs - 16;
        const size_t off = (static_cast<size_t>(pos) * 2 + kvh) * 256 + t;
        k_cache[off] = f32_to_bf16(r);
        v_cache[off] = f32_to_bf16(elem<IN_DT>::load(v, (static_cast<size_t>(tok) * 2 + kvh) * 256 + t));
    }
}

struct TileRegs {
    u32x4_t k[4];
    u32x4_t v[4];
};

// Thread t loads K row t/8 (dims 32*(t%8) .. +31) and V rows 4*(t/32) .. +3
// (dims 8*(t%32) .. +7) of the tile starting at p0; rows at or past kv_end
// read as zero.
__device__ __forceinline__ void tile_load(TileRegs& r, const uint16_t* __restrict__ kc,
                                          const uint16_t* __restrict__ vc, int kvh, int p0, int kv_end,
                                          int t) {
    const int kp = p0 + (t >> 3);
    const uint16_t* kr = kc + (static_cast<size_t>(kp) * 2 + kvh) * 256 + 32 * (t & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r.k[i] = kp < kv_end ? *reinterpret_cast<const u32x4_t*>(kr + 8 * i) : u32x4_t{0u, 0u, 0u, 0u};
    const int vp = p0 + 4 * (t >> 5);
    const int dg = t & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r.v[i] = (vp + i < kv_end)
                     ? *reinterpret_cast<const u32x4_t*>(vc + (static_cast<size_t>(vp + i) * 2 + kvh) * 256 + 8 * dg)
                     : u32x4_t{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ void tile_store(const TileRegs& r, uint16_t* __restrict__ ks,
                                           uint16_t* __restrict__ vt, int t) {
    uint16_t* kd = ks + (t >> 3) * kKStride + 32 * (t & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(kd + 8 * i) = r.k[i];
    // transpose 4 positions x 8 dims into vt[dim][position]
    const int pg = t >> 5, dg = t & 31;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        uint32_t lo, hi;
        if (e & 1) {
            lo = (r.v[0][w] >> 16) | (r.v[1][w] & 0xffff0000u);
            hi = (r.v[2][w] >> 16) | (r.v[3][w] & 0xffff0000u);
        } else {
            lo = (r.v[0][w] & 0xffffu) | (r.v[1][w] << 16);
            hi = (r.v[2][w] & 0xffffu) | (r.v[3][w] << 16);
        }
        *reinterpret_cast<u32x2_t*>(vt + (8 * dg + e) * kVStride + 4 * pg) = u32x2_t{lo, hi};
    }
}

// grid (ceil(T/16), 2 kv heads), 256 threads.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void gqa_prefill_attn_kernel(
    const uint16_t* __restrict__ qb, const void* __restrict__ q_gate, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int start, int T, void* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kPfKT * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][256 * kVStride];
    const int nqb = (T + kPfQB - 1) / kPfQB;
    const int q_blk = nqb - 1 - static_cast<int>(blockIdx.x);
    const int kvh = blockIdx.y;
    const int t0 = q_blk * kPfQB;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;

    // this lane's q row in each row tile r: token t0 + 4w + 2r + n/8, head n%8
    u32x4_t qreg[2][8];
    int lim[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int tok = min(t0 + 4 * wave + 2 * r + (n >> 3), T - 1);
        lim[r] = start + tok;
        const uint16_t* qrow = qb + (static_cast<size_t>(tok) * 16 + kvh * 8 + (n & 7)) * 256;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) qreg[r][jj] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * jj + 8 * kb);
    }
    const int kv_end = start + min(T, t0 + kPfQB);
    const int ntiles = (kv_end + kPfKT - 1) / kPfKT;

    float m_run[2] = {-INFINITY, -INFINITY}, d_run[2] = {0.0f, 0.0f};
    f32x4_t oacc[2][16];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int jd = 0; jd < 16; ++jd) oacc[r][jd] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    TileRegs regs;
    tile_load(regs, k_cache, v_cache, kvh, 0, kv_end, t);
    tile_store(regs, Ks[0], Vt[0], t);
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ntiles;
        if (more) tile_load(regs, k_cache, v_cache, kvh, (kt + 1) * kPfKT, kv_end, t);
        const int p0 = kt * kPfKT;
        // S^T = K Q^T for two 16-position tiles and both row tiles
        f32x4_t s[2][2];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int pt = 0; pt < 2; ++pt) s[r][pt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const u32x4_t a =
                    *reinterpret_cast<const u32x4_t*>(&Ks[cur][(16 * pt + n) * kKStride + 32 * jj + 8 * kb]);
                s[0][pt] = mfma_16x16x32_bf16(a, qreg[0][jj], s[0][pt]);
                s[1][pt] = mfma_16x16x32_bf16(a, qreg[1][jj], s[1][pt]);
            }
        // online softmax; lane holds q row n, positions p0 + 16pt + 4kb + i
        u32x4_t pa[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            float sv[2][4], tmax = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int p = p0 + 16 * pt + 4 * kb + i;
                    sv[pt][i] = (p <= lim[r]) ? s[r][pt][i] : -INFINITY;
                    tmax = fmaxf(tmax, sv[pt][i]);
                }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float m_new = fmaxf(m_run[r], tmax);
            const float alpha = expf(m_run[r] - m_new);
            float pe[2][4], psum = 0.0f;
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pe[pt][i] = expf(sv[pt][i] - m_new);
                    psum += pe[pt][i];
                }
            d_run[r] = d_run[r] * alpha + psum;
            m_run[r] = m_new;
            if (__any(alpha != 1.0f)) {
                float al[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
                for (int jd = 0; jd < 16; ++jd)
#pragma unroll
                    for (int i = 0; i < 4; ++i) oacc[r][jd][i] *= al[i];
            }
            // A operand of O += P V: k = 8kb + j <-> position 16(j/4) + 4kb + j%4
            pa[r] = u32x4_t{pack_bf16x2(pe[0][0], pe[0][1]), pack_bf16x2(pe[0][2], pe[0][3]),
                            pack_bf16x2(pe[1][0], pe[1][1]), pack_bf16x2(pe[1][2], pe[1][3])};
        }
        // O += P V, B operand = V^T rows (dim 16jd + n), the same position order
#pragma unroll
        for (int jd = 0; jd < 16; ++jd) {
            const uint16_t* vrow = &Vt[cur][(16 * jd + n) * kVStride];
            const u32x2_t v0 = *reinterpret_cast<const u32x2_t*>(vrow + 4 * kb);
            const u32x2_t v1 = *reinterpret_cast<const u32x2_t*>(vrow + 16 + 4 * kb);
            const u32x4_t b = u32x4_t{v0[0], v0[1], v1[0], v1[1]};
            oacc[0][jd] = mfma_16x16x32_bf16(pa[0], b, oacc[0][jd]);
            oacc[1][jd] = mfma_16x16x32_bf16(pa[1], b, oacc[1][jd]);
        }
        if (more) tile_store(regs, Ks[cur ^ 1], Vt[cur ^ 1], t);
        __syncthreads();
    }

    // epilogue: O / d * sigmoid(gate); oacc[r][jd][i] = O[row 4kb+i][dim 16jd+n]
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        float d = d_run[r];
        d += __shfl_xor(d, 16, 64);
        d += __shfl_xor(d, 32, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * kb + i;
            const float inv_d = 1.0f / __shfl(d, row, 64);
            const int tok = t0 + 4 * wave + 2 * r + (row >> 3);
            if (tok >= T) continue;
            const int h = kvh * 8 + (row & 7);
            const size_t qi = static_cast<size_t>(tok) * 16 + h;
#pragma unroll
            for (int jd = 0; jd < 16; ++jd) {
                const int dim = 16 * jd + n;
                const float g = elem<IN_DT>::load(q_gate, qi * 512 + 256 + dim);
                elem<OUT_DT>::store(out, qi * 256 + dim, oacc[r][jd][i] * inv_d * sigmoid(g));
            }
        }
    }
}

hipError_t launch_gqa_prefill(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                              const void* q_gate, const void* k, const void* v, qff_dtype in_dtype,
                              void* k_cache, void* v_cache, int start_pos, void* out,
                              qff_dtype out_dtype, int T, int) {
    // the bf16 q rows [T][16][256] reuse the DeltaNet prefill staging buffer
    uint16_t* qb = ctx->gqa_qb;
    uint16_t* kc = static_cast<uint16_t*>(k_cache);
    uint16_t* vc = static_cast<uint16_t*>(v_cache);
    const RopeFreqs rf = rope_freqs(p->rope_theta);
    {
        ProfScope prof(ctx, stream, "gqa_prefill_prep");
        if (in_dtype == QFF_BF16)
            gqa_prefill_prep_kernel<1><<<dim3(T, 18), 256, 0, stream>>>(q_gate, k, v, p->q_norm_w, p->k_norm_w, rf,
                                                                        p->scale, p->eps, start_pos, qb, kc, vc);
        else
            gqa_prefill_prep_kernel<0><<<dim3(T, 18), 256, 0, stream>>>(q_gate, k, v, p->q_norm_w, p->k_norm_w, rf,
                                                                        p->scale, p->eps, start_pos, qb, kc, vc);
    }
    const dim3 grid((T + kPfQB - 1) / kPfQB, 2);
    ProfScope prof(ctx, stream, "gqa_prefill_attn");
#define QFF_PFA(I, O) gqa_prefill_attn_kernel<I, O><<<grid, 256, 0, stream>>>(qb, q_gate, kc, vc, start_pos, T, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_PFA(1, 1); else QFF_PFA(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_PFA(0, 1); else QFF_PFA(0, 0);
    }
#undef QFF_PFA
    return hipGetLastError();
}

}  // namespace qff
