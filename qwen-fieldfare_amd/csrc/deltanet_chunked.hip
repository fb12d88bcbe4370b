// deltanet_chunked.hip -- the chunked (WY / UT) form of the gated delta rule
// for DeltaNet prefill, chunk C = 64, on gfx950 matrix cores.
//
// The reference runs prompts through the per-token recurrence
// (QwenDeltaNetKernel.swift:73-125, deltanet.metal:307-335, fed token by
// token at QwenQ4ActiveExpertStreamingRunner.swift:1545-1561). For one value
// head and one chunk of tokens 1..C with initial state S0 [v x k], cumulative
// log gates G_i = sum_{j<=i} log g_j and the recurrence
//   S_i = g_i S_{i-1} + u_i k_i^T,  u_i = beta_i (v_i - g_i S_{i-1} k_i),
// unrolling gives the chunk identities this file evaluates:
//   A_ij = beta_i e^{G_i - G_j} (k_i . k_j)  (j < i),     T = (I + A)^-1
//   W = T (beta e^G K),  U~ = T (beta V),  U = U~ - W S0^T
//   O = (e^G Q) S0^T + (e^{G_i - G_j} [j <= i] Q K^T) U
//   S_C = e^{G_C} S0 + U^T (e^{G_C - G} K)
// (tests/test_oracle_deltanet.py checks them against the sequential
// recurrence in fp64).
//
// Two kernels:
//   dn_chunk_local_kernel  one workgroup per (chunk, value head), all chunks
//       at once: A from K K^T, P = e^{G_i-G_j}[j<=i] Q K^T, T = (I + A)^-1
//       in 16x16 blocks (diagonal blocks by substitution, the rest on fp32
//       MFMAs, four waves in parallel), then W and U~; W, U~, P, the scaled
//       Q~ = e^G Q and K~ = e^{G_C - G} K (all split into bf16 hi/lo) and G
//       go to workspace.
//   dn_chunk_state_kernel  one workgroup per (32-row block of the state,
//       value head) walks the chunks in order with its state slice in
//       registers: U = U~ - W S^T, O = Q~ S^T + P U, S = e^{G_C} S + U^T K~.
// Every product runs as bf16x3 on v_mfma_f32_16x16x32_bf16 (a b ~ a_hi b_hi
// + a_hi b_lo + a_lo b_hi, ~2^-16 relative per product), which keeps the
// fp32 state within 1e-4 of the sequential fp32 recurrence; plain bf16
// operands would not.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kC = 64;      // chunk length
constexpr int kLD = 136;    // bf16 row stride of [64][128] LDS tiles (128 + 8)
constexpr int kLT = 72;     // bf16 row stride of [64][64] LDS tiles (64 + 8)

// grid (ceil(T/64), 32 value heads), 256 threads.
__global__ __launch_bounds__(256) void dn_chunk_local_kernel(
    int T, const float* __restrict__ pq, const float* __restrict__ pk, const float* __restrict__ pv,
    const float* __restrict__ plg, const float* __restrict__ pbeta, uint16_t* __restrict__ wh,
    uint16_t* __restrict__ wl, uint16_t* __restrict__ uh, uint16_t* __restrict__ ul, uint16_t* __restrict__ ph,
    uint16_t* __restrict__ pl, float* __restrict__ gout, uint16_t* __restrict__ qth, uint16_t* __restrict__ qtl,
    uint16_t* __restrict__ kth, uint16_t* __restrict__ ktl) {
    const int c = blockIdx.x, h = blockIdx.y, kh = h >> 1;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int t0 = c * kC;
    const int nv = min(kC, T - t0);
    const size_t ch = static_cast<size_t>(c) * 32 + h;

    __shared__ __attribute__((aligned(16))) uint16_t Kh[kC * kLD], Kl[kC * kLD];
    __shared__ __attribute__((aligned(16))) uint16_t Qh[kC * kLD], Ql[kC * kLD];   // Q, later X = beta e^G K
    __shared__ __attribute__((aligned(16))) uint16_t Vh[kC * kLD], Vl[kC * kLD];   // beta V
    __shared__ __attribute__((aligned(16))) uint16_t Th[kC * kLT], Tl[kC * kLT];
    __shared__ float Am[kC * 65];
    __shared__ float G[kC], Bt[kC];

    // gates: G = inclusive prefix sum of log g over the chunk; padded tokens
    // have log g = 0 and beta = 0, so they change nothing
    if (wave == 0) {
        const bool ok = lane < nv;
        float x = ok ? plg[static_cast<size_t>(t0 + lane) * 32 + h] : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        G[lane] = x;
        Bt[lane] = ok ? pbeta[static_cast<size_t>(t0 + lane) * 32 + h] : 0.0f;
        gout[ch * kC + lane] = x;
    }
    // K and Q rows of the key head: thread -> row t/4, dims 32*(t%4) .. +31
    const int r = t >> 2, d0 = 32 * (t & 3);
    {
        const float4* ks = reinterpret_cast<const float4*>(pk + (static_cast<size_t>(t0 + r) * 16 + kh) * 128 + d0);
        const float4* qs = reinterpret_cast<const float4*>(pq + (static_cast<size_t>(t0 + r) * 16 + kh) * 128 + d0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 kv = r < nv ? ks[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 qv = r < nv ? qs[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            store_split4(Kh, Kl, r * kLD + d0 + 4 * i, kv.x, kv.y, kv.z, kv.w);
            store_split4(Qh, Ql, r * kLD + d0 + 4 * i, qv.x, qv.y, qv.z, qv.w);
        }
    }
    __syncthreads();
    {
        const float b = Bt[r];
        const float4* vs = reinterpret_cast<const float4*>(pv + (static_cast<size_t>(t0 + r) * 32 + h) * 128 + d0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 vv = r < nv ? vs[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            store_split4(Vh, Vl, r * kLD + d0 + 4 * i, b * vv.x, b * vv.y, b * vv.z, b * vv.w);
        }
    }
    // K K^T -> A (strictly lower, scaled), Q K^T -> P (lower incl. diagonal)
#pragma unroll
    for (int cj = 0; cj < 4; ++cj) {
        const f32x4_t zero = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const f32x4_t kk = mma_nt_x3<128>(zero, Kh + 16 * wave * kLD, Kl + 16 * wave * kLD, kLD,
                                          Kh + 16 * cj * kLD, Kl + 16 * cj * kLD, kLD, lane);
        const f32x4_t qk = mma_nt_x3<128>(zero, Qh + 16 * wave * kLD, Ql + 16 * wave * kLD, kLD,
                                          Kh + 16 * cj * kLD, Kl + 16 * cj * kLD, kLD, lane);
        const int j = 16 * cj + n;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int i = 16 * wave + 4 * kb + ii;
            const float decay = j <= i ? expf(G[i] - G[j]) : 0.0f;
            Am[i * 65 + j] = j < i ? Bt[i] * decay * kk[ii] : 0.0f;
            uint16_t hh, ll;
            split_bf16(decay * qk[ii], hh, ll);
            ph[(ch * kC + i) * kC + j] = hh;
            pl[(ch * kC + i) * kC + j] = ll;
        }
    }
    __syncthreads();
    // T = (I + A)^-1 (lower unitriangular) in 16x16 blocks, fp32:
    //   diagonal blocks by forward substitution, one wave each;
    //   T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj for i > j, wave j walking
    //   column block j downwards (fp32 MFMA 16x16x4).
    float* Tm = reinterpret_cast<float*>(Qh);          // [64][65] fp32 (Q is consumed)
    float* scr = reinterpret_cast<float*>(Ql) + wave * (16 * 17);
    {
        const int bi = wave;
        if (lane < 16) {
            float tc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < i; ++j) acc = fmaf(Am[(16 * bi + i) * 65 + 16 * bi + j], tc[j], acc);
                tc[i] = (i == lane ? 1.0f : 0.0f) - acc;
                Tm[(16 * bi + i) * 65 + 16 * bi + lane] = tc[i];
            }
        }
        // blocks right of the diagonal are zero
        for (int idx = lane; idx < 16 * (48 - 16 * bi); idx += 64) {
            const int i = idx / (48 - 16 * bi), j = 16 * (bi + 1) + idx % (48 - 16 * bi);
            Tm[(16 * bi + i) * 65 + j] = 0.0f;
        }
    }
    __syncthreads();
    if (wave < 3) {
        const int bj = wave;
        for (int bi = bj + 1; bi < 4; ++bi) {
            f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
            for (int bk = bj; bk < bi; ++bk)
                acc = mm16_f32(Am + (16 * bi) * 65 + 16 * bk, 65, Tm + (16 * bk) * 65 + 16 * bj, 65, acc, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) scr[(4 * kb + ii) * 17 + n] = acc[ii];
            __builtin_amdgcn_wave_barrier();
            const f32x4_t res = mm16_f32(Tm + (16 * bi) * 65 + 16 * bi, 65, scr, 17,
                                         f32x4_t{0.f, 0.f, 0.f, 0.f}, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) Tm[(16 * bi + 4 * kb + ii) * 65 + 16 * bj + n] = -res[ii];
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
    for (int idx = t; idx < kC * kC; idx += 256) {
        const int i = idx >> 6, j = idx & 63;
        uint16_t hh, ll;
        split_bf16(Tm[i * 65 + j], hh, ll);
        Th[i * kLT + j] = hh;
        Tl[i * kLT + j] = ll;
    }
    __syncthreads();
    // X = beta e^G K into the Q buffers; Q~ = e^G Q and K~ = e^{G_C - G} K to
    // workspace (split) for the state pass
    for (int idx = t; idx < kC * 32; idx += 256) {
        const int rr = idx >> 5, q4 = idx & 31;
        const float eg = expf(G[rr]);
        const float sx = Bt[rr] * eg, sk = expf(G[kC - 1] - G[rr]);
        const size_t src = (static_cast<size_t>(t0 + rr) * 16 + kh) * 128;
        const float4 kv = rr < nv ? reinterpret_cast<const float4*>(pk + src)[q4] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 qv = rr < nv ? reinterpret_cast<const float4*>(pq + src)[q4] : make_float4(0.f, 0.f, 0.f, 0.f);
        store_split4(Qh, Ql, rr * kLD + 4 * q4, sx * kv.x, sx * kv.y, sx * kv.z, sx * kv.w);
        const size_t o = (ch * kC + rr) * 128 + 4 * q4;
        store_split4(qth + o, qtl + o, 0, eg * qv.x, eg * qv.y, eg * qv.z, eg * qv.w);
        store_split4(kth + o, ktl + o, 0, sk * kv.x, sk * kv.y, sk * kv.z, sk * kv.w);
    }
    __syncthreads();
    // W = T X and U~ = T (beta V): wave -> row tile, 8 column tiles of 16 dims
#pragma unroll 2
    for (int cd = 0; cd < 8; ++cd) {
        const f32x4_t zero = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const f32x4_t w = mma_nn_x3<kC>(zero, Th + 16 * wave * kLT, Tl + 16 * wave * kLT, kLT, Qh + 16 * cd,
                                        Ql + 16 * cd, kLD, lane);
        const f32x4_t u = mma_nn_x3<kC>(zero, Th + 16 * wave * kLT, Tl + 16 * wave * kLT, kLT, Vh + 16 * cd,
                                        Vl + 16 * cd, kLD, lane);
        const int d = 16 * cd + n;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const size_t o = (ch * kC + 16 * wave + 4 * kb + ii) * 128 + d;
            uint16_t hh, ll;
            split_bf16(w[ii], hh, ll);
            wh[o] = hh;
            wl[o] = ll;
            split_bf16(u[ii], hh, ll);
            uh[o] = hh;
            ul[o] = ll;
        }
    }
}

// grid (4 row blocks of 32, 32 value heads), 256 threads. Wave w keeps the
// state tiles (row tile 0/1) x (column tiles 2w, 2w+1) in registers.
__global__ __launch_bounds__(256) void dn_chunk_state_kernel(
    int T, const uint16_t* __restrict__ qth, const uint16_t* __restrict__ qtl, const uint16_t* __restrict__ kth,
    const uint16_t* __restrict__ ktl, const uint16_t* __restrict__ wh, const uint16_t* __restrict__ wl,
    const uint16_t* __restrict__ uh, const uint16_t* __restrict__ ul, const uint16_t* __restrict__ ph,
    const uint16_t* __restrict__ pl, const float* __restrict__ gin, float* __restrict__ ssm_state,
    float* __restrict__ po) {
    const int rb = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;

    __shared__ __attribute__((aligned(16))) uint16_t Sh[32 * kLD], Sl[32 * kLD];
    __shared__ __attribute__((aligned(16))) uint16_t Wh[kC * kLD], Wl[kC * kLD];   // W, then O staging
    __shared__ __attribute__((aligned(16))) uint16_t Qh[kC * kLD], Ql[kC * kLD];   // Q~ = e^G Q
    __shared__ __attribute__((aligned(16))) uint16_t Kh[kC * kLD], Kl[kC * kLD];   // K~ = e^{G_C - G} K
    __shared__ __attribute__((aligned(16))) uint16_t Ph[kC * kLT], Pl[kC * kLT];
    __shared__ __attribute__((aligned(16))) uint16_t Uh[32 * kLT], Ul[32 * kLT];   // U^T rows of this block
    __shared__ float G[kC];
    float* Os = reinterpret_cast<float*>(Wh);   // [64][33] fp32, after W is consumed

    float* Sg = ssm_state + (static_cast<size_t>(h) * 128 + 32 * rb) * 128;
    f32x4_t sacc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                sacc[rt][cc][ii] = Sg[(16 * rt + 4 * kb + ii) * 128 + 16 * (2 * wave + cc) + n];

    const int nch = (T + kC - 1) / kC;
    // Chunk inputs travel global -> registers -> LDS; the registers for chunk
    // c+1 are loaded while chunk c computes. Per thread: 4 x 16 B of each of
    // W, Q~, K~ (hi and lo), 2 x 16 B of P hi and lo, and the 16 U~ values
    // (hi, lo) its Y1 outputs need.
    u32x4_t pre[6][4], prep_[2][2];
    uint16_t preu[2][2][4][2];
    float preg = 0.0f;
    auto fetch = [&](int c) {
        const size_t ch = static_cast<size_t>(c) * 32 + h;
        // the small loads first: vmcnt retires in issue order, so consuming
        // them early must not wait on the bulk copies behind them
        const int rt = wave & 1;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int i = 16 * (2 * (wave >> 1) + cc) + n;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const size_t gu = (ch * kC + i) * 128 + 32 * rb + 16 * rt + 4 * kb + ii;
                preu[cc][0][ii][0] = uh[gu];
                preu[cc][0][ii][1] = ul[gu];
            }
        }
        if (t < kC) preg = gin[ch * kC + t];
        const size_t o = ch * kC * 128;
        const uint16_t* srcs[6] = {wh + o, wl + o, qth + o, qtl + o, kth + o, ktl + o};
#pragma unroll
        for (int a = 0; a < 6; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) pre[a][i] = reinterpret_cast<const u32x4_t*>(srcs[a])[t + 256 * i];
        const u32x4_t* gp_h = reinterpret_cast<const u32x4_t*>(ph + ch * kC * kC);
        const u32x4_t* gp_l = reinterpret_cast<const u32x4_t*>(pl + ch * kC * kC);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            prep_[0][i] = gp_h[t + 256 * i];
            prep_[1][i] = gp_l[t + 256 * i];
        }
    };
    fetch(0);
    for (int c = 0; c < nch; ++c) {
        const int t0 = c * kC;
        const int nv = min(kC, T - t0);
        // registers -> LDS
        {
            uint16_t* dst[6] = {Wh, Wl, Qh, Ql, Kh, Kl};
#pragma unroll
            for (int a = 0; a < 6; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int q = t + 256 * i;
                    *reinterpret_cast<u32x4_t*>(&dst[a][(q >> 4) * kLD + 8 * (q & 15)]) = pre[a][i];
                }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int q = t + 256 * i;
                *reinterpret_cast<u32x4_t*>(&Ph[(q >> 3) * kLT + 8 * (q & 7)]) = prep_[0][i];
                *reinterpret_cast<u32x4_t*>(&Pl[(q >> 3) * kLT + 8 * (q & 7)]) = prep_[1][i];
            }
            if (t < kC) G[t] = preg;
        }
        float ucur[2][4];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                ucur[cc][ii] = bf16_to_f32(preu[cc][0][ii][0]) + bf16_to_f32(preu[cc][0][ii][1]);
        // state -> LDS as the A operand (rows of this block)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    uint16_t hh, ll;
                    split_bf16(sacc[rt][cc][ii], hh, ll);
                    const int o = (16 * rt + 4 * kb + ii) * kLD + 16 * (2 * wave + cc) + n;
                    Sh[o] = hh;
                    Sl[o] = ll;
                }
        __syncthreads();
        if (c + 1 < nch) fetch(c + 1);
        const float gamma = expf(G[kC - 1]);
        // U^T[r][i] = U~[i][r] - sum_d S[r][d] W[i][d]: wave -> row tile w&1,
        // token tiles 2(w>>1), +1
        const int rt = wave & 1, ci0 = 2 * (wave >> 1);
        {
            f32x4_t sw[1][2] = {{f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}}};
            mma_block_x3<128, 1, 2, false>(sw, Sh, Sl, kLD, 16 * rt, Wh, Wl, kLD, 16 * ci0, lane);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int i = 16 * (ci0 + cc) + n;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int rr = 16 * rt + 4 * kb + ii;
                    uint16_t hh, ll;
                    split_bf16(ucur[cc][ii] - sw[0][cc][ii], hh, ll);
                    Uh[rr * kLT + i] = hh;
                    Ul[rr * kLT + i] = ll;
                }
            }
        }
        __syncthreads();
        // O^T[r][i] = sum_d S[r][d] Q~[i][d] + sum_j U^T[r][j] P[i][j]
        {
            f32x4_t o[1][2] = {{f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}}};
            mma_block_x3<128, 1, 2, false>(o, Sh, Sl, kLD, 16 * rt, Qh, Ql, kLD, 16 * ci0, lane);
            mma_block_x3<kC, 1, 2, false>(o, Uh, Ul, kLT, 16 * rt, Ph, Pl, kLT, 16 * ci0, lane);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int i = 16 * (ci0 + cc) + n;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) Os[i * 33 + 16 * rt + 4 * kb + ii] = o[0][cc][ii];
            }
        }
        __syncthreads();
        // pre-norm outputs of this block's 32 rows, token-major
        {
            const int i = t >> 2, r8 = 8 * (t & 3);
            if (i < nv) {
                float* dst = po + static_cast<size_t>(t0 + i) * 4096 + h * 128 + 32 * rb + r8;
#pragma unroll
                for (int e = 0; e < 8; ++e) dst[e] = Os[i * 33 + r8 + e];
            }
        }
        // S = e^{G_C} S + U^T K~
#pragma unroll
        for (int rt2 = 0; rt2 < 2; ++rt2)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) sacc[rt2][cc][ii] *= gamma;
        mma_block_x3<kC, 2, 2, true>(sacc, Uh, Ul, kLT, 0, Kh, Kl, kLD, 32 * wave, lane);
        __syncthreads();
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                Sg[(16 * rt + 4 * kb + ii) * 128 + 16 * (2 * wave + cc) + n] = sacc[rt][cc][ii];
}

hipError_t launch_deltanet_chunked(qff_ctx* ctx, hipStream_t stream, int T, float* ssm_state) {
    const int nch = (T + kC - 1) / kC;
    {
        ProfScope prof(ctx, stream, "dn_chunk_local");
        dn_chunk_local_kernel<<<dim3(nch, 32), 256, 0, stream>>>(
            T, ctx->pf_q, ctx->pf_k, ctx->pf_v, ctx->pf_g, ctx->pf_beta, ctx->pf_wh, ctx->pf_wl, ctx->pf_uh,
            ctx->pf_ul, ctx->pf_ph, ctx->pf_pl, ctx->pf_G, ctx->pf_qth, ctx->pf_qtl, ctx->pf_kth, ctx->pf_ktl);
    }
    ProfScope prof(ctx, stream, "dn_chunk_state");
    dn_chunk_state_kernel<<<dim3(4, 32), 256, 0, stream>>>(T, ctx->pf_qth, ctx->pf_qtl, ctx->pf_kth, ctx->pf_ktl,
                                                           ctx->pf_wh, ctx->pf_wl, ctx->pf_uh, ctx->pf_ul, ctx->pf_ph,
                                                           ctx->pf_pl, ctx->pf_G, ssm_state, ctx->pf_o);
    return hipGetLastError();
}

}  // namespace qff
