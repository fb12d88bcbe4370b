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
//   P_ij = e^{G_i - G_j} (q_i . k_j)  (j <= i)
//   O = (e^G Q) S0^T + P U = Qe S0^T + P U~,   Qe = e^G Q - P W
//   S_C = e^{G_C} S0 + U^T K~,  K~ = e^{G_C - G} K
// (tests/test_oracle_deltanet.py checks them against the sequential
// recurrence in fp64). Writing O through Qe takes U out of it, so the
// sequential pass forms U and O from the same S0 in one step.
//
// Two kernels:
//   dn_chunk_local_kernel  one workgroup per (chunk, value head), all chunks
//       at once: conv1d + SiLU of the chunk's q, k, v channels straight from
//       the projection (3 tokens of history from the input or the conv
//       state), L2 norms, gates, then A, P, T (16x16 blocks: diagonal blocks
//       by substitution, the rest on fp32 MFMAs), W, U~ and Qe; writes W, Qe,
//       K~^T, U~^T, P (bf16 hi/lo) and e^{G_C}.
//   dn_chunk_state_kernel  one workgroup per (block of RB state rows, value
//       head) walks the chunks in order with its state rows in registers:
//       U^T = U~^T - S W^T and O^T = S Qe^T + U~^T P^T in one pass over
//       [S | U~^T], then S = e^{G_C} S + U^T K~. Its MFMA B operands are read
//       from global memory straight into registers in operand layout, one
//       chunk ahead.
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

// ---- chunk-local pass --------------------------------------------------------

// Conv input of 8 consecutive channels at stream position pos: the token's
// projection for pos >= 0, conv-state slot pos + 4 for pos in [-3, -1].
template <int IN_DT>
__device__ __forceinline__ void load_e8(const void* __restrict__ qkv, const float* __restrict__ conv_state, int ch,
                                        int pos, float (&e)[8], bool may_precede) {
    if (!may_precede || pos >= 0) {
        if (IN_DT == 1) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(qkv) +
                                                                static_cast<size_t>(pos) * 8192 + ch);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                e[2 * k] = __uint_as_float(v[k] << 16);
                e[2 * k + 1] = __uint_as_float(v[k] & 0xffff0000u);
            }
        } else {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(qkv) +
                                                              static_cast<size_t>(pos) * 8192 + ch);
            const float4 v0 = p[0], v1 = p[1];
            e[0] = v0.x; e[1] = v0.y; e[2] = v0.z; e[3] = v0.w;
            e[4] = v1.x; e[5] = v1.y; e[6] = v1.z; e[7] = v1.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = conv_state[(ch + k) * 4 + pos + 4];
    }
}

// y[i][k] = SiLU(conv1d) of channel ch + k at token tok0 + i (deltanet.metal
// :120-137: taps w.x .. w.w over inputs tok-3 .. tok); 0 for tokens >= T.
// EDGE: the window may reach before token 0 (conv state) or past T - 1;
// chunks away from both ends take the branch-free path.
template <int IN_DT, int NT, bool EDGE>
__device__ __forceinline__ void conv8(const void* __restrict__ qkv, const float* __restrict__ conv_state,
                                      const float* __restrict__ conv_w, int ch, int tok0, int T,
                                      float (&y)[NT][8]) {
    float e[NT + 3][8];
#pragma unroll
    for (int i = 0; i < NT + 3; ++i) {
        const int pos = tok0 - 3 + i;
        if (!EDGE || pos < T) {
            load_e8<IN_DT>(qkv, conv_state, ch, pos, e[i], EDGE);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) e[i][k] = 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float4 w = reinterpret_cast<const float4*>(conv_w)[ch + k];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const float v = silu_fast(e[i][k] * w.x + e[i + 1][k] * w.y + e[i + 2][k] * w.z + e[i + 3][k] * w.w);
            y[i][k] = !EDGE || tok0 + i < T ? v : 0.0f;
        }
    }
}

template <int IN_DT, int NT>
__device__ __forceinline__ void conv8_any(bool edge, const void* __restrict__ qkv, const float* __restrict__ conv_state,
                                          const float* __restrict__ conv_w, int ch, int tok0, int T,
                                          float (&y)[NT][8]) {
    if (edge)
        conv8<IN_DT, NT, true>(qkv, conv_state, conv_w, ch, tok0, T, y);
    else
        conv8<IN_DT, NT, false>(qkv, conv_state, conv_w, ch, tok0, T, y);
}

// Interior chunks of bf16 input: the 7 projection rows tok0-3 .. tok0+3 of
// 8 channels are loaded up front (one 16-B load each), so every conv pass's
// loads are in flight together, and the conv runs from registers.
__device__ __forceinline__ void conv_rows_bf16(const void* __restrict__ qkv, int ch, int tok0, u32x4_t (&r)[7]) {
#pragma unroll
    for (int i = 0; i < 7; ++i)
        r[i] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(qkv) +
                                                 static_cast<size_t>(tok0 - 3 + i) * 8192 + ch);
}

__device__ __forceinline__ void conv_from_rows(const u32x4_t (&r)[7], const float* __restrict__ conv_w, int ch,
                                               float (&y)[4][8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float4 w = reinterpret_cast<const float4*>(conv_w)[ch + k];
        float e[7];
#pragma unroll
        for (int i = 0; i < 7; ++i)
            e[i] = (k & 1) ? __uint_as_float(r[i][k >> 1] & 0xffff0000u) : __uint_as_float(r[i][k >> 1] << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i][k] = silu_fast(e[i] * w.x + e[i + 1] * w.y + e[i + 2] * w.z + e[i + 3] * w.w);
    }
}

// Splits 8 floats into bf16 hi / lo and stores 16 B of each.
__device__ __forceinline__ void store_split8(uint16_t* hi, uint16_t* lo, const float (&x)[8]) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) split_bf16x2(x[2 * k], x[2 * k + 1], hw[k], lw[k]);
    *reinterpret_cast<u32x4_t*>(hi) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<u32x4_t*>(lo) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
}

// Operand-order layout of a row-major [rows][K] bf16 matrix that is read as
// 16x16x32 MFMA operand tiles (row r of a tile in lane r % 16, k = 8 k8 ..
// 8 k8 + 7 in lane group k8 % 4): the 8 elements (r, 8 k8 .. 8 k8 + 7) sit at
// element offset 8 * swz<K>(r, k8), so the 64 lanes' pieces of each (row
// tile, k step) are one contiguous 1 KB block and a wave's operand load is
// fully coalesced.
template <int K>
__device__ __forceinline__ int swz(int r, int k8) {
    return ((r >> 4) * (K / 32) + (k8 >> 2)) * 64 + (k8 & 3) * 16 + (r & 15);
}

// LDS carve-up of the chunk-local kernel (bytes)
constexpr int kTile128 = kC * kLD * 2;            // one [64][136] bf16 array
constexpr int kOffK = 0;                          // K hi, lo; then X = beta e^G K; then P W (fp32)
constexpr int kOffQ = 2 * kTile128;               // Q hi, lo; then T (fp32) + scratch; then W hi, lo
constexpr int kOffV = 4 * kTile128;               // beta V hi, lo
constexpr int kOffA = 6 * kTile128;               // A fp32 [64][65]
constexpr int kOffT = kOffA + kC * 65 * 4;        // P hi, lo, then T hi, lo, then P again: [64][72]
constexpr int kOffG = kOffT + 2 * kC * kLT * 2;   // G[64], beta[64]
constexpr int kLocalSmem = kOffG + 2 * kC * 4;

// grid (ceil(T/64), 32 value heads), 256 threads.
template <int IN_DT>
__global__ __launch_bounds__(256) void dn_chunk_local_kernel(
    int T, const void* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias, const float* __restrict__ conv_w,
    const float* __restrict__ conv_state, qff_dn_bufs out) {
    const int c = blockIdx.x, h = blockIdx.y, kh = h >> 1;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int t0 = c * kC;
    const int nv = min(kC, T - t0);
    const size_t ch = static_cast<size_t>(c) * 32 + h;
    const bool edge = c == 0 || t0 + kC > T;   // conv window leaves [0, T)

    __shared__ __attribute__((aligned(16))) unsigned char smem[kLocalSmem];
    uint16_t* Kh = reinterpret_cast<uint16_t*>(smem + kOffK);
    uint16_t* Kl = Kh + kC * kLD;
    uint16_t* Qh = reinterpret_cast<uint16_t*>(smem + kOffQ);
    uint16_t* Ql = Qh + kC * kLD;
    uint16_t* Vh = reinterpret_cast<uint16_t*>(smem + kOffV);
    uint16_t* Vl = Vh + kC * kLD;
    float* Am = reinterpret_cast<float*>(smem + kOffA);
    uint16_t* Th = reinterpret_cast<uint16_t*>(smem + kOffT);
    uint16_t* Tl = Th + kC * kLT;
    float* G = reinterpret_cast<float*>(smem + kOffG);
    float* Bt = G + kC;

    // Conv passes: thread -> channels 8oc .. 8oc+7 of a 128-channel block x
    // tokens 4g .. 4g+3 (q and k of key head kh, v of value head h).
    const int oc = t & 15, g = t >> 4;
    const bool fast = IN_DT == 1 && !edge;
    u32x4_t rq[7], rk[7], rv[7];
    if (fast) {
        conv_rows_bf16(qkv, kh * 128 + 8 * oc, t0 + 4 * g, rq);
        conv_rows_bf16(qkv, 2048 + kh * 128 + 8 * oc, t0 + 4 * g, rk);
        conv_rows_bf16(qkv, 4096 + h * 128 + 8 * oc, t0 + 4 * g, rv);
    }
    auto conv = [&](const u32x4_t (&r)[7], int chn, float (&y)[4][8]) {
        if (fast)
            conv_from_rows(r, conv_w, chn, y);
        else
            conv8_any<IN_DT, 4>(edge, qkv, conv_state, conv_w, chn, t0 + 4 * g, T, y);
    };
    // L2 norm per token over the 16 lanes of its head (deltanet.metal
    // :282-305), q then / sqrt(128); into LDS as bf16 hi/lo.
    auto l2norm_store = [&](float (&y)[4][8], bool isq, uint16_t* dh, uint16_t* dl) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) ss += y[i][k] * y[i][k];
            ss = group_sum<16>(ss);
            const float inv = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
            for (int k = 0; k < 8; ++k) y[i][k] = isq ? (y[i][k] * inv) * (1.0f / sqrtf(128.0f)) : y[i][k] * inv;
            store_split8(dh + (4 * g + i) * kLD + 8 * oc, dl + (4 * g + i) * kLD + 8 * oc, y[i]);
        }
    };

    // gates (deltanet.metal:250-280): log g = -e^{A_log} softplus(a + dt_bias),
    // beta = sigmoid(b); G = inclusive prefix sum over the chunk. Padded
    // tokens have log g = 0 and beta = 0, so they change nothing.
    if (wave == 0) {
        const bool ok = lane < nv;
        const size_t gi = static_cast<size_t>(t0 + lane) * 32 + h;
        float x = ok ? -expf(a_log[h]) * softplus(a[gi] + dt_bias[h]) : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        G[lane] = x;
        Bt[lane] = ok ? sigmoid(b[gi]) : 0.0f;
        if (lane == 63) out.gam[ch] = expf(x);
    }
    float qn[4][8], kn[4][8];
    conv(rq, kh * 128 + 8 * oc, qn);
    l2norm_store(qn, true, Qh, Ql);
    conv(rk, 2048 + kh * 128 + 8 * oc, kn);
    l2norm_store(kn, false, Kh, Kl);
    __syncthreads();
    // K~^T rows 8oc .. 8oc+7, tokens 4g .. 4g+3 (half of an operand piece)
    {
        const float gc = G[kC - 1];
        float sk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sk[i] = expf(gc - G[4 * g + i]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t h0, l0, h1, l1;
            split_bf16x2(sk[0] * kn[0][k], sk[1] * kn[1][k], h0, l0);
            split_bf16x2(sk[2] * kn[2][k], sk[3] * kn[3][k], h1, l1);
            const size_t o = ch * 128 * kC + 8 * swz<kC>(8 * oc + k, g >> 1) + 4 * (g & 1);
            *reinterpret_cast<u32x2_t*>(out.kth + o) = u32x2_t{h0, h1};
            *reinterpret_cast<u32x2_t*>(out.ktl + o) = u32x2_t{l0, l1};
        }
    }
    // beta v of value head h
    {
        float y[4][8];
        conv(rv, 4096 + h * 128 + 8 * oc, y);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * g + i;
            const float bb = Bt[row];
#pragma unroll
            for (int k = 0; k < 8; ++k) y[i][k] *= bb;
            store_split8(Vh + row * kLD + 8 * oc, Vl + row * kLD + 8 * oc, y[i]);
        }
    }
    // Q~ = e^G q, kept for Qe
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float eg = expf(G[4 * g + i]);
#pragma unroll
        for (int k = 0; k < 8; ++k) qn[i][k] *= eg;
    }
    __syncthreads();

    // K K^T -> A (strictly lower, scaled), Q K^T -> P (lower incl. diagonal)
    {
        f32x4_t kk[1][4], qk[1][4];
#pragma unroll
        for (int cj = 0; cj < 4; ++cj) kk[0][cj] = qk[0][cj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<128, 1, 4, false>(kk, Kh, Kl, kLD, 16 * wave, Kh, Kl, kLD, 0, lane);
        mma_block_x3<128, 1, 4, false>(qk, Qh, Ql, kLD, 16 * wave, Kh, Kl, kLD, 0, lane);
#pragma unroll
        for (int cj = 0; cj < 4; ++cj) {
            const int j = 16 * cj + n;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * wave + 4 * kb + ii;
                const float decay = j <= i ? expf(G[i] - G[j]) : 0.0f;
                Am[i * 65 + j] = j < i ? Bt[i] * decay * kk[0][cj][ii] : 0.0f;
                uint16_t hh, ll;
                split_bf16(decay * qk[0][cj][ii], hh, ll);
                Th[i * kLT + j] = hh;
                Tl[i * kLT + j] = ll;
            }
        }
    }
    __syncthreads();
    // P out, 16 B per thread and piece; the pieces stay in registers until
    // the T region is free again
    u32x4_t pkeep[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = t + 256 * k, arr = q >> 9, row = (q & 511) >> 3, c8 = 8 * (q & 7);
        pkeep[k] = *reinterpret_cast<const u32x4_t*>((arr ? Tl : Th) + row * kLT + c8);
        *reinterpret_cast<u32x4_t*>((arr ? out.pl : out.ph) + ch * kC * kC + 8 * swz<kC>(row, q & 7)) = pkeep[k];
    }
    // T = (I + A)^-1 (lower unitriangular) in 16x16 blocks, fp32:
    //   diagonal blocks by forward substitution, one wave each;
    //   T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj for i > j, wave j walking
    //   column block j downwards (fp32 MFMA 16x16x4).
    float* Tm = reinterpret_cast<float*>(smem + kOffQ);   // [64][65] (Q is consumed)
    float* scr = reinterpret_cast<float*>(smem + kOffQ + kTile128) + wave * (16 * 17);
    {
        const int bi = wave;
        if (lane < 16) {
            float tc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < i; ++j) acc[j & 3] = fmaf(Am[(16 * bi + i) * 65 + 16 * bi + j], tc[j], acc[j & 3]);
                tc[i] = (i == lane ? 1.0f : 0.0f) - ((acc[0] + acc[1]) + (acc[2] + acc[3]));
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
    // T -> bf16 hi/lo; X = beta e^G K in place of K
    for (int idx = t; idx < kC * kC; idx += 256) {
        const int i = idx >> 6, j = idx & 63;
        uint16_t hh, ll;
        split_bf16(Tm[i * 65 + j], hh, ll);
        Th[i * kLT + j] = hh;
        Tl[i * kLT + j] = ll;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = t + 256 * k, row = q >> 4, c8 = 8 * (q & 15);
        const float s = Bt[row] * expf(G[row]);
        const u32x4_t hv = *reinterpret_cast<const u32x4_t*>(Kh + row * kLD + c8);
        const u32x4_t lv = *reinterpret_cast<const u32x4_t*>(Kl + row * kLD + c8);
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = s * (__uint_as_float(hv[e] << 16) + __uint_as_float(lv[e] << 16));
            x[2 * e + 1] = s * (__uint_as_float(hv[e] & 0xffff0000u) + __uint_as_float(lv[e] & 0xffff0000u));
        }
        store_split8(Kh + row * kLD + c8, Kl + row * kLD + c8, x);
    }
    __syncthreads();
    // W = T X -> LDS (Q region); U~ = T (beta V) -> U~^T out.
    // Wave -> row tile (16 tokens), 8 column tiles of 16 dims in two halves.
    uint16_t* Wh = Qh;
    uint16_t* Wl = Ql;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        f32x4_t w[1][4], u[1][4];
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) w[0][cd] = u[0][cd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<kC, 1, 4, true>(w, Th, Tl, kLT, 16 * wave, Kh, Kl, kLD, 64 * half, lane);
        mma_block_x3<kC, 1, 4, true>(u, Th, Tl, kLT, 16 * wave, Vh, Vl, kLD, 64 * half, lane);
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) {
            const int d = 64 * half + 16 * cd + n;
            uint16_t uh4[4], ul4[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * wave + 4 * kb + ii;
                uint16_t hh, ll;
                split_bf16(w[0][cd][ii], hh, ll);
                Wh[i * kLD + d] = hh;
                Wl[i * kLD + d] = ll;
                split_bf16(u[0][cd][ii], uh4[ii], ul4[ii]);
            }
            const size_t o = (ch * 128 + d) * kC + 16 * wave + 4 * kb;
            *reinterpret_cast<u32x2_t*>(out.uth + o) =
                u32x2_t{uh4[0] | (static_cast<uint32_t>(uh4[1]) << 16), uh4[2] | (static_cast<uint32_t>(uh4[3]) << 16)};
            *reinterpret_cast<u32x2_t*>(out.utl + o) =
                u32x2_t{ul4[0] | (static_cast<uint32_t>(ul4[1]) << 16), ul4[2] | (static_cast<uint32_t>(ul4[3]) << 16)};
        }
    }
    __syncthreads();
    // W out; P back into the T region (T is consumed)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int q = t + 256 * k, arr = q >> 10, row = (q & 1023) >> 4, c8 = 8 * (q & 15);
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>((arr ? Wl : Wh) + row * kLD + c8);
        *reinterpret_cast<u32x4_t*>((arr ? out.wl : out.wh) + ch * kC * 128 + 8 * swz<128>(row, q & 15)) = v;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = t + 256 * k, arr = q >> 9, row = (q & 511) >> 3, c8 = 8 * (q & 7);
        *reinterpret_cast<u32x4_t*>((arr ? Tl : Th) + row * kLT + c8) = pkeep[k];
    }
    __syncthreads();
    // P W -> fp32 [64][132] in the K region (X is consumed)
    float* PW = reinterpret_cast<float*>(smem + kOffK);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        f32x4_t pw[1][4];
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) pw[0][cd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<kC, 1, 4, true>(pw, Th, Tl, kLT, 16 * wave, Wh, Wl, kLD, 64 * half, lane);
#pragma unroll
        for (int cd = 0; cd < 4; ++cd)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                PW[(16 * wave + 4 * kb + ii) * 132 + 64 * half + 16 * cd + n] = pw[0][cd][ii];
    }
    __syncthreads();
    // Qe = Q~ - P W
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * g + i;
        const float4 p0 = *reinterpret_cast<const float4*>(PW + row * 132 + 8 * oc);
        const float4 p1 = *reinterpret_cast<const float4*>(PW + row * 132 + 8 * oc + 4);
        const float pw[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        float y[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = qn[i][k] - pw[k];
        const size_t o = ch * kC * 128 + 8 * swz<128>(row, oc);
        store_split8(out.qeh + o, out.qel + o, y);
    }
}

// ---- sequential state pass ---------------------------------------------------

// One workgroup per (16-row block of the state, value head), 512 threads; a
// 1-D grid of 256 workgroups. Workgroups are dispatched to the 8 XCDs
// round-robin by linear id, so the id -> (head, row block) map puts all row
// blocks of a head on one XCD, whose L2 then serves the chunk inputs they
// share.
// Waves 0-3 form U^T for tokens 16w .. 16w+15, waves 4-7 O^T for tokens
// 16(w-4) .. +15; wave w keeps state columns 16w .. 16w+15. Two waves per
// SIMD, each with short MFMA chains, so one wave's LDS and MFMA latencies
// overlap the other's work.
constexpr int kStateThreads = 512;
constexpr int kLA = 200;   // [S | U~^T] row stride: 128 + 64 + 8

__global__ __launch_bounds__(kStateThreads) void dn_chunk_state_kernel(int T, qff_dn_bufs in,
                                                                      float* __restrict__ ssm_state,
                                                                      float* __restrict__ po) {
    const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
    const int h = xcd * 4 + (slot >> 3), rb = slot & 7;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const bool owave = wave >= 4;          // wave-uniform role
    const int tt = wave & 3;               // token tile of U^T / O^T

    __shared__ __attribute__((aligned(16))) uint16_t Ah[16 * kLA], Al[16 * kLA];
    __shared__ __attribute__((aligned(16))) uint16_t Uh[16 * kLT], Ul[16 * kLT];

    float* Sg = ssm_state + (static_cast<size_t>(h) * 128 + 16 * rb) * 128;
    f32x4_t sacc;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) sacc[ii] = Sg[(4 * kb + ii) * 128 + 16 * wave + n];

    const int nch = (T + kC - 1) / kC;
    // Operands of one chunk. op[0..7]: W (U waves) or Qe (O waves) token
    // tile tt, [k step][hi, lo]; op[8..11]: P token tile tt (O waves; the U
    // waves load W's first steps there again, an L1 hit, so that every wave
    // runs the same loads). kr: K~^T column tile `wave`. ur: this thread's
    // piece of the block's U~^T rows (threads < 256). Two stages: each is
    // refilled with chunk c+2 as soon as its operands are consumed.
    struct Stage {
        u32x4_t op[12], kr[2][2], ur;
        float gam;
    };
    const uint16_t* oph = owave ? in.qeh : in.wh;
    const uint16_t* opl = owave ? in.qel : in.wl;
    const uint16_t* pph = owave ? in.ph : in.wh;
    const uint16_t* ppl = owave ? in.pl : in.wl;
    const int pstride = owave ? kC * kC : kC * 128;   // elements per (chunk, head) block
    auto fetch_u = [&](Stage& S, int c) {
        const size_t ch = static_cast<size_t>(c) * 32 + h;
        const int q = t & 255, arr = q >> 7, rem = q & 127;
        S.ur = *reinterpret_cast<const u32x4_t*>((arr ? in.utl : in.uth) + (ch * 128 + 16 * rb + (rem >> 3)) * kC +
                                                 8 * (rem & 7));
        S.gam = in.gam[ch];
    };
    auto fetch_op = [&](Stage& S, int c) {
        const size_t ch = static_cast<size_t>(c) * 32 + h;
        const size_t ow = ch * kC * 128 + 8 * (tt * 4 * 64 + lane);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            S.op[2 * ks] = *reinterpret_cast<const u32x4_t*>(oph + ow + 512 * ks);
            S.op[2 * ks + 1] = *reinterpret_cast<const u32x4_t*>(opl + ow + 512 * ks);
        }
        const size_t op = ch * pstride + 8 * (tt * (owave ? 2 : 4) * 64 + lane);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            S.op[8 + 2 * ks] = *reinterpret_cast<const u32x4_t*>(pph + op + 512 * ks);
            S.op[9 + 2 * ks] = *reinterpret_cast<const u32x4_t*>(ppl + op + 512 * ks);
        }
    };
    auto fetch_k = [&](Stage& S, int c) {
        const size_t ch = static_cast<size_t>(c) * 32 + h;
        const size_t ok = ch * 128 * kC + 8 * (wave * 2 * 64 + lane);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            S.kr[ks][0] = *reinterpret_cast<const u32x4_t*>(in.kth + ok + 512 * ks);
            S.kr[ks][1] = *reinterpret_cast<const u32x4_t*>(in.ktl + ok + 512 * ks);
        }
    };
    // One chunk from stage S, refilling S with chunk cn. The refill loads are
    // unconditional (cn is clamped to the last chunk) and so are the output
    // stores (the output buffer holds whole chunks): with no branch around a
    // memory instruction the compiler's vmcnt bookkeeping stays exact and
    // each wait covers only the loads it needs.
    auto step = [&](Stage& S, int c, int cn) {
        // [S | U~^T] -> LDS
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            uint16_t hh, ll;
            split_bf16(sacc[ii], hh, ll);
            const int o = (4 * kb + ii) * kLA + 16 * wave + n;
            Ah[o] = hh;
            Al[o] = ll;
        }
        if (t < 256) {
            const int arr = t >> 7, rem = t & 127;
            *reinterpret_cast<u32x4_t*>((arr ? Al : Ah) + (rem >> 3) * kLA + 128 + 8 * (rem & 7)) = S.ur;
        }
        const float g = S.gam;
        __syncthreads();
        fetch_u(S, cn);
        // U waves: acc = S W^T (k = d, 4 steps); O waves: acc = S Qe^T +
        // U~^T P^T (6 steps). Three accumulators (lo*hi, hi*lo, hi*hi) keep
        // the dependent MFMA chains short.
        f32x4_t a0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
        for (int ks = 0; ks < 6; ++ks) {
            if (ks >= 4 && !owave) break;
            const u32x4_t a_h = *reinterpret_cast<const u32x4_t*>(Ah + n * kLA + 32 * ks + 8 * kb);
            const u32x4_t a_l = *reinterpret_cast<const u32x4_t*>(Al + n * kLA + 32 * ks + 8 * kb);
            a0 = mfma_16x16x32_bf16(a_l, S.op[2 * ks], a0);
            a1 = mfma_16x16x32_bf16(a_h, S.op[2 * ks + 1], a1);
            a2 = mfma_16x16x32_bf16(a_h, S.op[2 * ks], a2);
        }
        fetch_op(S, cn);
        const f32x4_t acc = a0 + a1 + a2;
        const int i = 16 * tt + n;
        if (owave) {
            // O^T -> pre-norm output (token-major)
            *reinterpret_cast<f32x4_t*>(po + static_cast<size_t>(c * kC + i) * 4096 + h * 128 + 16 * rb + 4 * kb) = acc;
        } else {
            // U^T = U~^T - S W^T -> LDS
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int row = 4 * kb + ii;
                const float ut = bf16_to_f32(Ah[row * kLA + 128 + i]) + bf16_to_f32(Al[row * kLA + 128 + i]) - acc[ii];
                uint16_t hh, ll;
                split_bf16(ut, hh, ll);
                Uh[row * kLT + i] = hh;
                Ul[row * kLT + i] = ll;
            }
        }
        __syncthreads();
        // S = e^{G_C} S + U^T K~ (k = token, 2 steps)
        f32x4_t s1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
        sacc *= g;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const u32x4_t a_h = *reinterpret_cast<const u32x4_t*>(Uh + n * kLT + 32 * ks + 8 * kb);
            const u32x4_t a_l = *reinterpret_cast<const u32x4_t*>(Ul + n * kLT + 32 * ks + 8 * kb);
            s1 = mfma_16x16x32_bf16(a_l, S.kr[ks][0], s1);
            s1 = mfma_16x16x32_bf16(a_h, S.kr[ks][1], s1);
            sacc = mfma_16x16x32_bf16(a_h, S.kr[ks][0], sacc);
        }
        sacc += s1;
        fetch_k(S, cn);
    };
    Stage s0, s1;
    fetch_u(s0, 0);
    fetch_op(s0, 0);
    fetch_k(s0, 0);
    const int c1 = min(1, nch - 1);
    fetch_u(s1, c1);
    fetch_op(s1, c1);
    fetch_k(s1, c1);
    int c = 0;
    for (; c + 1 < nch; c += 2) {
        step(s0, c, min(c + 2, nch - 1));
        step(s1, c + 1, min(c + 3, nch - 1));
    }
    if (c < nch) step(s0, c, c);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) Sg[(4 * kb + ii) * 128 + 16 * wave + n] = sacc[ii];
}

hipError_t launch_deltanet_chunked(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, qff_dtype in_dtype, const float* a, const float* b,
                                   const float* conv_state, float* ssm_state, int T) {
    const int nch = (T + kC - 1) / kC;
    {
        ProfScope prof(ctx, stream, "dn_chunk_local");
        const dim3 grid(nch, 32);
        if (in_dtype == QFF_BF16)
            dn_chunk_local_kernel<1><<<grid, 256, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                               conv_state, ctx->dn);
        else
            dn_chunk_local_kernel<0><<<grid, 256, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                               conv_state, ctx->dn);
    }
    ProfScope prof(ctx, stream, "dn_chunk_state");
    dn_chunk_state_kernel<<<256, kStateThreads, 0, stream>>>(T, ctx->dn, ssm_state, ctx->pf_o);
    return hipGetLastError();
}

}  // namespace qff
