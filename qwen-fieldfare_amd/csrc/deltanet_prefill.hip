// deltanet_prefill.hip -- T tokens of one sequence through the Gated DeltaNet
// layer core.
//
// The reference has no prefill kernel: prompts go token by token through the
// decode path (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561). This file
// computes the same result for a whole sequence:
//   chunked    conv1d + SiLU, L2 norms, gates and the chunked WY form of the
//              gated delta rule (deltanet_chunked.hip): per-chunk operands
//              and each chunk's starting state to workspace;
//   out        the chunk outputs O = Qe S_c^T + P U~ and the gated RMSNorm
//              of every (token, value head) row, and (32 extra workgroups of
//              the same launch) the conv state after the last token.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

// e[i] of channel c: the 4 conv-state slots, then the T inputs.
template <int IN_DT>
__device__ __forceinline__ float conv_ext(const float* __restrict__ conv_state, const void* __restrict__ qkv,
                                          int c, int i) {
    return i < 4 ? conv_state[c * 4 + i] : elem<IN_DT>::load(qkv, static_cast<size_t>(i - 4) * 8192 + c);
}

constexpr int kChunk = 64;   // tokens per chunk (the chunked pass's C)

// Output pass: one workgroup per (chunk, value head), 512 threads, after the
// state pass has written every chunk's starting state S_c. Wave w owns value
// rows 16w .. 16w+15 for the chunk's 64 tokens:
//   O^T = S_c Qe^T + U~^T P^T     (bf16x3 on 16x16x32 MFMAs; A operands S_c
//                                  and U~^T rows from global memory, B
//                                  operands Qe and P staged once in LDS)
// then the gated RMSNorm of each (token, head) row over its 128 values
// (QwenDeltaNetKernel.swift:127-151: o * rsqrt(mean(o^2) + eps) * w *
// silu(z)), the per-wave sums of squares meeting in LDS. The 32 workgroups
// past the units write the conv state after the last token.
constexpr int kOutThreads = 512;

template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(kOutThreads) void dn_chunk_out_kernel(int T, qff_dn_bufs in, const void* __restrict__ z,
                                                                   const float* __restrict__ norm_w, float eps,
                                                                   void* __restrict__ out,
                                                                   const void* __restrict__ qkv,
                                                                   float* __restrict__ conv_state) {
    const int units = ((T + 63) / 64) * 32;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (static_cast<int>(blockIdx.x) >= units) {
        // conv state after the last token: slots = e[T .. T+3] of channel c
        // (the chunk-local pass has read the old slots before this launch)
        if (t >= 256) return;
        const int c = (blockIdx.x - units) * 256 + t;
        const float e0 = conv_ext<IN_DT>(conv_state, qkv, c, T);
        const float e1 = conv_ext<IN_DT>(conv_state, qkv, c, T + 1);
        const float e2 = conv_ext<IN_DT>(conv_state, qkv, c, T + 2);
        const float e3 = conv_ext<IN_DT>(conv_state, qkv, c, T + 3);
        reinterpret_cast<float4*>(conv_state)[c] = make_float4(e0, e1, e2, e3);
        return;
    }
    const int c = blockIdx.x >> 5, h = blockIdx.x & 31;
    const size_t ch = static_cast<size_t>(blockIdx.x);   // == c * 32 + h
    const int n = lane & 15, kb = lane >> 4;
    __shared__ u32x4_t qes[2][16 * 64];   // Qe hi, lo: 16 operand blocks of 1 KB
    __shared__ u32x4_t ps[2][8 * 64];     // P hi, lo: 8 blocks
    __shared__ float red[8][64];

    // Qe and P in operand order, copied block for block
    const u32x4_t* gqh = reinterpret_cast<const u32x4_t*>(in.qeh + ch * kChunk * 128);
    const u32x4_t* gql = reinterpret_cast<const u32x4_t*>(in.qel + ch * kChunk * 128);
    const u32x4_t* gph = reinterpret_cast<const u32x4_t*>(in.ph + ch * kChunk * kChunk);
    const u32x4_t* gpl = reinterpret_cast<const u32x4_t*>(in.pl + ch * kChunk * kChunk);
    u32x4_t st[6];
    st[0] = gqh[t];
    st[1] = gqh[t + kOutThreads];
    st[2] = gql[t];
    st[3] = gql[t + kOutThreads];
    st[4] = gph[t];
    st[5] = gpl[t];
    // this wave's A operands: S_c rows 16w .. (operand blocks (w, k step))
    // and the same rows of U~^T (tokens 32 ks + 8 kb .. +7)
    const u32x4_t* gsh = reinterpret_cast<const u32x4_t*>(in.sh + ch * 128 * 128);
    const u32x4_t* gsl = reinterpret_cast<const u32x4_t*>(in.sl + ch * 128 * 128);
    u32x4_t sa_h[4], sa_l[4], ua_h[2], ua_l[2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        sa_h[ks] = gsh[(wave * 4 + ks) * 64 + lane];
        sa_l[ks] = gsl[(wave * 4 + ks) * 64 + lane];
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const size_t o = (ch * 128 + 16 * wave + n) * kChunk + 32 * ks + 8 * kb;
        ua_h[ks] = *reinterpret_cast<const u32x4_t*>(in.uth + o);
        ua_l[ks] = *reinterpret_cast<const u32x4_t*>(in.utl + o);
    }
    // gate inputs and norm weights of this lane's outputs: values 16w + 4kb
    // .. +3 of tokens 16 tt + n
    const int t0 = c * kChunk;
    const int v0 = 16 * wave + 4 * kb;
    float zz[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const size_t zi = static_cast<size_t>(min(t0 + 16 * tt + n, T - 1)) * 4096 + h * 128 + v0;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) zz[tt][ii] = elem<IN_DT>::load(z, zi + ii);
    }
    const float4 nw = *reinterpret_cast<const float4*>(norm_w + v0);
    qes[0][t] = st[0];
    qes[0][t + kOutThreads] = st[1];
    qes[1][t] = st[2];
    qes[1][t + kOutThreads] = st[3];
    ps[0][t] = st[4];
    ps[1][t] = st[5];
    __syncthreads();

    f32x4_t acc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        f32x4_t a0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const u32x4_t bh = qes[0][(tt * 4 + ks) * 64 + lane], bl = qes[1][(tt * 4 + ks) * 64 + lane];
            a0 = mfma_16x16x32_bf16(sa_l[ks], bh, a0);
            a1 = mfma_16x16x32_bf16(sa_h[ks], bl, a1);
            a2 = mfma_16x16x32_bf16(sa_h[ks], bh, a2);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const u32x4_t bh = ps[0][(tt * 2 + ks) * 64 + lane], bl = ps[1][(tt * 2 + ks) * 64 + lane];
            a0 = mfma_16x16x32_bf16(ua_l[ks], bh, a0);
            a1 = mfma_16x16x32_bf16(ua_h[ks], bl, a1);
            a2 = mfma_16x16x32_bf16(ua_h[ks], bh, a2);
        }
        acc[tt] = a0 + a1 + a2;   // O^T[16w + 4kb + ii][16 tt + n]
    }
    // sum of squares of each token over this wave's 16 values
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        float ss = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) ss += acc[tt][ii] * acc[tt][ii];
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (kb == 0) red[wave][16 * tt + n] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int tok = t0 + 16 * tt + n;
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) tot += red[w][16 * tt + n];
        const float inv = 1.0f / sqrtf(tot / 128.0f + eps);
        const float wv[4] = {nw.x, nw.y, nw.z, nw.w};
        float y[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) y[ii] = acc[tt][ii] * inv * wv[ii] * silu(zz[tt][ii]);
        if (tok < T) {
            const size_t oi = static_cast<size_t>(tok) * 4096 + h * 128 + v0;
            if (OUT_DT == 1) {
                __builtin_nontemporal_store(u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])},
                                            reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(out) + oi));
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(out) + oi) = make_float4(y[0], y[1], y[2], y[3]);
            }
        }
    }
}

hipError_t launch_deltanet_prefill(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, const void* z, qff_dtype in_dtype,
                                   const float* a, const float* b, float* conv_state,
                                   float* ssm_state, void* out, qff_dtype out_dtype, int T) {
    const bool bf = in_dtype == QFF_BF16;
    {
        hipError_t e = launch_deltanet_chunked(ctx, stream, p, qkv, in_dtype, a, b, conv_state, ssm_state, T);
        if (e != hipSuccess) return e;
    }
    const dim3 ng(((T + 63) / 64) * 32 + 32);
    ProfScope prof(ctx, stream, "dn_chunk_out");
#define QFF_NORM(I, O) \
    dn_chunk_out_kernel<I, O><<<ng, kOutThreads, 0, stream>>>(T, ctx->dn, z, p->norm_w, p->eps, out, qkv, conv_state)
    if (bf) {
        if (out_dtype == QFF_BF16) QFF_NORM(1, 1); else QFF_NORM(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_NORM(0, 1); else QFF_NORM(0, 0);
    }
#undef QFF_NORM
    return hipGetLastError();
}

}  // namespace qff
