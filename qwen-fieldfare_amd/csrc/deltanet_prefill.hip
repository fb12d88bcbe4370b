// deltanet_prefill.hip -- T tokens of one sequence through the Gated DeltaNet
// layer core.
//
// The reference has no prefill kernel: prompts go token by token through the
// decode path (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561). This file
// computes the same result for a whole sequence:
//   prep       conv1d + SiLU over time for all 8192 channels (each token only
//              needs the 3 previous inputs, so tokens run in parallel), L2
//              norms of q (then / sqrt(128)) and k per key head, and the
//              per-token log gate and beta of every value head;
//   chunked    the chunked WY form of the gated delta rule
//              (deltanet_chunked.hip), pre-norm outputs to workspace;
//   norm       gated RMSNorm of every (token, value head) output row;
//   conv state the conv state after the last token.
#include "common.hpp"
#include "internal.hpp"

namespace qff {

// e[i] of channel c: the 4 conv-state slots, then the T inputs.
template <int IN_DT>
__device__ __forceinline__ float conv_ext(const float* __restrict__ conv_state, const void* __restrict__ qkv,
                                          int c, int i) {
    return i < 4 ? conv_state[c * 4 + i] : elem<IN_DT>::load(qkv, static_cast<size_t>(i - 4) * 8192 + c);
}

constexpr int kPrepTokens = 16;   // tokens per prep workgroup

// grid (ceil(T/16), 32 channel blocks of 256), 256 threads: thread = channel,
// walking 16 tokens with a sliding 4-tap window (one new input per token).
// Channel blocks 0-7 hold q (two key heads each), 8-15 k, 16-31 v. Block 0
// also forms the 16 tokens' log gates and betas.
template <int IN_DT>
__global__ __launch_bounds__(256) void dn_prefill_prep_kernel(
    int T, const void* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias, const float* __restrict__ conv_w,
    const float* __restrict__ conv_state, float* __restrict__ pq, float* __restrict__ pk,
    float* __restrict__ pv, float* __restrict__ plg, float* __restrict__ pbeta) {
    __shared__ float red[kPrepTokens][4];
    const int tb = blockIdx.x * kPrepTokens, blk = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int c = blk * 256 + t;
    const int nt = min(kPrepTokens, T - tb);
    const float4 w = reinterpret_cast<const float4*>(conv_w)[c];
    // token tok uses e[tok+1 .. tok+4] (deltanet.metal:120-137 after the shift)
    float e1 = conv_ext<IN_DT>(conv_state, qkv, c, tb + 1);
    float e2 = conv_ext<IN_DT>(conv_state, qkv, c, tb + 2);
    float e3 = conv_ext<IN_DT>(conv_state, qkv, c, tb + 3);
    float y[kPrepTokens];
#pragma unroll
    for (int i = 0; i < kPrepTokens; ++i) {
        const float e4 = i < nt ? elem<IN_DT>::load(qkv, static_cast<size_t>(tb + i) * 8192 + c) : 0.0f;
        y[i] = silu(e1 * w.x + e2 * w.y + e3 * w.z + e4 * w.w);
        e1 = e2; e2 = e3; e3 = e4;
    }
    if (blk < 16) {
        // L2 norm per key head: waves 0-1 one head, waves 2-3 the other
#pragma unroll
        for (int i = 0; i < kPrepTokens; ++i) {
            const float ss = group_sum<64>(y[i] * y[i]);
            if (lane == 0) red[i][wave] = ss;
        }
        __syncthreads();
        const int hw = wave & 2;
        float* dst = blk < 8 ? pq : pk;
        const int cc = blk < 8 ? c : c - 2048;
#pragma unroll
        for (int i = 0; i < kPrepTokens; ++i) {
            if (i >= nt) break;
            const float inv = 1.0f / sqrtf(red[i][hw] + red[i][hw + 1] + 1e-6f);
            const float v = blk < 8 ? (y[i] * inv) * (1.0f / sqrtf(128.0f)) : y[i] * inv;
            dst[static_cast<size_t>(tb + i) * 2048 + cc] = v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kPrepTokens; ++i) {
            if (i >= nt) break;
            pv[static_cast<size_t>(tb + i) * 4096 + (c - 4096)] = y[i];
        }
    }
    if (blk == 0) {
        for (int idx = t; idx < nt * 32; idx += 256) {
            const int hh = idx & 31;
            const size_t gi = static_cast<size_t>(tb) * 32 + idx;
            plg[gi] = -expf(a_log[hh]) * softplus(a[gi] + dt_bias[hh]);   // log g
            pbeta[gi] = sigmoid(b[gi]);
        }
    }
}

// grid (T), 256 threads: thread -> value head t/8, rows 16*(t%8) .. +15.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void dn_prefill_norm_kernel(const float* __restrict__ po,
                                                              const void* __restrict__ z,
                                                              const float* __restrict__ norm_w, float eps,
                                                              void* __restrict__ out) {
    const int tok = blockIdx.x, t = threadIdx.x;
    const int r0 = 16 * (t & 7);
    const size_t base = static_cast<size_t>(tok) * 4096 + (t >> 3) * 128 + r0;
    const float4* src = reinterpret_cast<const float4*>(po + base);
    float o[16], ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = src[i];
        o[4 * i] = v.x; o[4 * i + 1] = v.y; o[4 * i + 2] = v.z; o[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) ss += o[i] * o[i];
    ss = group_sum<8>(ss);
    const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
#pragma unroll
    for (int i = 0; i < 16; ++i)
        elem<OUT_DT>::store(out, base + i, o[i] * inv * norm_w[r0 + i] * silu(elem<IN_DT>::load(z, base + i)));
}

// conv state after the last token: slots = e[T .. T+3]. grid 32 x 256.
template <int IN_DT>
__global__ __launch_bounds__(256) void dn_prefill_conv_state_kernel(int T, const void* __restrict__ qkv,
                                                                    float* __restrict__ conv_state) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const float e0 = conv_ext<IN_DT>(conv_state, qkv, c, T);
    const float e1 = conv_ext<IN_DT>(conv_state, qkv, c, T + 1);
    const float e2 = conv_ext<IN_DT>(conv_state, qkv, c, T + 2);
    const float e3 = conv_ext<IN_DT>(conv_state, qkv, c, T + 3);
    reinterpret_cast<float4*>(conv_state)[c] = make_float4(e0, e1, e2, e3);
}

hipError_t launch_deltanet_prefill(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, const void* z, qff_dtype in_dtype,
                                   const float* a, const float* b, float* conv_state,
                                   float* ssm_state, void* out, qff_dtype out_dtype, int T) {
    const bool bf = in_dtype == QFF_BF16;
    {
    ProfScope prof(ctx, stream, "dn_prefill_prep");
    if (bf)
        dn_prefill_prep_kernel<1><<<dim3((T + kPrepTokens - 1) / kPrepTokens, 32), 256, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                  conv_state, ctx->pf_q, ctx->pf_k, ctx->pf_v,
                                                                  ctx->pf_g, ctx->pf_beta);
    else
        dn_prefill_prep_kernel<0><<<dim3((T + kPrepTokens - 1) / kPrepTokens, 32), 256, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                  conv_state, ctx->pf_q, ctx->pf_k, ctx->pf_v,
                                                                  ctx->pf_g, ctx->pf_beta);
    }
    {
        hipError_t e = launch_deltanet_chunked(ctx, stream, T, ssm_state);
        if (e != hipSuccess) return e;
    }
    const dim3 ng(T);
    {
    ProfScope prof(ctx, stream, "dn_prefill_norm");
#define QFF_NORM(I, O) dn_prefill_norm_kernel<I, O><<<ng, 256, 0, stream>>>(ctx->pf_o, z, p->norm_w, p->eps, out)
    if (bf) {
        if (out_dtype == QFF_BF16) QFF_NORM(1, 1); else QFF_NORM(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_NORM(0, 1); else QFF_NORM(0, 0);
    }
#undef QFF_NORM
    }
    ProfScope prof(ctx, stream, "dn_prefill_conv_state");
    if (bf) dn_prefill_conv_state_kernel<1><<<32, 256, 0, stream>>>(T, qkv, conv_state);
    else dn_prefill_conv_state_kernel<0><<<32, 256, 0, stream>>>(T, qkv, conv_state);
    return hipGetLastError();
}

}  // namespace qff
