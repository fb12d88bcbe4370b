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

// grid (T, 64 channel blocks of 128), 128 threads.
template <int IN_DT>
__global__ __launch_bounds__(128) void dn_prefill_prep_kernel(
    const void* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias, const float* __restrict__ conv_w,
    const float* __restrict__ conv_state, float* __restrict__ pq, float* __restrict__ pk,
    float* __restrict__ pv, float* __restrict__ pg, float* __restrict__ pbeta) {
    const int tok = blockIdx.x, blk = blockIdx.y, t = threadIdx.x;
    const int c = blk * 128 + t;
    const float4 w = reinterpret_cast<const float4*>(conv_w)[c];
    // token tok uses e[tok+1 .. tok+4] (deltanet.metal:120-137 after the shift)
    const float e0 = conv_ext<IN_DT>(conv_state, qkv, c, tok + 1);
    const float e1 = conv_ext<IN_DT>(conv_state, qkv, c, tok + 2);
    const float e2 = conv_ext<IN_DT>(conv_state, qkv, c, tok + 3);
    const float e3 = conv_ext<IN_DT>(conv_state, qkv, c, tok + 4);
    const float y = silu(e0 * w.x + e1 * w.y + e2 * w.z + e3 * w.w);
    if (blk < 32) {
        __shared__ float red[2];
        const float ss = group_sum<64>(y * y);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        const float inv = 1.0f / sqrtf(red[0] + red[1] + 1e-6f);
        if (blk < 16) pq[static_cast<size_t>(tok) * 2048 + c] = (y * inv) * (1.0f / sqrtf(128.0f));
        else pk[static_cast<size_t>(tok) * 2048 + (c - 2048)] = y * inv;
    } else {
        pv[static_cast<size_t>(tok) * 4096 + (c - 4096)] = y;
    }
    if (blk == 0 && t < 32) {
        const int i = tok * 32 + t;
        pg[i] = -expf(a_log[t]) * softplus(a[i] + dt_bias[t]);   // log g
        pbeta[i] = sigmoid(b[i]);
    }
}

// grid (T, 16), 256 threads: value heads 2*blockIdx.y (waves 0-1) and +1.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void dn_prefill_norm_kernel(const float* __restrict__ po,
                                                              const void* __restrict__ z,
                                                              const float* __restrict__ norm_w, float eps,
                                                              void* __restrict__ out) {
    __shared__ float red[4];
    const int tok = blockIdx.x, t = threadIdx.x;
    const int hh = blockIdx.y * 2 + (t >> 7), r = t & 127;
    const size_t i = static_cast<size_t>(tok) * 4096 + hh * 128 + r;
    const float o = po[i];
    const float ss = group_sum<64>(o * o);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = (t < 128) ? (red[0] + red[1]) : (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / 128.0f + eps);
    elem<OUT_DT>::store(out, i, o * inv * norm_w[r] * silu(elem<IN_DT>::load(z, i)));
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
        dn_prefill_prep_kernel<1><<<dim3(T, 64), 128, 0, stream>>>(qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                  conv_state, ctx->pf_q, ctx->pf_k, ctx->pf_v,
                                                                  ctx->pf_g, ctx->pf_beta);
    else
        dn_prefill_prep_kernel<0><<<dim3(T, 64), 128, 0, stream>>>(qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                  conv_state, ctx->pf_q, ctx->pf_k, ctx->pf_v,
                                                                  ctx->pf_g, ctx->pf_beta);
    }
    {
        hipError_t e = launch_deltanet_chunked(ctx, stream, T, ssm_state);
        if (e != hipSuccess) return e;
    }
    const dim3 ng(T, 16);
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
