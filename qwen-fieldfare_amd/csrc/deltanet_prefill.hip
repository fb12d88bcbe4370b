// deltanet_prefill.hip -- T tokens of one sequence through the Gated DeltaNet
// layer core.
//
// The reference has no prefill kernel: prompts go token by token through the
// decode path (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561). This file
// computes the same result for a whole sequence:
//   chunked    conv1d + SiLU, L2 norms, gates and the chunked WY form of the
//              gated delta rule (deltanet_chunked.hip), pre-norm outputs to
//              workspace (fp32);
//   norm       gated RMSNorm of every (token, value head) output row, and
//              (32 extra workgroups of the same launch) the conv state after
//              the last token.
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

// 8 consecutive elements of a dtype-DT row in one or two 16-B accesses.
template <int DT> __device__ __forceinline__ void load8(const void* p, size_t i, float (&x)[8]) {
    if (DT == 2) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[2 * k] = f16_to_f32(static_cast<uint16_t>(v[k]));
            x[2 * k + 1] = f16_to_f32(static_cast<uint16_t>(v[k] >> 16));
        }
    } else if (DT == 1) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[2 * k] = __uint_as_float(v[k] << 16);
            x[2 * k + 1] = __uint_as_float(v[k] & 0xffff0000u);
        }
    } else {
        const float4 a = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[0];
        const float4 b = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
}
template <int DT> __device__ __forceinline__ void store8(void* p, size_t i, const float (&x)[8]) {
    if (DT == 1) {
        u32x4_t v;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = pack_bf16x2(x[2 * k], x[2 * k + 1]);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p) + i));
    } else {
        __builtin_nontemporal_store(f32x4_t{x[0], x[1], x[2], x[3]},
                                    reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i));
        __builtin_nontemporal_store(f32x4_t{x[4], x[5], x[6], x[7]},
                                    reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i) + 1);
    }
}

// Gated RMSNorm (QwenDeltaNetKernel.swift:127-151: o * rsqrt(mean(o^2) + eps)
// * w * silu(z)) of the fp32 pre-norm outputs the state pass wrote.
// grid (T + 32), 256 threads: thread -> value head t/8, rows 16*(t%8) .. +15;
// the 32 workgroups past the tokens write the conv state after the last token.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void dn_prefill_norm_kernel(const float* __restrict__ po,
                                                              const void* __restrict__ z,
                                                              const float* __restrict__ norm_w, float eps,
                                                              void* __restrict__ out, int T,
                                                              const void* __restrict__ qkv,
                                                              float* __restrict__ conv_state) {
    const int t = threadIdx.x;
    if (blockIdx.x >= static_cast<unsigned>(T)) {
        // conv state after the last token: slots = e[T .. T+3] of channel c
        // (the chunk-local pass has read the old slots before this launch)
        const int c = (blockIdx.x - T) * 256 + t;
        const float e0 = conv_ext<IN_DT>(conv_state, qkv, c, T);
        const float e1 = conv_ext<IN_DT>(conv_state, qkv, c, T + 1);
        const float e2 = conv_ext<IN_DT>(conv_state, qkv, c, T + 2);
        const float e3 = conv_ext<IN_DT>(conv_state, qkv, c, T + 3);
        reinterpret_cast<float4*>(conv_state)[c] = make_float4(e0, e1, e2, e3);
        return;
    }
    const int tok = blockIdx.x;
    const int r0 = 16 * (t & 7);
    const size_t base = static_cast<size_t>(tok) * 4096 + (t >> 3) * 128 + r0;
    float o[2][8], zz[2][8], ss = 0.0f;
    load8<0>(po, base, o[0]);
    load8<0>(po, base + 8, o[1]);
    load8<IN_DT>(z, base, zz[0]);
    load8<IN_DT>(z, base + 8, zz[1]);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += o[hh][i] * o[hh][i];
    ss = group_sum<8>(ss);
    const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = o[hh][i] * inv * norm_w[r0 + 8 * hh + i] * silu(zz[hh][i]);
        store8<OUT_DT>(out, base + 8 * hh, y);
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
    const dim3 ng(T + 32);
    ProfScope prof(ctx, stream, "dn_prefill_norm");
#define QFF_NORM(I, O)                                                                                   \
    dn_prefill_norm_kernel<I, O><<<ng, 256, 0, stream>>>(ctx->pf_o, z, p->norm_w, p->eps, out, T, qkv, \
                                                         conv_state)
    if (bf) {
        if (out_dtype == QFF_BF16) QFF_NORM(1, 1); else QFF_NORM(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_NORM(0, 1); else QFF_NORM(0, 0);
    }
#undef QFF_NORM
    return hipGetLastError();
}

}  // namespace qff
