// deltanet_decode.hip -- one decode step of the Gated DeltaNet layer core on
// gfx950, fused into a single launch.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1001-1022 dispatches
// qwen_conv1d_f32 (deltanet.metal:112-138) then qwen_fused_deltanet_step_f32
// (deltanet.metal:250-356) with one 128-thread threadgroup per value head.
//
// Layout here: one workgroup per (row block of 16 state rows, value head,
// sequence) -> 8 x 32 x B workgroups of 256 threads, so even batch 1 puts
// 256 workgroups (one per CU) on the 2 MiB of state each step streams.
//   phase 1  each workgroup runs the conv + SiLU for the 256 q/k channels of
//            its key head (h/2) and L2-normalises them in LDS, and runs the
//            conv for the 16 v channels of its own rows (those conv-state
//            slots belong to it alone, so it writes them back at once);
//   phase 2  each wave64 streams 4 state rows as float4 per lane (lanes 0-31
//            row r, lanes 32-63 row r+1; column block = lane % 32) and does
//            decay, k^T S, the rank-1 update and S q with 32-lane butterfly
//            sums, writing the pre-norm output row to workspace;
//   phase 3  the q/k conv state is read by the 16 workgroups of a key head,
//            so only the last of them to arrive (one atomic counter per
//            (sequence, key head)) writes it back; that workgroup also has
//            every output row of both value heads and applies the gated
//            RMSNorm. The counter is reset to zero for the next call.
// Traffic per sequence-step: 2 MiB state read + 2 MiB written, coalesced
// 16 B per lane; conv state, weights and activations are ~0.2 MiB more.
#include "common.hpp"
#include "internal.hpp"

namespace qff {

constexpr int kDnRowsPerBlock = 16;
constexpr int kDnRowBlocks = 128 / kDnRowsPerBlock;

template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void deltanet_decode_kernel(
    const void* __restrict__ qkv, const void* __restrict__ z, const float* __restrict__ a,
    const float* __restrict__ b, const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    const float* __restrict__ conv_w, const float* __restrict__ norm_w, float eps,
    float* __restrict__ conv_state, float* __restrict__ ssm_state, float* __restrict__ o_raw,
    int* __restrict__ counters, void* __restrict__ out) {
    const int rb = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
    const int kh = h >> 1;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

    __shared__ float q_s[128], k_s[128], v_s[kDnRowsPerBlock], red[4];
    __shared__ int is_last;

    // ---- phase 1: conv + SiLU + L2 norm of the key head's q and k -------------
    // deltanet.metal:120-137 (conv), :282-305 (L2 norms, q * 1/sqrt(128)).
    const size_t seq_ch = static_cast<size_t>(seq) * 8192;
    const int ch = (t < 128) ? (kh * 128 + t) : (2048 + kh * 128 + (t - 128));
    const float4 st = reinterpret_cast<const float4*>(conv_state)[seq_ch + ch];
    const float4 w4 = reinterpret_cast<const float4*>(conv_w)[ch];
    const float4 ns = make_float4(st.y, st.z, st.w, elem<IN_DT>::load(qkv, seq_ch + ch));
    const float y = silu(ns.x * w4.x + ns.y * w4.y + ns.z * w4.z + ns.w * w4.w);
    const float ss = group_sum<64>(y * y);
    if (lane == 0) red[wave] = ss;
    if (t < kDnRowsPerBlock) {
        const int vch = 4096 + h * 128 + rb * kDnRowsPerBlock + t;
        float4* vp = reinterpret_cast<float4*>(conv_state) + seq_ch + vch;
        const float4 vs = *vp;
        const float4 vw = reinterpret_cast<const float4*>(conv_w)[vch];
        const float4 vn = make_float4(vs.y, vs.z, vs.w, elem<IN_DT>::load(qkv, seq_ch + vch));
        *vp = vn;
        v_s[t] = silu(vn.x * vw.x + vn.y * vw.y + vn.z * vw.z + vn.w * vw.w);
    }
    __syncthreads();
    {
        const float tot = (t < 128) ? (red[0] + red[1]) : (red[2] + red[3]);
        const float inv = 1.0f / sqrtf(tot + 1e-6f);
        if (t < 128) q_s[t] = (y * inv) * (1.0f / sqrtf(128.0f));
        else k_s[t - 128] = y * inv;
    }
    __syncthreads();

    // ---- phase 2: gated delta rule on 16 rows ----------------------------------
    // QwenDeltaNetKernel.swift:86-124; deltanet.metal:307-335.
    const int col4 = lane & 31;
    const float4 k4 = reinterpret_cast<const float4*>(k_s)[col4];
    const float4 q4 = reinterpret_cast<const float4*>(q_s)[col4];
    const int sh = seq * 32 + h;
    const float beta = sigmoid(b[sh]);
    const float g = expf(-expf(a_log[h]) * softplus(a[sh] + dt_bias[h]));
    float4* S = reinterpret_cast<float4*>(ssm_state) + static_cast<size_t>(sh) * (128 * 32);
    constexpr int kPairs = kDnRowsPerBlock / 8;  // row pairs per wave
    float4 s[kPairs];
    int rl[kPairs];
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        rl[i] = wave * (kDnRowsPerBlock / 4) + i * 2 + (lane >> 5);
        s[i] = S[(rb * kDnRowsPerBlock + rl[i]) * 32 + col4];
    }
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        float4 v = s[i];
        v.x *= g; v.y *= g; v.z *= g; v.w *= g;
        const float kv = group_sum<32>(dot4(v, k4));
        const float delta = (v_s[rl[i]] - kv) * beta;
        v.x = fmaf(k4.x, delta, v.x); v.y = fmaf(k4.y, delta, v.y);
        v.z = fmaf(k4.z, delta, v.z); v.w = fmaf(k4.w, delta, v.w);
        const int row = rb * kDnRowsPerBlock + rl[i];
        S[row * 32 + col4] = v;
        const float o = group_sum<32>(dot4(v, q4));
        if (col4 == 0) o_raw[static_cast<size_t>(sh) * 128 + row] = o;
    }

    // ---- phase 3: last arriver of the key head finishes ------------------------
    __threadfence();
    __syncthreads();
    if (t == 0) {
        const int prev = atomicAdd(&counters[seq * 16 + kh], 1);
        is_last = (prev == 2 * kDnRowBlocks - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    reinterpret_cast<float4*>(conv_state)[seq_ch + ch] = ns;
    // gated RMSNorm of value heads 2kh (waves 0-1) and 2kh+1 (waves 2-3):
    // QwenDeltaNetKernel.swift:127-151; deltanet.metal:337-355.
    const int hh = 2 * kh + (t >> 7), r = t & 127;
    const float o = o_raw[static_cast<size_t>(seq * 32 + hh) * 128 + r];
    const float oss = group_sum<64>(o * o);
    if (lane == 0) red[wave] = oss;
    __syncthreads();
    const float tot = (t < 128) ? (red[0] + red[1]) : (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / 128.0f + eps);
    const size_t oi = static_cast<size_t>(seq) * 4096 + hh * 128 + r;
    elem<OUT_DT>::store(out, oi, o * inv * norm_w[r] * silu(elem<IN_DT>::load(z, oi)));
    if (t == 0) counters[seq * 16 + kh] = 0;
}

hipError_t launch_deltanet_decode(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                  const void* qkv, const void* z, qff_dtype in_dtype,
                                  const float* a, const float* b, float* conv_state,
                                  float* ssm_state, void* out, qff_dtype out_dtype, int batch) {
    dim3 grid(kDnRowBlocks, 32, batch);
    ProfScope prof(ctx, stream, "deltanet_decode");
#define QFF_DN_LAUNCH(I, O)                                                                   \
    deltanet_decode_kernel<I, O><<<grid, 256, 0, stream>>>(qkv, z, a, b, p->a_log, p->dt_bias, \
                                                           p->conv_w, p->norm_w, p->eps,      \
                                                           conv_state, ssm_state,             \
                                                           ctx->dn_o_raw, ctx->dn_counters, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_DN_LAUNCH(1, 1); else QFF_DN_LAUNCH(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_DN_LAUNCH(0, 1); else QFF_DN_LAUNCH(0, 0);
    }
#undef QFF_DN_LAUNCH
    return hipGetLastError();
}

}  // namespace qff
