// deltanet_decode.hip -- one decode step of the Gated DeltaNet layer core on
// gfx950.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1001-1022 dispatches
// qwen_conv1d_f32 (deltanet.metal:112-138) then qwen_fused_deltanet_step_f32
// (deltanet.metal:250-356) with one 128-thread threadgroup per value head.
//
// One launch at every batch size, one workgroup per (value head, sequence)
// (dn_decode_head_kernel below). Traffic per sequence-step: 2 MiB state read
// + 2 MiB written, 16 B per lane, fully coalesced; the rest is ~0.2 MiB.
// Measured against a plain in-place pass over the same state bytes with the
// same access pattern and no compute (cold HBM, graph of back-to-back
// steps): 17.7 vs 15.0 us at batch 16 and 31.6 vs 27.5 us at batch 32;
// 5.1 us at batch 1, where 32 workgroups cannot fill the chip.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {


// One workgroup per (value head, sequence), NT threads (1024 up to batch 16;
// 512 above, at 64 VGPRs, so that four workgroups share a CU and batch 32
// runs in one resident round).
//   phase 1  threads 0-383: conv + SiLU of the key head's 128 q and 128 k
//            channels and the head's 128 v channels, q and k L2-normalised
//            (q then / sqrt(128)) in LDS; the head's 64 KiB of state rows
//            are requested before any of it is computed;
//   phase 2  NT/64 waves x 128/(NT/64) state rows (lanes 0-31 row r, 32-63
//            row r+1, column block lane % 32): decay, k^T S, the rank-1
//            update and S q with 32-lane butterfly sums;
//   phase 3  gated RMSNorm of the head from LDS.
// The two value heads of a key head read the same q/k conv-state slots, and
// the slots are rewritten in the same step. Each workgroup counts itself in
// on a per-(sequence, key head) counter after phase 2, when every one of its
// conv-state reads has long returned (their values were consumed before the
// first barrier), and the second one in rewrites the q/k slots and resets
// the counter: the slots are written only after both heads have read them,
// and no workgroup ever waits for another (only an ordering of reads before
// writes is needed, which the counter gives without a fence; counting in
// earlier would hold the phase-2 barrier for the atomic's return, measured
// 0.4 us slower at batch 1). The v slots of a head are read and written by
// its own workgroup.
template <int IN_DT, int OUT_DT, int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT == 512 ? 8 : 4))) void dn_decode_head_kernel(
    const void* __restrict__ qkv, const void* __restrict__ z, const float* __restrict__ a,
    const float* __restrict__ b, const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    const float* __restrict__ conv_w, const float* __restrict__ norm_w, float eps,
    float* __restrict__ conv_state, float* __restrict__ ssm_state, void* __restrict__ out,
    unsigned* __restrict__ arrivals) {
    constexpr int kWaves = NT / 64, kRowsW = 128 / kWaves, kNS = kRowsW / 2;
    static_assert(NT >= 384 && kNS >= 1 && 128 % kWaves == 0, "384+ threads, 2+ state rows per wave");
    const int h = blockIdx.x, kh = h >> 1, seq = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

    __shared__ __attribute__((aligned(16))) float q_s[128];
    __shared__ __attribute__((aligned(16))) float k_s[128];
    __shared__ float v_s[128], o_s[128], red[8], gb[2];
    __shared__ int qk_last;

    // ---- phase 1: conv + SiLU (deltanet.metal:120-137), L2 norms (:282-305) ----
    const size_t seq_ch = static_cast<size_t>(seq) * 8192;
    // threads 384+ load the head's last v channel again (no branch around the loads)
    const int tc = min(t, 383);
    const int ch = tc < 128 ? kh * 128 + tc : tc < 256 ? 2048 + kh * 128 + (tc - 128) : 4096 + h * 128 + (tc - 256);
    float4* sp = reinterpret_cast<float4*>(conv_state) + seq_ch + ch;
    const float4 st = *sp;
    const float4 w4 = reinterpret_cast<const float4*>(conv_w)[ch];
    const float xin = elem<IN_DT>::load(qkv, seq_ch + ch);
    const int sg = seq * 32 + h;
    const float a_in = a[sg], b_in = b[sg], alog = a_log[h], dtb = dt_bias[h];
    const size_t oi = static_cast<size_t>(seq) * 4096 + h * 128 + (t & 127);   // phase-3 output index
    const float zin = elem<IN_DT>::load(z, oi), nw = norm_w[t & 127];
    __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the state stream
    const int col4 = lane & 31;
    const int rbase = wave * kRowsW + (lane >> 5);
    float4* S = reinterpret_cast<float4*>(ssm_state) + (static_cast<size_t>(seq) * 32 + h) * (128 * 32);
    float4 s[kNS];
#pragma unroll
    for (int i = 0; i < kNS; ++i) {
        // the state streams through once a step: non-temporal loads and
        // stores (`nt`) keep it from displacing the caches' other contents
        // (batch 32: 27.2 against 31.6 us a step; batch 16: 15.3 against 17.8)
        const f32x4_t u = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(S) + (rbase + 2 * i) * 32 + col4);
        s[i] = make_float4(u[0], u[1], u[2], u[3]);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float4 ns = make_float4(st.y, st.z, st.w, xin);
    const float y = silu(ns.x * w4.x + ns.y * w4.y + ns.z * w4.z + ns.w * w4.w);
    if (t >= 256 && t < 384) v_s[t - 256] = y;
    if (t < 256) {
        const float ss = group_sum<64>(y * y);
        if (lane == 0) red[wave] = ss;
    }
    if (t == 0) {
        // beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias))
        gb[0] = expf(-expf(alog) * softplus(a_in + dtb));
        gb[1] = sigmoid(b_in);
    }
    __syncthreads();
    // every conv-state read of the workgroup has returned: count it in
    if (t < 256) {
        const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
        const float inv = 1.0f / sqrtf(tot + 1e-6f);
        if (t < 128) q_s[t] = (y * inv) * (1.0f / sqrtf(128.0f));
        else k_s[t - 128] = y * inv;
    }
    __syncthreads();

    // ---- phase 2: gated delta rule (QwenDeltaNetKernel.swift:86-124;
    // deltanet.metal:307-335) ------------------------------------------------
    const float4 k4 = reinterpret_cast<const float4*>(k_s)[col4];
    const float4 q4 = reinterpret_cast<const float4*>(q_s)[col4];
    const float g = gb[0], beta = gb[1];
#pragma unroll
    for (int i = 0; i < kNS; ++i) {
        float4 v = s[i];
        v.x *= g; v.y *= g; v.z *= g; v.w *= g;
        const float kv = group_sum<32>(dot4(v, k4));
        const int r = rbase + 2 * i;
        const float delta = (v_s[r] - kv) * beta;
        v.x = fmaf(k4.x, delta, v.x); v.y = fmaf(k4.y, delta, v.y);
        v.z = fmaf(k4.z, delta, v.z); v.w = fmaf(k4.w, delta, v.w);
        __builtin_nontemporal_store(f32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_t*>(S) + r * 32 + col4);
        const float o = group_sum<32>(dot4(v, q4));
        if (col4 == 0) o_s[r] = o;
    }
    if (t == 0) qk_last = atomicAdd(&arrivals[seq * 16 + kh], 1u) == 1u;
    __syncthreads();

    // conv state after the token: the head's v slots always, the key head's
    // q/k slots by its second workgroup in (which also resets the counter)
    if ((t >= 256 && t < 384) || (t < 256 && qk_last)) *sp = ns;
    if (t == 0 && qk_last) atomicExch(&arrivals[seq * 16 + kh], 0u);

    // ---- phase 3: gated RMSNorm (QwenDeltaNetKernel.swift:127-151) ------------
    float o = 0.0f;
    if (t < 128) {
        o = o_s[t];
        const float ss = group_sum<64>(o * o);
        if (lane == 0) red[4 + wave] = ss;
    }
    __syncthreads();
    if (t < 128) {
        const float inv = 1.0f / sqrtf((red[4] + red[5]) / 128.0f + eps);
        elem<OUT_DT>::store(out, oi, o * inv * nw * silu(zin));
    }
}

hipError_t launch_deltanet_decode(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                  const void* qkv, const void* z, qff_dtype in_dtype,
                                  const float* a, const float* b, float* conv_state,
                                  float* ssm_state, void* out, qff_dtype out_dtype, int batch) {
    ProfScope prof(ctx, stream, "deltanet_decode");
    const bool bf_in = in_dtype == QFF_BF16, bf_out = out_dtype == QFF_BF16;
    // 1024 threads up to batch 16 (more lanes per head); 512 above (four
    // workgroups per CU). Measured: 512 everywhere is 0.5-0.6 us slower at
    // batch 1-8; 1024 at batch 32 0.6 us slower.
    const int nt = batch <= 16 ? 1024 : 512;
    const dim3 grid(32, batch);
#define QFF_DN_LAUNCH(I, O, N)                                                                        \
    dn_decode_head_kernel<I, O, N><<<grid, N, 0, stream>>>(qkv, z, a, b, p->a_log, p->dt_bias, p->conv_w, \
                                                           p->norm_w, p->eps, conv_state, ssm_state, out,  \
                                                           ctx->dn_arrive)
#define QFF_DN_NT_CASE(N)                                              \
    if (bf_in) {                                                       \
        if (bf_out) QFF_DN_LAUNCH(1, 1, N); else QFF_DN_LAUNCH(1, 0, N); \
    } else {                                                           \
        if (bf_out) QFF_DN_LAUNCH(0, 1, N); else QFF_DN_LAUNCH(0, 0, N); \
    }
    if (nt == 1024) {
        QFF_DN_NT_CASE(1024)
    } else {
        QFF_DN_NT_CASE(512)
    }
#undef QFF_DN_NT_CASE
#undef QFF_DN_LAUNCH
    return hipGetLastError();
}

}  // namespace qff
