// deltanet_decode.hip -- one decode step of the Gated DeltaNet layer core on
// gfx950.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1001-1022 dispatches
// qwen_conv1d_f32 (deltanet.metal:112-138) then qwen_fused_deltanet_step_f32
// (deltanet.metal:250-356) with one 128-thread threadgroup per value head.
//
// Batch > 4: one launch, one 1024-thread workgroup per (key head,
// sequence). A key head's q/k channels feed value heads 2kh and 2kh+1, and
// their conv-state slots are read and rewritten in the same step, so the
// workgroup that owns the key head owns both value heads: every conv-state
// slot and state row then has exactly one owner and no workgroup waits for
// another (a cross-workgroup handshake needs a device-scope fence, which on
// the multi-XCD MI355X writes back L2 and costs far more than the step).
//   phase 1  threads 0-511: conv + SiLU of the 128 q, 128 k and 256 v
//            channels, conv state rewritten in place; q and k L2-normalised
//            (q then / sqrt(128)) in LDS;
//   phase 2  16 waves x 16 state rows (waves 0-7 value head 2kh, 8-15 value
//            head 2kh+1); each lane streams 8 float4 of state (lanes 0-31
//            row r, 32-63 row r+1, column block lane % 32), all loads in
//            flight at once, then decay, k^T S, the rank-1 update and S q
//            with 32-lane butterfly sums;
//   phase 3  gated RMSNorm of both heads from LDS.
// Batch <= 4: 16 workgroups per sequence would leave the chip idle, so the
// step is split over 256 workgroups per sequence in two launches; every
// workgroup of the first reads the old conv state, the second writes it:
//   dn_decode_state_kernel  grid (32 value heads x 8 row parts, batch), 256
//       threads: conv + SiLU of the key head's q and k channels and the
//       part's v channels (conv state read only), L2 norms, then the 16
//       state rows of the part as above (2 float4 per lane); pre-norm output
//       rows to the context workspace;
//   dn_decode_norm_kernel  grid (32 heads, batch): gated RMSNorm of each
//       head's output, and the conv-state shift of 256 channels per
//       workgroup.
// Traffic per sequence-step: 2 MiB state read + 2 MiB written, 16 B per
// lane, fully coalesced; the rest is ~0.2 MiB.
#include "common.hpp"
#include "internal.hpp"

namespace qff {

constexpr int kDnSplitMaxBatch = 4;   // largest batch that takes the two-launch split

template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(1024) void deltanet_decode_kernel(
    const void* __restrict__ qkv, const void* __restrict__ z, const float* __restrict__ a,
    const float* __restrict__ b, const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    const float* __restrict__ conv_w, const float* __restrict__ norm_w, float eps,
    float* __restrict__ conv_state, float* __restrict__ ssm_state, void* __restrict__ out) {
    const int kh = blockIdx.x, seq = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

    __shared__ __attribute__((aligned(16))) float q_s[128];
    __shared__ __attribute__((aligned(16))) float k_s[128];
    __shared__ float v_s[256], o_s[256], red[16], gb[4];

    // ---- phase 1: conv + SiLU (deltanet.metal:120-137), L2 norms (:282-305) ----
    // Its loads go first, then the phase-2 state loads, which do not depend
    // on phase 1 and stream while it computes (loads complete in issue order,
    // so phase 1 waits for its own loads only).
    const size_t seq_ch = static_cast<size_t>(seq) * 8192;
    // threads 512+ load a clamped channel too (no branch around the loads)
    const int ch = min(t < 128 ? kh * 128 + t : t < 256 ? 2048 + kh * 128 + (t - 128) : 4096 + kh * 256 + (t - 256),
                       8191);
    float4* sp = reinterpret_cast<float4*>(conv_state) + seq_ch + ch;
    const float4 st = *sp;
    const float4 w4 = reinterpret_cast<const float4*>(conv_w)[ch];
    const float xin = elem<IN_DT>::load(qkv, seq_ch + ch);
    const int hg = 2 * kh + (t & 1), sg = seq * 32 + hg;   // gate inputs (used by threads 0, 1)
    const float a_in = a[sg], b_in = b[sg], alog = a_log[hg], dtb = dt_bias[hg];
    const size_t oi = static_cast<size_t>(seq) * 4096 + kh * 256 + (t & 255);   // phase-3 output index
    const float zin = elem<IN_DT>::load(z, oi), nw = norm_w[t & 127];
    __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the state stream
    const int hsel = wave >> 3;                 // 0: head 2kh, 1: head 2kh+1
    const int h = 2 * kh + hsel;
    const int col4 = lane & 31;
    const int rbase = (wave & 7) * 16 + (lane >> 5);
    float4* S = reinterpret_cast<float4*>(ssm_state) + (static_cast<size_t>(seq) * 32 + h) * (128 * 32);
    float4 s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = S[(rbase + 2 * i) * 32 + col4];
    __builtin_amdgcn_sched_barrier(0);
    // computed by every thread (used by 0-511) so the loads stay where they are
    const float4 ns = make_float4(st.y, st.z, st.w, xin);
    float y = silu(ns.x * w4.x + ns.y * w4.y + ns.z * w4.z + ns.w * w4.w);
    if (t >= 256 && t < 512) v_s[t - 256] = y;
    if (t < 256) {
        const float ss = group_sum<64>(y * y);
        if (lane == 0) red[wave] = ss;
    }
    if (t < 2) {
        // per value head: beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias))
        gb[2 * t] = expf(-expf(alog) * softplus(a_in + dtb));
        gb[2 * t + 1] = sigmoid(b_in);
    }
    __syncthreads();
    if (t < 256) {
        const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
        const float inv = 1.0f / sqrtf(tot + 1e-6f);
        if (t < 128) q_s[t] = (y * inv) * (1.0f / sqrtf(128.0f));
        else k_s[t - 128] = y * inv;
    }
    __syncthreads();

    // ---- phase 2: gated delta rule, 16 rows per wave --------------------------
    // QwenDeltaNetKernel.swift:86-124; deltanet.metal:307-335.
    const float4 k4 = reinterpret_cast<const float4*>(k_s)[col4];
    const float4 q4 = reinterpret_cast<const float4*>(q_s)[col4];
    const float g = gb[2 * hsel], beta = gb[2 * hsel + 1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 v = s[i];
        v.x *= g; v.y *= g; v.z *= g; v.w *= g;
        const float kv = group_sum<32>(dot4(v, k4));
        const int r = rbase + 2 * i;
        const float delta = (v_s[hsel * 128 + r] - kv) * beta;
        v.x = fmaf(k4.x, delta, v.x); v.y = fmaf(k4.y, delta, v.y);
        v.z = fmaf(k4.z, delta, v.z); v.w = fmaf(k4.w, delta, v.w);
        S[r * 32 + col4] = v;
        const float o = group_sum<32>(dot4(v, q4));
        if (col4 == 0) o_s[hsel * 128 + r] = o;
    }
    __syncthreads();

    // the conv-state rewrite waits until here: a store pending at the phase-1
    // barriers would make them wait for the state loads issued before it
    if (t < 512) *sp = ns;

    // ---- phase 3: gated RMSNorm (QwenDeltaNetKernel.swift:127-151) ------------
    float o = 0.0f;
    if (t < 256) {
        o = o_s[t];
        const float ss = group_sum<64>(o * o);
        if (lane == 0) red[4 + wave] = ss;
    }
    __syncthreads();
    if (t < 256) {
        const float tot = t < 128 ? red[4] + red[5] : red[6] + red[7];
        const float inv = 1.0f / sqrtf(tot / 128.0f + eps);
        elem<OUT_DT>::store(out, oi, o * inv * nw * silu(zin));
    }
}

template <int IN_DT, int R>
__global__ __launch_bounds__(256) void dn_decode_state_kernel(
    const void* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias, const float* __restrict__ conv_w,
    const float* __restrict__ conv_state, float* __restrict__ ssm_state, float* __restrict__ o_pre) {
    constexpr int kRows = 128 / R;          // state rows of this workgroup
    constexpr int kNS = 16 / R;             // float4 of state per lane
    const int h = blockIdx.x / R, part = blockIdx.x % R, kh = h >> 1, seq = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r0 = part * kRows;

    __shared__ __attribute__((aligned(16))) float q_s[128];
    __shared__ __attribute__((aligned(16))) float k_s[128];
    __shared__ float v_s[kRows], red[4], gb[2];

    // the state rows first: their loads are the bulk of the step and depend on
    // nothing computed here
    const int col4 = lane & 31;
    const int rloc = wave * (kRows / 4) + (lane >> 5);   // row within the part
    float4* S = reinterpret_cast<float4*>(ssm_state) + (static_cast<size_t>(seq) * 32 + h) * (128 * 32);
    float4 s[kNS];
#pragma unroll
    for (int i = 0; i < kNS; ++i) s[i] = S[(r0 + rloc + 2 * i) * 32 + col4];

    // ---- conv + SiLU (deltanet.metal:120-137), L2 norms (:282-305) ----------
    const size_t seq_ch = static_cast<size_t>(seq) * 8192;
    const int ch = t < 128 ? kh * 128 + t : 2048 + kh * 128 + (t - 128);
    const float4 st = reinterpret_cast<const float4*>(conv_state)[seq_ch + ch];
    const float4 w4 = reinterpret_cast<const float4*>(conv_w)[ch];
    const float x = elem<IN_DT>::load(qkv, seq_ch + ch);
    const bool has_v = t < kRows;
    const int vch = 4096 + h * 128 + r0 + (has_v ? t : 0);
    const float4 vst = reinterpret_cast<const float4*>(conv_state)[seq_ch + vch];
    const float4 vw4 = reinterpret_cast<const float4*>(conv_w)[vch];
    const float vx = elem<IN_DT>::load(qkv, seq_ch + vch);
    const float y = silu(st.y * w4.x + st.z * w4.y + st.w * w4.z + x * w4.w);
    if (has_v) v_s[t] = silu(vst.y * vw4.x + vst.z * vw4.y + vst.w * vw4.z + vx * vw4.w);
    {
        const float ss = group_sum<64>(y * y);
        if (lane == 0) red[wave] = ss;
    }
    if (t == 0) {
        // beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias))
        const int sh = seq * 32 + h;
        gb[0] = expf(-expf(a_log[h]) * softplus(a[sh] + dt_bias[h]));
        gb[1] = sigmoid(b[sh]);
    }
    __syncthreads();
    {
        const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
        const float inv = 1.0f / sqrtf(tot + 1e-6f);
        if (t < 128) q_s[t] = (y * inv) * (1.0f / sqrtf(128.0f));
        else k_s[t - 128] = y * inv;
    }
    __syncthreads();

    // ---- gated delta rule on the part's rows ---------------------------------
    // QwenDeltaNetKernel.swift:86-124; deltanet.metal:307-335.
    const float4 k4 = reinterpret_cast<const float4*>(k_s)[col4];
    const float4 q4 = reinterpret_cast<const float4*>(q_s)[col4];
    const float g = gb[0], beta = gb[1];
    float* op = o_pre + static_cast<size_t>(seq) * 4096 + h * 128 + r0;
#pragma unroll
    for (int i = 0; i < kNS; ++i) {
        float4 v = s[i];
        v.x *= g; v.y *= g; v.z *= g; v.w *= g;
        const float kv = group_sum<32>(dot4(v, k4));
        const int r = rloc + 2 * i;
        const float delta = (v_s[r] - kv) * beta;
        v.x = fmaf(k4.x, delta, v.x); v.y = fmaf(k4.y, delta, v.y);
        v.z = fmaf(k4.z, delta, v.z); v.w = fmaf(k4.w, delta, v.w);
        S[(r0 + r) * 32 + col4] = v;
        const float o = group_sum<32>(dot4(v, q4));
        if (col4 == 0) op[r] = o;
    }
}

// Gated RMSNorm (QwenDeltaNetKernel.swift:127-151) of head h, and the conv
// state shift of channels 128h .. 128h+127 (q/k block) and 4096 + 128h ..
// (v block): slot j <- slot j+1, slot 3 <- x_t (deltanet.metal:120-137).
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void dn_decode_norm_kernel(
    const void* __restrict__ qkv, const void* __restrict__ z, const float* __restrict__ norm_w, float eps,
    const float* __restrict__ o_pre, float* __restrict__ conv_state, void* __restrict__ out) {
    const int h = blockIdx.x, seq = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    __shared__ float red[2];
    const size_t oi = static_cast<size_t>(seq) * 4096 + h * 128 + (t & 127);
    float o = 0.0f;
    if (t < 128) {
        o = o_pre[oi];
        const float ss = group_sum<64>(o * o);
        if (lane == 0) red[wave] = ss;
    }
    {
        const size_t ch = static_cast<size_t>(seq) * 8192 + (t < 128 ? 0 : 4096) + h * 128 + (t & 127);
        float4* sp = reinterpret_cast<float4*>(conv_state) + ch;
        const float4 st = *sp;
        *sp = make_float4(st.y, st.z, st.w, elem<IN_DT>::load(qkv, ch));
    }
    __syncthreads();
    if (t < 128) {
        const float inv = 1.0f / sqrtf((red[0] + red[1]) / 128.0f + eps);
        elem<OUT_DT>::store(out, oi, o * inv * norm_w[t] * silu(elem<IN_DT>::load(z, oi)));
    }
}

hipError_t launch_deltanet_decode(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                  const void* qkv, const void* z, qff_dtype in_dtype,
                                  const float* a, const float* b, float* conv_state,
                                  float* ssm_state, void* out, qff_dtype out_dtype, int batch) {
    ProfScope prof(ctx, stream, "deltanet_decode");
    const bool bf_in = in_dtype == QFF_BF16, bf_out = out_dtype == QFF_BF16;
    if (batch > kDnSplitMaxBatch) {
#define QFF_DN_LAUNCH(I, O)                                                                               \
    deltanet_decode_kernel<I, O><<<dim3(16, batch), 1024, 0, stream>>>(qkv, z, a, b, p->a_log, p->dt_bias, \
                                                                       p->conv_w, p->norm_w, p->eps,      \
                                                                       conv_state, ssm_state, out)
        if (bf_in) {
            if (bf_out) QFF_DN_LAUNCH(1, 1); else QFF_DN_LAUNCH(1, 0);
        } else {
            if (bf_out) QFF_DN_LAUNCH(0, 1); else QFF_DN_LAUNCH(0, 0);
        }
#undef QFF_DN_LAUNCH
        return hipGetLastError();
    }
    constexpr int R = 8;   // row parts per head (4 and 16 measured slower at batch 1)
    const dim3 sgrid(32 * R, batch), ngrid(32, batch);
    if (bf_in)
        dn_decode_state_kernel<1, R><<<sgrid, 256, 0, stream>>>(qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                conv_state, ssm_state, ctx->dn_o);
    else
        dn_decode_state_kernel<0, R><<<sgrid, 256, 0, stream>>>(qkv, a, b, p->a_log, p->dt_bias, p->conv_w,
                                                                conv_state, ssm_state, ctx->dn_o);
#define QFF_DN_NORM(I, O)                                                                             \
    dn_decode_norm_kernel<I, O><<<ngrid, 256, 0, stream>>>(qkv, z, p->norm_w, p->eps, ctx->dn_o, \
                                                           conv_state, out)
    if (bf_in) {
        if (bf_out) QFF_DN_NORM(1, 1); else QFF_DN_NORM(1, 0);
    } else {
        if (bf_out) QFF_DN_NORM(0, 1); else QFF_DN_NORM(0, 0);
    }
#undef QFF_DN_NORM
    return hipGetLastError();
}

}  // namespace qff
