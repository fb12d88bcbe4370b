// router.hip -- MoE router of a decoder layer on gfx950: affine-Q8 logits
// and top-8 expert selection.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1177-1190 dispatches
// qwen_router_q8_logits_simd_f32 (deltanet.metal:2229-2281: one SIMD group
// per expert row, the factored accumulation scale * sum(q x) + bias * sum(x)
// per 64-column group) and qwen_router_top8_logits_f32 (:2283-2329: the eight
// largest logits by insertion, ties keeping the lower expert index, softmax
// over all logits, the eight probabilities renormalised).
//
// Format (MLX affine Q8, group 64, deltanet.metal:863-900): element c of row
// r is byte c of the row, i.e. byte c % 4 (lowest first) of uint32 word
// w[r * cols/4 + c/4]; value = byte * scale[r, c/64] + bias[r, c/64].
//
// Two kernels:
//   router_logits_kernel  one wave per (expert row, block of NT tokens): lane l
//       holds bytes 32l .. 32l+31 of each 2048-column piece (two 16-B loads),
//       converts them with v_cvt_f32_ubyte and accumulates in fp32 in the
//       factored form; a lane-group sum per token. x stays fp32. All NT
//       tokens' x loads are issued together and the logits stored at the
//       end (a store between tokens would hold the next token's loads:
//       vmcnt counts stores too).
//   router_top8_kernel    one wave per token: the logits in registers (up to
//       4 per lane), eight rounds of a wave maximum (DPP) and a ballot for
//       the lowest index holding it, then the reference's softmax and
//       renormalisation.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

// tokens per logits workgroup: 1 for a single token, else 4 (at batch 16,
// 4 tokens a wave: logits 7.7-7.8 us event-timed, against 11.3 with 8 and
// 7.9-8.0 with 2; 12.3 with 8 tokens a wave each waiting for the previous
// one's store)
static int rt_tokens(int batch) { return batch <= 1 ? 1 : 4; }

template <int I>
__device__ __forceinline__ float rt_ubyte(uint32_t v) { return static_cast<float>((v >> (8 * I)) & 0xffu); }

// grid (ceil(E / 4), ceil(batch / NT)), 256 threads; KW = 2048-column pieces
template <int SB_DT, int X_DT, int KW, int NT>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ biases,
                                                            const void* __restrict__ x, float* __restrict__ logits,
                                                            int experts, int cols, int batch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = blockIdx.x * 4 + wave;
    const int ec = min(e, experts - 1);
    const int m0 = blockIdx.y * NT;
    const int G = cols / 64, W4 = cols / 4, npc = cols / 32;   // 32-byte pieces per row
    u32x4_t wq[KW][2];
    float sv[KW], bv[KW];
    bool live[KW];
#pragma unroll
    for (int k = 0; k < KW; ++k) {
        const int pc = lane + 64 * k;
        live[k] = pc < npc;
        const int pcc = min(pc, npc - 1);
        const uint32_t* src = w + static_cast<size_t>(ec) * W4 + 8 * pcc;
        wq[k][0] = *reinterpret_cast<const u32x4_t*>(src);
        wq[k][1] = *reinterpret_cast<const u32x4_t*>(src + 4);
        sv[k] = elem<SB_DT>::load(scales, static_cast<size_t>(ec) * G + pcc / 2);
        bv[k] = elem<SB_DT>::load(biases, static_cast<size_t>(ec) * G + pcc / 2);
    }
    // every token of the block, its index clamped into the batch, so no load
    // waits behind a branch or a store
    float accs[NT];
#pragma unroll
    for (int mi = 0; mi < NT; ++mi) {
        const int m = min(m0 + mi, batch - 1);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int pcc = min(lane + 64 * k, npc - 1);
            float xv[32];
            if (X_DT == 1) {
                const uint16_t* xp = static_cast<const uint16_t*>(x) + static_cast<size_t>(m) * cols + 32 * pcc;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4_t u = *reinterpret_cast<const u32x4_t*>(xp + 8 * q);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        xv[8 * q + 2 * j] = __uint_as_float(u[j] << 16);
                        xv[8 * q + 2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
                    }
                }
            } else {
                const float4* xp =
                    reinterpret_cast<const float4*>(static_cast<const float*>(x) + static_cast<size_t>(m) * cols + 32 * pcc);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 f = xp[q];
                    xv[4 * q] = f.x;
                    xv[4 * q + 1] = f.y;
                    xv[4 * q + 2] = f.z;
                    xv[4 * q + 3] = f.w;
                }
            }
            float dot = 0.0f, sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t wd = wq[k][j >> 2][j & 3];
                dot = fmaf(rt_ubyte<0>(wd), xv[4 * j], dot);
                dot = fmaf(rt_ubyte<1>(wd), xv[4 * j + 1], dot);
                dot = fmaf(rt_ubyte<2>(wd), xv[4 * j + 2], dot);
                dot = fmaf(rt_ubyte<3>(wd), xv[4 * j + 3], dot);
                sum += (xv[4 * j] + xv[4 * j + 1]) + (xv[4 * j + 2] + xv[4 * j + 3]);
            }
            // half a group per lane; pieces past the row end (cols < 2048) add nothing
            const float sk = live[k] ? sv[k] : 0.0f, bk = live[k] ? bv[k] : 0.0f;
            acc = fmaf(sk, dot, acc);
            acc = fmaf(bk, sum, acc);
        }
        accs[mi] = group_sum<64>(acc);
    }
    if (lane == 0 && e < experts) {
#pragma unroll
        for (int mi = 0; mi < NT; ++mi)
            if (m0 + mi < batch) logits[static_cast<size_t>(m0 + mi) * experts + e] = accs[mi];
    }
}

// grid ceil(batch / 4), 256 threads: wave w ranks token 4 blockIdx.x + w.
__global__ __launch_bounds__(256) void router_top8_kernel(const float* __restrict__ logits,
                                                          int32_t* __restrict__ indices, float* __restrict__ scores,
                                                          int experts, int batch) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= batch) return;   // wave-uniform
    const float* lg = logits + static_cast<size_t>(m) * experts;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = lane + 64 * j;
        v[j] = i < experts ? lg[i] : -INFINITY;
    }
    bool taken[4] = {false, false, false, false};
    float top_v[8];
    int top_i[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        // the largest untaken logit, then its lowest index: the index blocks
        // j hold experts 64j .. 64j+63 in lane order, so the first block
        // whose ballot hits gives the lowest index through its lowest lane
        float lm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < experts && !taken[j]) lm = fmaxf(lm, v[j]);
        const float wm = group_max<64>(lm);
        int idx = -1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned long long hit = __ballot(lane + 64 * j < experts && !taken[j] && v[j] == wm);
            if (idx < 0 && hit) idx = 64 * j + __ffsll(static_cast<long long>(hit)) - 1;
        }
        top_v[k] = wm;
        top_i[k] = idx;
#pragma unroll
        for (int j = 0; j < 4; ++j) taken[j] = taken[j] || idx == lane + 64 * j;
    }
    // softmax over all logits with the top value as the shift, eight
    // probabilities renormalised
    const float mx = top_v[0];
    float den = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < experts) den += expf(v[j] - mx);
    den = group_sum<64>(den);
    float p[8], tot = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        p[k] = expf(top_v[k] - mx) / den;
        tot += p[k];
    }
    if (lane < 8) {
        float pk = p[0];
        int ik = top_i[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            pk = lane == k ? p[k] : pk;
            ik = lane == k ? top_i[k] : ik;
        }
        indices[static_cast<size_t>(m) * 8 + lane] = ik;
        scores[static_cast<size_t>(m) * 8 + lane] = pk / tot;
    }
}

// Q8 dequant test hook: one word (4 bytes) per thread -> 4 floats.
template <int SB_DT>
__global__ __launch_bounds__(256) void q8_dequant_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         float* __restrict__ out, int rows, int cols) {
    const size_t words = static_cast<size_t>(rows) * (cols / 4);
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const int r = static_cast<int>(i / (cols / 4));
    const int c0 = static_cast<int>(i % (cols / 4)) * 4;
    const size_t gi = static_cast<size_t>(r) * (cols / 64) + c0 / 64;
    const float s = elem<SB_DT>::load(scales, gi);
    const float b = elem<SB_DT>::load(biases, gi);
    const uint32_t word = w[i];
    reinterpret_cast<float4*>(out + static_cast<size_t>(r) * cols + c0)[0] =
        make_float4(rt_ubyte<0>(word) * s + b, rt_ubyte<1>(word) * s + b, rt_ubyte<2>(word) * s + b,
                    rt_ubyte<3>(word) * s + b);
}

hipError_t launch_q8_dequant(hipStream_t stream, const uint32_t* w, const void* scales, const void* biases,
                             qff_dtype sb_dtype, float* out, int rows, int cols) {
    const size_t words = static_cast<size_t>(rows) * (cols / 4);
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    const uint16_t* s = static_cast<const uint16_t*>(scales);
    const uint16_t* b = static_cast<const uint16_t*>(biases);
    if (sb_dtype == QFF_BF16) q8_dequant_kernel<1><<<blocks, 256, 0, stream>>>(w, s, b, out, rows, cols);
    else q8_dequant_kernel<2><<<blocks, 256, 0, stream>>>(w, s, b, out, rows, cols);
    return hipGetLastError();
}

hipError_t launch_router_top8(qff_ctx* ctx, hipStream_t stream, const uint32_t* w, const void* scales,
                              const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                              float* logits, int32_t* indices, float* scores, int experts, int cols, int batch) {
    const uint16_t* s = static_cast<const uint16_t*>(scales);
    const uint16_t* b = static_cast<const uint16_t*>(biases);
    const int nt = rt_tokens(batch);
    const dim3 grid((experts + 3) / 4, (batch + nt - 1) / nt);
    const bool k2 = cols > 2048;
    {
        ProfScope prof(ctx, stream, "router_logits");
#define QFF_RL_NT(S, X, K)                                                                                     \
    if (nt == 1) router_logits_kernel<S, X, K, 1><<<grid, 256, 0, stream>>>(w, s, b, x, logits, experts, cols, batch); \
    else router_logits_kernel<S, X, K, 4><<<grid, 256, 0, stream>>>(w, s, b, x, logits, experts, cols, batch)
#define QFF_RL(S, X)                   \
    if (k2) { QFF_RL_NT(S, X, 2); }     \
    else { QFF_RL_NT(S, X, 1); }
#define QFF_RL_X(S) \
    if (x_dtype == QFF_BF16) { QFF_RL(S, 1); } else { QFF_RL(S, 0); }
        if (sb_dtype == QFF_BF16) { QFF_RL_X(1); } else { QFF_RL_X(2); }
#undef QFF_RL_X
#undef QFF_RL
#undef QFF_RL_NT
    }
    ProfScope prof(ctx, stream, "router_top8");
    router_top8_kernel<<<(batch + 3) / 4, 256, 0, stream>>>(logits, indices, scores, experts, batch);
    return hipGetLastError();
}

}  // namespace qff
