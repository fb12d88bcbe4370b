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
//   dn_chunk_local_kernel  persistent, one (chunk, key head) unit at a time
//       from a work queue, all chunks independent: conv1d + SiLU of the
//       chunk's q, k and both value heads' v channels straight from the
//       projection (3 tokens of history from the input or the conv state),
//       L2 norms, gates, the Gram products K K^T and Q K^T once for both
//       value heads, then per value head A, P, T (16x16 blocks: diagonal
//       blocks by substitution, the rest on fp32 MFMAs), W, U~ and Qe;
//       writes W, Qe, K~^T, U~^T, P (bf16 hi/lo) and e^{G_C}.
//   dn_chunk_state_kernel  one workgroup per (16 state rows, value head)
//       walks the chunks in order with its state rows in registers, twelve
//       waves in three roles: U = U~ - W S^T, S = e^{G_C} S + U^T K~ and the
//       pre-norm output O^T = S Qe^T + U~^T P^T. Its MFMA operands come from
//       global memory straight into registers in operand layout, one or two
//       chunks ahead.
// Every product runs as bf16x3 on v_mfma_f32_16x16x32_bf16 (a b ~ a_hi b_hi
// + a_hi b_lo + a_lo b_hi, ~2^-16 relative per product), which keeps the
// fp32 state within 1e-4 of the sequential fp32 recurrence; plain bf16
// operands would not.
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kC = 64;      // chunk length
constexpr int kLD = 136;    // bf16 row stride of [64][128] LDS tiles (128 + 8)
constexpr int kLT = 72;     // bf16 row stride of [64][64] LDS tiles (64 + 8)

// ---- chunk-local pass --------------------------------------------------------

constexpr float kLog2e = 1.44269504088896341f;

// Raw projection pair (channels ch, ch+1) as stored: two bf16 in one word,
// or two floats.
template <int IN_DT> struct RawPair;
template <> struct RawPair<1> {
    uint32_t v;
    __device__ __forceinline__ void load(const void* p, size_t i) {
        v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
    }
    __device__ __forceinline__ float lo() const { return __uint_as_float(v << 16); }
    __device__ __forceinline__ float hi() const { return __uint_as_float(v & 0xffff0000u); }
};
template <> struct RawPair<0> {
    float2 v;
    __device__ __forceinline__ void load(const void* p, size_t i) {
        v = *reinterpret_cast<const float2*>(static_cast<const float*>(p) + i);
    }
    __device__ __forceinline__ float lo() const { return v.x; }
    __device__ __forceinline__ float hi() const { return v.y; }
};

// Everything one (chunk, key head) unit reads from global memory, for one
// thread (wave w: tokens 8w .. 8w+7 of the chunk; lane l: channels 2l, 2l+1
// of the key head's q and k blocks and of the v blocks of its two value
// heads): the conv input rows at positions tok-3 .. tok+7 clamped into
// [0, T), the conv weights, and per value head the gate inputs of token
// lane and the head's A_log and dt_bias. Every load is unconditional and in
// bounds, so the loads of the next unit can be issued while the current one
// is processed and the compiler's vmcnt accounting stays exact. (The
// conv-state slots that chunk 0 needs are read when that unit is processed.)
template <int IN_DT>
struct UnitIn {
    RawPair<IN_DT> r[4][11];
    float4 w[4][2];
    float av[2], bv[2], alog[2], dtb[2];
};

__device__ __forceinline__ void unit_coords(int u, int& c, int& kh) {
    c = u >> 4;
    kh = u & 15;
}

template <int IN_DT>
__device__ __forceinline__ void fetch_unit(UnitIn<IN_DT>& in, int u, int T, const void* __restrict__ qkv,
                                           const float* __restrict__ a, const float* __restrict__ b,
                                           const float* __restrict__ a_log, const float* __restrict__ dt_bias,
                                           const float* __restrict__ conv_w, const float* __restrict__ conv_state,
                                           int wave, int lane) {
    int c, kh;
    unit_coords(u, c, kh);
    const int t0 = c * kC, tw = t0 + 8 * wave;
    const int chs[4] = {kh * 128 + 2 * lane, 2048 + kh * 128 + 2 * lane, 4096 + 2 * kh * 128 + 2 * lane,
                        4096 + (2 * kh + 1) * 128 + 2 * lane};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int j = 0; j < 2; ++j) in.w[p][j] = reinterpret_cast<const float4*>(conv_w)[chs[p] + j];
#pragma unroll
        for (int i = 0; i < 11; ++i) {
            const int pos = min(max(tw - 3 + i, 0), T - 1);
            in.r[p][i].load(qkv, static_cast<size_t>(pos) * 8192 + chs[p]);
        }
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const size_t gi = static_cast<size_t>(min(t0 + lane, T - 1)) * 32 + 2 * kh + hh;
        in.av[hh] = a[gi];
        in.bv[hh] = b[gi];
        in.alog[hh] = a_log[2 * kh + hh];
        in.dtb[hh] = dt_bias[2 * kh + hh];
    }
}

// Conv inputs e[i][c] of pass p, channels ch + c, at positions tw-3+i: the
// projection inside [0, T), 0 past the end (TAIL: the chunk reaches past
// T - 1); before token 0 (wave 0 of chunk 0 only) the conv-state slots
// pos + 4.
template <int IN_DT, bool TAIL>
__device__ __forceinline__ void unit_rows(const UnitIn<IN_DT>& in, int p, int tw, int T, int ch,
                                          const float* __restrict__ conv_state, float (&e)[11][2]) {
#pragma unroll
    for (int i = 0; i < 11; ++i) {
        const int pos = tw - 3 + i;
        e[i][0] = !TAIL || pos < T ? in.r[p][i].lo() : 0.0f;
        e[i][1] = !TAIL || pos < T ? in.r[p][i].hi() : 0.0f;
    }
    if (tw == 0) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            e[i][0] = conv_state[ch * 4 + 1 + i];
            e[i][1] = conv_state[(ch + 1) * 4 + 1 + i];
        }
        // waited for here, on the one wave that reads them: a wait after the
        // branch would hold every wave until the previous unit's stores drain
        __builtin_amdgcn_s_waitcnt(0);
    }
}

// y[i][c] = SiLU(conv1d) of channel ch + c at token tok0 + i (deltanet.metal
// :120-137: taps w.x .. w.w over inputs tok-3 .. tok); 0 for tokens >= T.
template <bool TAIL>
__device__ __forceinline__ void conv2x8(const float (&e)[11][2], const float4 (&w)[2], int tok0, int T,
                                        float (&y)[8][2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = silu_fast(e[i][c] * w[c].x + e[i + 1][c] * w[c].y + e[i + 2][c] * w[c].z +
                                      e[i + 3][c] * w[c].w);
            y[i][c] = !TAIL || tok0 + i < T ? v : 0.0f;
        }
}

// Totals over the 64 lanes of a wave of eight per-lane partials, in every
// lane: a reduce-scatter (exchanges with lane ^ 32, ^ 16, ^ 8 halve the set
// each time), the last three butterfly steps, then one readlane per value.
__device__ __forceinline__ void wave_sum8(const float (&p)[8], float (&tot)[8], int lane) {
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
    float q4[4], q2[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float keep = b5 ? p[4 + j] : p[j], give = b5 ? p[j] : p[4 + j];
        q4[j] = keep + __shfl_xor(give, 32, 64);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float keep = b4 ? q4[2 + j] : q4[j], give = b4 ? q4[j] : q4[2 + j];
        q2[j] = keep + __shfl_xor(give, 16, 64);
    }
    float q1 = (b3 ? q2[1] : q2[0]) + __shfl_xor(b3 ? q2[0] : q2[1], 8, 64);
    q1 += __shfl_xor(q1, 4, 64);
    q1 += __shfl_xor(q1, 2, 64);
    q1 += __shfl_xor(q1, 1, 64);
    // lane L now holds the total of value (L >> 3) & 7
#pragma unroll
    for (int j = 0; j < 8; ++j)
        tot[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q1), 8 * j));
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
// Its inverse: piece p -> (r, k8). Writers walk p with the thread index, so
// each store instruction covers one contiguous 1 KB block.
template <int K>
__device__ __forceinline__ void unswz(int p, int& r, int& k8) {
    const int q = p >> 6;
    r = (q / (K / 32)) * 16 + (p & 15);
    k8 = (q % (K / 32)) * 4 + ((p >> 4) & 3);
}

// bf16x3 block product like mma_block_x3 (NN), with the k elements of A
// scaled by asc[k] on the way in: the A operand (hi, lo) is recombined,
// scaled in fp32 and split again (exact to ~2^-16 like the operands
// themselves).
template <int K, int NC>
__device__ __forceinline__ void mma_block_x3_ascale(f32x4_t (&acc)[1][NC], const uint16_t* ah, const uint16_t* al,
                                                    int lda, int ar, const float* asc, const uint16_t* bh,
                                                    const uint16_t* bl, int ldb, int bc, int lane) {
    const int n = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 32) {
        const int ao = (ar + n) * lda + k0 + 8 * kb;
        const u32x4_t h = *reinterpret_cast<const u32x4_t*>(ah + ao);
        const u32x4_t l = *reinterpret_cast<const u32x4_t*>(al + ao);
        const float4 s0 = *reinterpret_cast<const float4*>(asc + k0 + 8 * kb);
        const float4 s1 = *reinterpret_cast<const float4*>(asc + k0 + 8 * kb + 4);
        const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        u32x4_t a_h, a_l;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x0 = (__uint_as_float(h[e] << 16) + __uint_as_float(l[e] << 16)) * sc[2 * e];
            const float x1 = (__uint_as_float(h[e] & 0xffff0000u) + __uint_as_float(l[e] & 0xffff0000u)) * sc[2 * e + 1];
            uint32_t hw, lw;
            split_bf16x2(x0, x1, hw, lw);
            a_h[e] = hw;
            a_l[e] = lw;
        }
        u32x4_t b_h[NC], b_l[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int bo = (k0 + 8 * kb + (n >> 2)) * ldb + bc + 16 * c + 4 * (n & 3);
            const u32x2_t h0 = lds_read_tr16(bh + bo), h1 = lds_read_tr16(bh + bo + 4 * ldb);
            const u32x2_t l0 = lds_read_tr16(bl + bo), l1 = lds_read_tr16(bl + bo + 4 * ldb);
            b_h[c] = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
            b_l[c] = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[0][c] = mfma_16x16x32_bf16(a_l, b_h[c], acc[0][c]);
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[0][c] = mfma_16x16x32_bf16(a_h, b_l[c], acc[0][c]);
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[0][c] = mfma_16x16x32_bf16(a_h, b_h[c], acc[0][c]);
    }
}

// Packed lower triangle (j <= i) of a 64 x 64 matrix.
__device__ __forceinline__ int tri(int i, int j) { return i * (i + 1) / 2 + j; }

// LDS carve-up of the chunk-local kernel (bytes)
constexpr int kTile128 = kC * kLD * 2;            // one [64][136] bf16 array
constexpr int kOffK = 0;                          // K hi, lo (both value heads)
constexpr int kOffQ = 2 * kTile128;               // Q hi, lo; then T (fp32) + scratch; then W hi, lo
constexpr int kOffV = 4 * kTile128;               // beta V hi, lo; then P W, Qe (fp32 [64][132])
constexpr int kOffA = 6 * kTile128;               // A fp32 [64][65]
constexpr int kOffT = kOffA + kC * 65 * 4;        // P hi, lo, then T hi, lo, then P again: [64][72]
constexpr int kTri = kC * (kC + 1) / 2;           // packed lower triangle
constexpr int kOffR = kOffT + 2 * kC * kLT * 2;   // raw K K^T and Q K^T lower triangles (fp32)
constexpr int kOffG = kOffR + 2 * kTri * 4;       // per value head: G[64], beta[64], beta e^G [64]
constexpr int kLocalSmem = kOffG + 2 * 3 * kC * 4;

// Persistent: grid = min(units, CUs) workgroups of 512 threads (eight
// waves, two per SIMD) walk the (chunk, key head) units. Units 0 .. 2g-1
// go out statically (g = grid size), the rest through an atomic counter, so
// a workgroup on a CU that runs slow (or shares its XCD with other work)
// simply takes fewer units; the launch's last workgroup resets the counter.
// A key head's q and k feed both of its value heads, so a unit runs the
// conv, norms and the Gram products K K^T and Q K^T once and keeps the raw
// products (packed lower triangles) for the second head, whose A and P
// differ only by the per-head gates. Per value head: K~^T out, beta V, A
// and P, T = (I + A)^-1, W = T diag(beta e^G) K (the scaling applied to T's
// operand, so K stays as it is for the other head), U~ = T (beta V), P W
// and Qe. While a unit is processed the inputs of the workgroup's next unit
// are already loading into registers (UnitIn), issued by the second head
// once its T = (I + A)^-1 is complete (earlier, they would not fit the
// registers of the rest of the unit: issuing them on the waves idle during
// the off-diagonal solve spilled 170 registers).
// Conv passes map wave w to tokens 8w .. 8w+7 and lane l to channels 2l,
// 2l+1 of a 128-channel block, so a lane's 8 tokens of a channel are one
// K~^T operand piece and each conv input row is one 256-B load per wave.
// Global loads are issued before the stores of the same head (vmcnt counts
// stores too on gfx950, so a load consumed after stores would wait for them).
constexpr int kLocalThreads = 512;

template <int IN_DT>
__global__ __launch_bounds__(kLocalThreads) void dn_chunk_local_kernel(
    int T, const void* __restrict__ qkv, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ a_log, const float* __restrict__ dt_bias, const float* __restrict__ conv_w,
    const float* __restrict__ conv_state, qff_dn_bufs out, unsigned* __restrict__ sched) {
    const int units = ((T + kC - 1) / kC) * 16;
    const int grid = gridDim.x;

    __shared__ __attribute__((aligned(16))) unsigned char smem[kLocalSmem];
    __shared__ int s_next;
    uint16_t* Kh = reinterpret_cast<uint16_t*>(smem + kOffK);
    uint16_t* Kl = Kh + kC * kLD;
    uint16_t* Qh = reinterpret_cast<uint16_t*>(smem + kOffQ);
    uint16_t* Ql = Qh + kC * kLD;
    uint16_t* Vh = reinterpret_cast<uint16_t*>(smem + kOffV);
    uint16_t* Vl = Vh + kC * kLD;
    float* Am = reinterpret_cast<float*>(smem + kOffA);
    uint16_t* Th = reinterpret_cast<uint16_t*>(smem + kOffT);
    uint16_t* Tl = Th + kC * kLT;
    float* KKr = reinterpret_cast<float*>(smem + kOffR);
    float* QKr = KKr + kTri;
    float* Gs = reinterpret_cast<float*>(smem + kOffG);   // [hh][64]
    float* Bs = Gs + 2 * kC;                              // [hh][64]
    float* Ss = Bs + 2 * kC;                              // [hh][64]: beta e^G

    int u = blockIdx.x, un = blockIdx.x + grid;
    UnitIn<IN_DT> in;
    fetch_unit<IN_DT>(in, u, T, qkv, a, b, a_log, dt_bias, conv_w, conv_state, threadIdx.x >> 6, threadIdx.x & 63);
    if (threadIdx.x == 0) s_next = 2 * grid + static_cast<int>(atomicAdd(sched, 1u));
    // Wait here for the first unit's loads: the loop's own waits then only
    // count the operations of the previous iteration, which issues stores
    // after its prefetch, so consuming the prefetch does not wait for them.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    while (u < units) {
    // thread coordinates re-derived in every iteration through an opaque
    // copy, so the compiler recomputes the index arithmetic built on them
    // where it is used instead of keeping it live across the whole loop
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    const int lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int rt = wave & 3, role = wave >> 2;   // MFMA row tile; which of a wave pair's two products
    int c, kh;
    unit_coords(u, c, kh);
    const int t0 = c * kC;
    const int nv = min(kC, T - t0);
    const int tw = t0 + 8 * wave;                  // this wave's first token

    // gates (deltanet.metal:250-280), waves 0 and 1 one value head each:
    // log g = -e^{A_log} softplus(a + dt_bias), beta = sigmoid(b); G =
    // inclusive prefix sum over the chunk. Padded tokens have log g = 0 and
    // beta = 0, so they change nothing.
    if (wave < 2) {
        const int hh = wave;
        const bool ok = lane < nv;
        const float av = hh ? in.av[1] : in.av[0], bv = hh ? in.bv[1] : in.bv[0];
        const float alog = hh ? in.alog[1] : in.alog[0], dtb = hh ? in.dtb[1] : in.dtb[0];
        float x = ok ? -expf(alog) * softplus(av + dtb) : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        const float beta = ok ? sigmoid(bv) : 0.0f;
        Gs[hh * kC + lane] = x;
        Bs[hh * kC + lane] = beta;
        Ss[hh * kC + lane] = beta * __builtin_amdgcn_exp2f(x * kLog2e);
        if (lane == 63) out.gam[static_cast<size_t>(c) * 32 + 2 * kh + hh] = expf(x);
    }
    const int chs[4] = {kh * 128 + 2 * lane, 2048 + kh * 128 + 2 * lane, 4096 + 2 * kh * 128 + 2 * lane,
                        4096 + (2 * kh + 1) * 128 + 2 * lane};
    const bool tail = t0 + kC > T;
    auto conv = [&](int p, float (&y)[8][2]) {
        float e[11][2];
        if (tail) {
            unit_rows<IN_DT, true>(in, p, tw, T, chs[p], conv_state, e);
            conv2x8<true>(e, in.w[p], tw, T, y);
        } else {
            unit_rows<IN_DT, false>(in, p, tw, T, chs[p], conv_state, e);
            conv2x8<false>(e, in.w[p], tw, T, y);
        }
    };

    // ---- conv + SiLU, L2 norms over each token's 128 channels (deltanet.metal
    // :282-305, q then / sqrt(128)); q, k to LDS as bf16 hi/lo ---------------
    auto norm_store = [&](float (&y)[8][2], float post, uint16_t* dh, uint16_t* dl) {
        float ss[8], tot[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[i] = y[i][0] * y[i][0] + y[i][1] * y[i][1];
        wave_sum8(ss, tot, lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float sc = __builtin_amdgcn_rsqf(tot[i] + 1e-6f) * post;
            y[i][0] *= sc;
            y[i][1] *= sc;
            uint32_t hh, ll;
            split_bf16x2(y[i][0], y[i][1], hh, ll);
            const int o = (8 * wave + i) * kLD + 2 * lane;
            *reinterpret_cast<uint32_t*>(dh + o) = hh;
            *reinterpret_cast<uint32_t*>(dl + o) = ll;
        }
    };
    // (k is kept in LDS only: K~^T is formed from the hi/lo copy)
    float qn[8][2], vn[2][8][2];
    {
        float kn[8][2];
        conv(0, qn);
        norm_store(qn, 0.08838834764831845f, Qh, Ql);   // 1 / sqrt(128)
        conv(1, kn);
        norm_store(kn, 1.0f, Kh, Kl);
    }
    conv(2, vn[0]);
    conv(3, vn[1]);
    __syncthreads();

    // grabbed now, published at the end of the unit, when it has long arrived
    unsigned grabbed = 0;
    if (t == 0) grabbed = atomicAdd(sched, 1u);
    int unn = 0;

#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
    const int h = 2 * kh + hh;
    const size_t ch = static_cast<size_t>(c) * 32 + h;   // (chunk, value head) record
    const float* G = Gs + hh * kC;
    const float* Bt = Bs + hh * kC;

    // ---- K~^T out (channels 2l, 2l+1 x this wave's 8 tokens: one operand
    // piece each), beta v to LDS; A and P -------------------------------------
    {
        const float gc = G[kC - 1];
        float gw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) gw[i] = G[8 * wave + i];
        float kn[8][2];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t kh2 = *reinterpret_cast<const uint32_t*>(Kh + (8 * wave + i) * kLD + 2 * lane);
            const uint32_t kl2 = *reinterpret_cast<const uint32_t*>(Kl + (8 * wave + i) * kLD + 2 * lane);
            kn[i][0] = __uint_as_float(kh2 << 16) + __uint_as_float(kl2 << 16);
            kn[i][1] = __uint_as_float(kh2 & 0xffff0000u) + __uint_as_float(kl2 & 0xffff0000u);
        }
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                split_bf16x2(__builtin_amdgcn_exp2f((gc - gw[2 * j]) * kLog2e) * kn[2 * j][cc],
                             __builtin_amdgcn_exp2f((gc - gw[2 * j + 1]) * kLog2e) * kn[2 * j + 1][cc], hw[j], lw[j]);
            const size_t o = ch * 128 * kC + 8 * swz<kC>(2 * lane + cc, wave);
            *reinterpret_cast<u32x4_t*>(out.kth + o) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
            *reinterpret_cast<u32x4_t*>(out.ktl + o) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float bb = Bt[8 * wave + i];
            uint32_t hq, lq;
            split_bf16x2(bb * vn[hh][i][0], bb * vn[hh][i][1], hq, lq);
            const int o = (8 * wave + i) * kLD + 2 * lane;
            *reinterpret_cast<uint32_t*>(Vh + o) = hq;
            *reinterpret_cast<uint32_t*>(Vl + o) = lq;
        }
    }
    // waves 0-3: K K^T -> A (strictly lower, scaled); waves 4-7: Q K^T -> P
    // (lower incl. diagonal); row tile rt each. The first head forms the
    // products and keeps them raw; the second reads them back.
    {
        f32x4_t acc[1][4];
        if (hh == 0) {
#pragma unroll
            for (int cj = 0; cj < 4; ++cj) acc[0][cj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            mma_block_x3<128, 1, 4, false>(acc, role ? Qh : Kh, role ? Ql : Kl, kLD, 16 * rt, Kh, Kl, kLD, 0, lane);
        }
        float* raw = role ? QKr : KKr;
        float gi[4], bi[4], gj[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            gi[ii] = G[16 * rt + 4 * kb + ii] * kLog2e;
            bi[ii] = Bt[16 * rt + 4 * kb + ii];
            gj[ii] = G[16 * ii + n] * kLog2e;
        }
#pragma unroll
        for (int cj = 0; cj < 4; ++cj) {
            const int j = 16 * cj + n;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 16 * rt + 4 * kb + ii;
                float g;
                if (hh == 0) {
                    g = acc[0][cj][ii];
                    if (j <= i) raw[tri(i, j)] = g;
                } else {
                    g = j <= i ? raw[tri(i, j)] : 0.0f;
                }
                // e^{G_i - G_j}; for j > i the product is discarded by the select
                const float v = __builtin_amdgcn_exp2f(gi[ii] - gj[cj]) * g;
                if (role == 0) {
                    Am[i * 65 + j] = j < i ? bi[ii] * v : 0.0f;
                } else {
                    uint16_t hq, lq;
                    split_bf16(j <= i ? v : 0.0f, hq, lq);
                    Th[i * kLT + j] = hq;
                    Tl[i * kLT + j] = lq;
                }
            }
        }
    }
    __syncthreads();
    // ---- P out, one coalesced 1 KB block per wave and array; the pieces stay in
    // registers until the T region is free again --------------------------------
    u32x4_t pkeep[2];
    {
        int row, k8;
        unswz<kC>(t, row, k8);
        pkeep[0] = *reinterpret_cast<const u32x4_t*>(Th + row * kLT + 8 * k8);
        pkeep[1] = *reinterpret_cast<const u32x4_t*>(Tl + row * kLT + 8 * k8);
        // P and Qe are read only by the output pass, after the state pass:
        // streamed past the caches so that W, K~ and U~, which the state pass
        // reads next, stay in the last-level cache
        __builtin_nontemporal_store(pkeep[0], reinterpret_cast<u32x4_t*>(out.ph + ch * kC * kC + 8 * t));
        __builtin_nontemporal_store(pkeep[1], reinterpret_cast<u32x4_t*>(out.pl + ch * kC * kC + 8 * t));
    }
    // T = (I + A)^-1 (lower unitriangular) in 16x16 blocks, fp32:
    //   diagonal blocks by forward substitution, waves 0-3 one each;
    //   T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj for i > j, wave j walking
    //   column block j downwards (fp32 MFMA 16x16x4).
    float* Tm = reinterpret_cast<float*>(smem + kOffQ);   // [64][65] (Q is consumed)
    float* scr = reinterpret_cast<float*>(smem + kOffQ + kTile128) + rt * (16 * 17);
    if (role == 0) {
        const int bi = wave;
        if (lane < 16) {
            float tc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < i; ++j) ac[j & 3] = fmaf(Am[(16 * bi + i) * 65 + 16 * bi + j], tc[j], ac[j & 3]);
                tc[i] = (i == lane ? 1.0f : 0.0f) - ((ac[0] + ac[1]) + (ac[2] + ac[3]));
                Tm[(16 * bi + i) * 65 + 16 * bi + lane] = tc[i];
            }
        }
    } else {
        // blocks right of the diagonal are zero
        const int bi = rt;
        for (int idx = lane; idx < 16 * (48 - 16 * bi); idx += 64) {
            const int i = idx / (48 - 16 * bi), j = 16 * (bi + 1) + idx % (48 - 16 * bi);
            Tm[(16 * bi + i) * 65 + j] = 0.0f;
        }
    }
    __syncthreads();
    if (wave < 3) {
        const int bj = wave;
        for (int bi = bj + 1; bi < 4; ++bi) {
            f32x4_t ac = f32x4_t{0.f, 0.f, 0.f, 0.f};
            for (int bk = bj; bk < bi; ++bk)
                ac = mm16_f32(Am + (16 * bi) * 65 + 16 * bk, 65, Tm + (16 * bk) * 65 + 16 * bj, 65, ac, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) scr[(4 * kb + ii) * 17 + n] = ac[ii];
            __builtin_amdgcn_wave_barrier();
            const f32x4_t res = mm16_f32(Tm + (16 * bi) * 65 + 16 * bi, 65, scr, 17,
                                         f32x4_t{0.f, 0.f, 0.f, 0.f}, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) Tm[(16 * bi + 4 * kb + ii) * 65 + 16 * bj + n] = -res[ii];
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
    if (hh == 1) {
        // the next unit's inputs (the unit index is clamped, so the loads stay
        // in bounds when the queue has run out), early enough to land before
        // it starts and late enough to keep them out of the registers of
        // the rest of the unit
        unn = s_next;
        fetch_unit<IN_DT>(in, un < units ? un : u, T, qkv, a, b, a_log, dt_bias, conv_w, conv_state, wave, lane);
    }
    // ---- T -> bf16 hi/lo ----------------------------------------------------
    for (int idx = t; idx < kC * kC; idx += kLocalThreads) {
        const int i = idx >> 6, j = idx & 63;
        uint16_t hq, lq;
        split_bf16(Tm[i * 65 + j], hq, lq);
        Th[i * kLT + j] = hq;
        Tl[i * kLT + j] = lq;
    }
    __syncthreads();
    // ---- waves 0-3: W = T diag(beta e^G) K -> LDS (Q region); waves 4-7:
    // U~ = T (beta V) -> U~^T out. Row tile rt (16 tokens), 8 column tiles of
    // 16 dims in two halves. -------------------------------------------------
    uint16_t* Wh = Qh;
    uint16_t* Wl = Ql;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        f32x4_t w[1][4];
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) w[0][cd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (role == 0)
            mma_block_x3_ascale<kC, 4>(w, Th, Tl, kLT, 16 * rt, Ss + hh * kC, Kh, Kl, kLD, 64 * half, lane);
        else
            mma_block_x3<kC, 1, 4, true>(w, Th, Tl, kLT, 16 * rt, Vh, Vl, kLD, 64 * half, lane);
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) {
            const int d = 64 * half + 16 * cd + n;
            uint16_t h4[4], l4[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) split_bf16(w[0][cd][ii], h4[ii], l4[ii]);
            if (role == 0) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int i = 16 * rt + 4 * kb + ii;
                    Wh[i * kLD + d] = h4[ii];
                    Wl[i * kLD + d] = l4[ii];
                }
            } else {
                const size_t o = (ch * 128 + d) * kC + 16 * rt + 4 * kb;
                *reinterpret_cast<u32x2_t*>(out.uth + o) =
                    u32x2_t{h4[0] | (static_cast<uint32_t>(h4[1]) << 16), h4[2] | (static_cast<uint32_t>(h4[3]) << 16)};
                *reinterpret_cast<u32x2_t*>(out.utl + o) =
                    u32x2_t{l4[0] | (static_cast<uint32_t>(l4[1]) << 16), l4[2] | (static_cast<uint32_t>(l4[3]) << 16)};
            }
        }
    }
    __syncthreads();
    // ---- W out (coalesced); P back into the T region (T is consumed) ------------
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int p = t + kLocalThreads * k;
        int row, k8;
        unswz<128>(p, row, k8);
        const u32x4_t vh = *reinterpret_cast<const u32x4_t*>(Wh + row * kLD + 8 * k8);
        const u32x4_t vl = *reinterpret_cast<const u32x4_t*>(Wl + row * kLD + 8 * k8);
        *reinterpret_cast<u32x4_t*>(out.wh + ch * kC * 128 + 8 * p) = vh;
        *reinterpret_cast<u32x4_t*>(out.wl + ch * kC * 128 + 8 * p) = vl;
    }
    {
        int row, k8;
        unswz<kC>(t, row, k8);
        *reinterpret_cast<u32x4_t*>(Th + row * kLT + 8 * k8) = pkeep[0];
        *reinterpret_cast<u32x4_t*>(Tl + row * kLT + 8 * k8) = pkeep[1];
    }
    __syncthreads();
    // ---- P W -> fp32 [64][132] in the V region (beta V is consumed); wave ->
    // row tile rt, column half `role` -------------------------------------------
    float* PW = reinterpret_cast<float*>(smem + kOffV);
    {
        f32x4_t pw[1][4];
#pragma unroll
        for (int cd = 0; cd < 4; ++cd) pw[0][cd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<kC, 1, 4, true>(pw, Th, Tl, kLT, 16 * rt, Wh, Wl, kLD, 64 * role, lane);
#pragma unroll
        for (int cd = 0; cd < 4; ++cd)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                PW[(16 * rt + 4 * kb + ii) * 132 + 64 * role + 16 * cd + n] = pw[0][cd][ii];
    }
    __syncthreads();
    // ---- Qe = e^G q - P W, in place (each thread its own channel pairs) --------
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float eg = __builtin_amdgcn_exp2f(G[8 * wave + i] * kLog2e);
        float2* pp = reinterpret_cast<float2*>(PW + (8 * wave + i) * 132 + 2 * lane);
        const float2 pw = *pp;
        *pp = make_float2(qn[i][0] * eg - pw.x, qn[i][1] * eg - pw.y);
    }
    __syncthreads();
    // ---- Qe out (coalesced) -----------------------------------------------------
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int p = t + kLocalThreads * k;
        int row, k8;
        unswz<128>(p, row, k8);
        const float4 v0 = *reinterpret_cast<const float4*>(PW + row * 132 + 8 * k8);
        const float4 v1 = *reinterpret_cast<const float4*>(PW + row * 132 + 8 * k8 + 4);
        const float y[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const size_t o = ch * kC * 128 + 8 * p;
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) split_bf16x2(y[2 * k2], y[2 * k2 + 1], hw[k2], lw[k2]);
        __builtin_nontemporal_store(u32x4_t{hw[0], hw[1], hw[2], hw[3]}, reinterpret_cast<u32x4_t*>(out.qeh + o));
        __builtin_nontemporal_store(u32x4_t{lw[0], lw[1], lw[2], lw[3]}, reinterpret_cast<u32x4_t*>(out.qel + o));
    }
    __syncthreads();
    }   // value heads
    if (t == 0) s_next = 2 * grid + static_cast<int>(grabbed);
    __syncthreads();
    u = un;
    un = unn;
    }
    // the last workgroup out resets the queue for the next launch (every
    // workgroup has finished taking units by then)
    if (threadIdx.x == 0 && atomicAdd(sched + 1, 1u) == static_cast<unsigned>(grid - 1)) {
        atomicExch(sched, 0u);
        atomicExch(sched + 1, 0u);
    }
}

// ---- sequential state pass ---------------------------------------------------

// One workgroup per (16-row block of the state, value head), 768 threads; a
// 1-D grid of 256 workgroups. Workgroups are dispatched to the 8 XCDs
// round-robin by linear id, so the id -> (head, row block) map puts all row
// blocks of a head on one XCD, whose L2 then serves the chunk inputs they
// share. Twelve waves with fixed roles:
//   waves 0-3 (U waves): token tile tt = wave: U = U~ - W S^T
//       (A = W from global memory, B = S rows from LDS);
//   waves 4-7 (S waves): state columns 32(w-4) .. +31 held as S^T tiles:
//       S^T = e^{G_C} S^T + K~^T U (A = K~^T from global memory, B = U from
//       LDS); they publish S_c to LDS;
//   waves 8-11 (O waves): token tile tt = wave - 8: the block's pre-norm
//       output rows O^T = S_c Qe^T + U~^T P^T (Qe, P from global memory).
// Per chunk c:
//   [S waves publish S_c, U waves publish U~ rows]
//   A  U waves form U;  O waves copy S_c and U~ rows (their A operands) to
//      registers;  S waves request K~ of chunk c+2
//   B  S waves update the state;  O waves form and store O^T, then request
//      Qe, P of chunk c+1;  U waves request W, U~ of chunk c+2
// so the chain (U, then the state update) never waits on a global load it
// issues itself: issuing loads stalls a wave for as long as the CU's load
// path is busy. With U and S^T as the chain's product outputs every LDS
// store is one 8-byte access per lane. The roles run separate loops (same
// barriers), so each loop's loads and waits are straight-line code.
constexpr int kStateThreads = 768;
constexpr int kSA = 136;   // S hi / lo row stride: 128 + 8

__global__ __launch_bounds__(kStateThreads) void dn_chunk_state_kernel(int T, qff_dn_bufs in,
                                                                      float* __restrict__ ssm_state,
                                                                      float* __restrict__ po) {
    const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
    const int h = xcd * 4 + (slot >> 3), rb = slot & 7;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;

    __shared__ __attribute__((aligned(16))) uint16_t Sh[16 * kSA], Sl[16 * kSA];   // S_c [16 rows][128]
    __shared__ __attribute__((aligned(16))) uint16_t Uh[16 * kLT], Ul[16 * kLT];   // U^T [16 rows][64 tokens]
    __shared__ __attribute__((aligned(16))) uint16_t Vh[16 * kLT], Vl[16 * kLT];   // U~^T rows [16][64]

    const int nch = (T + kC - 1) / kC;
    if (wave >= 8) {
        // ---- O waves ------------------------------------------------------
        const int tt = wave - 8;
        struct Stage {
            u32x4_t qe[8];   // Qe token tile tt: [k step][hi, lo]
            u32x4_t p[4];    // P token tile tt: [k step][hi, lo]
        };
        auto fetch = [&](Stage& S, int c) {
            const size_t ch = static_cast<size_t>(c) * 32 + h;
            const size_t ow = ch * kC * 128 + 8 * (tt * 4 * 64 + lane);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                S.qe[2 * ks] = *reinterpret_cast<const u32x4_t*>(in.qeh + ow + 512 * ks);
                S.qe[2 * ks + 1] = *reinterpret_cast<const u32x4_t*>(in.qel + ow + 512 * ks);
            }
            const size_t op = ch * kC * kC + 8 * (tt * 2 * 64 + lane);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                S.p[2 * ks] = *reinterpret_cast<const u32x4_t*>(in.ph + op + 512 * ks);
                S.p[2 * ks + 1] = *reinterpret_cast<const u32x4_t*>(in.pl + op + 512 * ks);
            }
        };
        Stage st;
        fetch(st, 0);
        for (int c = 0; c < nch; ++c) {
            __syncthreads();   // A(c)
            u32x4_t sa_h[4], sa_l[4], ua_h[2], ua_l[2];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                sa_h[ks] = *reinterpret_cast<const u32x4_t*>(Sh + n * kSA + 32 * ks + 8 * kb);
                sa_l[ks] = *reinterpret_cast<const u32x4_t*>(Sl + n * kSA + 32 * ks + 8 * kb);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                ua_h[ks] = *reinterpret_cast<const u32x4_t*>(Vh + n * kLT + 32 * ks + 8 * kb);
                ua_l[ks] = *reinterpret_cast<const u32x4_t*>(Vl + n * kLT + 32 * ks + 8 * kb);
            }
            __syncthreads();   // B(c): (the barrier waits for these LDS reads)
            f32x4_t a0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                a0 = mfma_16x16x32_bf16(sa_l[ks], st.qe[2 * ks], a0);
                a1 = mfma_16x16x32_bf16(sa_h[ks], st.qe[2 * ks + 1], a1);
                a2 = mfma_16x16x32_bf16(sa_h[ks], st.qe[2 * ks], a2);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                a0 = mfma_16x16x32_bf16(ua_l[ks], st.p[2 * ks], a0);
                a1 = mfma_16x16x32_bf16(ua_h[ks], st.p[2 * ks + 1], a1);
                a2 = mfma_16x16x32_bf16(ua_h[ks], st.p[2 * ks], a2);
            }
            fetch(st, min(c + 1, nch - 1));
            // O^T[row 4kb + ii][token 16 tt + n] -> pre-norm output (token-major)
            *reinterpret_cast<f32x4_t*>(po + static_cast<size_t>(c * kC + 16 * tt + n) * 4096 + h * 128 + 16 * rb +
                                        4 * kb) = a0 + a1 + a2;
        }
    } else if (wave < 4) {
        // ---- U waves ------------------------------------------------------
        const int tt = wave;
        struct Stage {
            u32x4_t w[8];   // W token tile tt: [k step][hi, lo]
            u32x4_t ur;     // this thread's 16 B of the block's U~^T rows
        };
        auto fetch = [&](Stage& S, int c) {
            const size_t ch = static_cast<size_t>(c) * 32 + h;
            const size_t ow = ch * kC * 128 + 8 * (tt * 4 * 64 + lane);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                S.w[2 * ks] = *reinterpret_cast<const u32x4_t*>(in.wh + ow + 512 * ks);
                S.w[2 * ks + 1] = *reinterpret_cast<const u32x4_t*>(in.wl + ow + 512 * ks);
            }
            const int arr = t >> 7, rem = t & 127;
            S.ur = *reinterpret_cast<const u32x4_t*>((arr ? in.utl : in.uth) +
                                                     (ch * 128 + 16 * rb + (rem >> 3)) * kC + 8 * (rem & 7));
        };
        auto step = [&](Stage& S, int cn) {
            {
                const int arr = t >> 7, rem = t & 127;
                *reinterpret_cast<u32x4_t*>((arr ? Vl : Vh) + (rem >> 3) * kLT + 8 * (rem & 7)) = S.ur;
            }
            __syncthreads();   // A: S_c and U~^T rows in LDS
            // acc[tok][row] = sum_k W[tok][k] S[row][k] (three accumulators:
            // lo*hi, hi*lo, hi*hi)
            f32x4_t a0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const u32x4_t b_h = *reinterpret_cast<const u32x4_t*>(Sh + n * kSA + 32 * ks + 8 * kb);
                const u32x4_t b_l = *reinterpret_cast<const u32x4_t*>(Sl + n * kSA + 32 * ks + 8 * kb);
                a0 = mfma_16x16x32_bf16(S.w[2 * ks + 1], b_h, a0);
                a1 = mfma_16x16x32_bf16(S.w[2 * ks], b_l, a1);
                a2 = mfma_16x16x32_bf16(S.w[2 * ks], b_h, a2);
            }
            const f32x4_t acc = a0 + a1 + a2;
            // U[tok][row] = U~[tok][row] - acc for row n, tokens 16 tt + 4 kb + ii:
            // four consecutive tokens of row n in the [row][token] tiles
            const int o = n * kLT + 16 * tt + 4 * kb;
            const u32x2_t vh = *reinterpret_cast<const u32x2_t*>(Vh + o);
            const u32x2_t vl = *reinterpret_cast<const u32x2_t*>(Vl + o);
            float u[4];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                u[2 * e] = __uint_as_float(vh[e] << 16) + __uint_as_float(vl[e] << 16) - acc[2 * e];
                u[2 * e + 1] = __uint_as_float(vh[e] & 0xffff0000u) + __uint_as_float(vl[e] & 0xffff0000u) -
                               acc[2 * e + 1];
            }
            uint32_t h0, l0, h1, l1;
            split_bf16x2(u[0], u[1], h0, l0);
            split_bf16x2(u[2], u[3], h1, l1);
            *reinterpret_cast<u32x2_t*>(Uh + o) = u32x2_t{h0, h1};
            *reinterpret_cast<u32x2_t*>(Ul + o) = u32x2_t{l0, l1};
            __syncthreads();   // B: U in LDS
            fetch(S, cn);
        };
        Stage s0, s1;
        fetch(s0, 0);
        fetch(s1, min(1, nch - 1));
        int c = 0;
        for (; c + 1 < nch; c += 2) {
            step(s0, min(c + 2, nch - 1));
            step(s1, min(c + 3, nch - 1));
        }
        if (c < nch) step(s0, c);
    } else {
        // ---- S waves ------------------------------------------------------
        // sacc[ct][ii] = S[row n][col 32 sw + 16 ct + 4 kb + ii]: the C tile of
        // S^T for state columns 32 sw + 16 ct .. +15
        const int sw = wave - 4;
        float* Sg = ssm_state + (static_cast<size_t>(h) * 128 + 16 * rb + n) * 128 + 32 * sw + 4 * kb;
        f32x4_t sacc[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) sacc[ct] = *reinterpret_cast<const f32x4_t*>(Sg + 16 * ct);
        struct Stage {
            u32x4_t k[2][4];   // K~^T column tiles 2 sw + ct: [k step][hi, lo]
            float gam;
        };
        auto fetch = [&](Stage& S, int c) {
            const size_t ch = static_cast<size_t>(c) * 32 + h;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const size_t ok = ch * 128 * kC + 8 * ((2 * sw + ct) * 2 * 64 + lane);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    S.k[ct][2 * ks] = *reinterpret_cast<const u32x4_t*>(in.kth + ok + 512 * ks);
                    S.k[ct][2 * ks + 1] = *reinterpret_cast<const u32x4_t*>(in.ktl + ok + 512 * ks);
                }
            }
            S.gam = in.gam[ch];
        };
        // step computes from stage S and refills stage F (last used in the
        // previous step) with chunk cn = c + 2
        auto step = [&](Stage& S, Stage& F, int cn) {
            // publish S_c: row n, four consecutive columns per tile
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                uint32_t h0, l0, h1, l1;
                split_bf16x2(sacc[ct][0], sacc[ct][1], h0, l0);
                split_bf16x2(sacc[ct][2], sacc[ct][3], h1, l1);
                const int o = n * kSA + 32 * sw + 16 * ct + 4 * kb;
                *reinterpret_cast<u32x2_t*>(Sh + o) = u32x2_t{h0, h1};
                *reinterpret_cast<u32x2_t*>(Sl + o) = u32x2_t{l0, l1};
            }
            __syncthreads();   // A
            fetch(F, cn);
            const float g = S.gam;
            __syncthreads();   // B
            // S^T = e^{G_C} S^T + K~^T U (k = token, 2 steps)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const u32x4_t b_h = *reinterpret_cast<const u32x4_t*>(Uh + n * kLT + 32 * ks + 8 * kb);
                const u32x4_t b_l = *reinterpret_cast<const u32x4_t*>(Ul + n * kLT + 32 * ks + 8 * kb);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    if (ks == 0) sacc[ct] *= g;
                    f32x4_t s1 = mfma_16x16x32_bf16(S.k[ct][2 * ks + 1], b_h, f32x4_t{0.f, 0.f, 0.f, 0.f});
                    s1 = mfma_16x16x32_bf16(S.k[ct][2 * ks], b_l, s1);
                    sacc[ct] = mfma_16x16x32_bf16(S.k[ct][2 * ks], b_h, sacc[ct]);
                    sacc[ct] += s1;
                }
            }
        };
        Stage s0, s1, s2;
        fetch(s0, 0);
        fetch(s1, min(1, nch - 1));
        int c = 0;
        for (; c + 2 < nch; c += 3) {
            step(s0, s2, min(c + 2, nch - 1));
            step(s1, s0, min(c + 3, nch - 1));
            step(s2, s1, min(c + 4, nch - 1));
        }
        if (c < nch) step(s0, s2, min(c + 2, nch - 1));
        if (c + 1 < nch) step(s1, s0, c + 1);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) *reinterpret_cast<f32x4_t*>(Sg + 16 * ct) = sacc[ct];
    }
}

hipError_t launch_deltanet_chunked(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, qff_dtype in_dtype, const float* a, const float* b,
                                   const float* conv_state, float* ssm_state, int T) {
    const int nch = (T + kC - 1) / kC;
    {
        ProfScope prof(ctx, stream, "dn_chunk_local");
        const int units = nch * 16;   // (chunk, key head)
        const int grid = std::min(units, std::max(ctx->num_cu, 1));
        unsigned* sched = ctx->sched + 2 * kSchedChunkLocal;
        if (in_dtype == QFF_BF16)
            dn_chunk_local_kernel<1><<<grid, kLocalThreads, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias,
                                                                         p->conv_w, conv_state, ctx->dn, sched);
        else
            dn_chunk_local_kernel<0><<<grid, kLocalThreads, 0, stream>>>(T, qkv, a, b, p->a_log, p->dt_bias,
                                                                         p->conv_w, conv_state, ctx->dn, sched);
    }
    ProfScope prof(ctx, stream, "dn_chunk_state");
    dn_chunk_state_kernel<<<256, kStateThreads, 0, stream>>>(T, ctx->dn, ssm_state, ctx->pf_o);
    return hipGetLastError();
}

}  // namespace qff
