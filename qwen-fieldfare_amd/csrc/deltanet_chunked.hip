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
//   U = T (beta V - diag(beta e^G) K S0^T)
//   P_ij = e^{G_i - G_j} (q_i . k_j)  (j <= i)
//   O = diag(e^G) Q S0^T + P U
//   S_C = e^{G_C} S0 + U^T diag(e^{G_C - G}) K
// (tests/test_oracle_deltanet.py checks the chunked form against the
// sequential recurrence in fp64). Everything that depends on S0 is formed
// from the key head's K and Q, which both of its value heads share; the
// per-head data are T, P and the gates.
//
// Two kernels:
//   dn_chunk_local_kernel  persistent, one (chunk, key head) unit at a time
//       from a work queue, all chunks independent: conv1d + SiLU of the
//       chunk's q and k channels straight from the projection (3 tokens of
//       history from the input or the conv state), L2 norms, both value
//       heads' gates, the Gram products K K^T and K Q^T, then per value head
//       A, P and T = (I + A)^-1 (16x16 blocks: diagonal blocks by
//       substitution, the rest on fp32 MFMAs), and the conv1d + SiLU of both
//       heads' v channels times beta. Writes K (bf16 hi/lo, in the state
//       pass's LDS image), Q, T and P (bf16 hi/lo) as MFMA operand blocks,
//       beta V and the per-token gate factors.
//   dn_chunk_state_kernel  one workgroup per (16 state rows, value head)
//       walks the chunks in order: four chain waves hold the block's state
//       (key quarters) in accumulators and form X = K S^T, U = T (beta V -
//       D X) and the state update, a token tile or key quarter each; four
//       helper waves stage the next chunk's operands in LDS and form the
//       pre-norm output rows O = diag(e^G) Q S^T + P U one chunk behind.
//
// Operand order. A 16x16x32 MFMA gives lane l of its A and B operands the
// 8 k-elements e = 0..7 of lane group g = l / 16; here they are the k indices
//   pq(g, e) = 4g + e (e < 4),  16 + 4g + (e - 4) (e >= 4)
// of each 32-wide k step, which is where two stacked 16x16 fp32 accumulator
// tiles (rows 0-15, 16-31) keep them (lane l: column l % 16, rows 4g .. 4g+3
// of each tile). So a product's accumulators become the next product's B
// operand (k = the accumulator rows) in registers, with no exchange, when
// the A operand walks k in the same order; every operand block below is
// written in it.
//
// Precision: every product runs as bf16x3 on v_mfma_f32_16x16x32_bf16
// (a b ~ a_hi b_hi + a_hi b_lo + a_lo b_hi, ~2^-16 relative per product):
// the chain's (X, U and the state update), which keeps the fp32 state within
// 1e-4 of the sequential fp32 recurrence, the Gram products, and the output
// products Q S^T and P U, whose fp32 result is the pre-norm output. Their
// error is relative to the operands whatever their scale (bf16 has fp32's
// exponent range), so tiny and huge value heads keep their precision
// through the gated RMSNorm.
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kC = 64;      // chunk length
constexpr int kLD = 136;    // bf16 row stride of [64][128] LDS tiles (128 + 8)
constexpr int kBlk = 512;   // 16-bit elements of one operand block (64 lanes x 8)

constexpr float kLog2e = 1.44269504088896341f;

// Workspace records (16-bit elements unless noted), per chunk c:
constexpr int kKImg = 2 * kC * 128;   // per key head: K hi, lo, each [64][128] in the LDS image order
constexpr int kQOp = 2 * 16 * kBlk;   // per key head: Q hi, lo, blocks (token tile tt, k step j), tt * 4 + j
constexpr int kTOp = 2 * 6 * kBlk;    // per value head: T hi, lo, blocks tblk(tt, j)
constexpr int kPOp = 2 * 6 * kBlk;    // per value head: P hi, lo, blocks tblk(tt, j)
constexpr int kGates = 4 * kC;        // per value head (floats): beta, beta e^G, e^{G_C - G}, e^G
constexpr int kBV = kC * 128;         // per value head (floats): beta V, [16-channel block][token tile][lane][4]

// k index of element e of lane group g in a 32-wide k step (see above)
__device__ __forceinline__ int pq(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

// The lower-triangular [64][64] operands (T, P) as 16-row tiles tt x 32-wide
// k steps j <= tt / 2: blocks (0,0) (1,0) (2,0) (2,1) (3,0) (3,1).
__device__ __forceinline__ int tblk(int tt, int j) { return tt < 2 ? tt : 2 * tt - 2 + j; }

// K image: row r (token), logical 16-byte piece q holds keys 32(q/4) +
// 4(q%4) .. +3 and 32(q/4) + 16 + 4(q%4) .. +3 (one lane group's operand
// piece); it sits at physical piece q ^ (r % 16), so the 16 rows of an
// operand read (and the 16 rows of a transposed read) fall on different
// LDS banks. Element offset of logical piece q of row r:
__device__ __forceinline__ int kimg_off(int r, int q) { return r * 128 + ((q ^ (r & 15)) << 3); }

// ---- chunk-local pass --------------------------------------------------------

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
// of the key head's q and k blocks and of its two value heads' v blocks):
// the conv input rows at positions
// tok-3 .. tok+7 clamped into [0, T), the conv weights, and per value head
// the gate inputs of token lane and the head's A_log and dt_bias. Every load
// is unconditional and in bounds, so the loads of the next unit can be
// issued while the current one is processed. (The conv-state slots that
// chunk 0 needs are read when that unit is processed.)
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
                                           const float* __restrict__ conv_w, int wave, int lane) {
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

// LDS carve-up of the chunk-local kernel (bytes). T (fp32) reuses the Q
// region once Q has been written out.
constexpr int kTile128 = kC * kLD * 2;            // one [64][136] bf16 array
constexpr int kOffK = 0;                          // K hi, lo
constexpr int kOffQ = 2 * kTile128;               // Q hi, lo; then T fp32 [2][64][65]
constexpr int kOffA = 4 * kTile128;               // A fp32 [2][64][65]
constexpr int kOffS = kOffA + 2 * kC * 65 * 4;    // off-diagonal solve scratch [6][16][17] fp32
constexpr int kOffG = kOffS + 6 * 16 * 17 * 4;    // G [2][64], beta [2][64]
constexpr int kLocalSmem = kOffG + 4 * kC * 4;
static_assert(2 * kC * 65 * 4 <= 2 * kTile128, "T must fit the Q region");

// Persistent: grid = min(units, CUs) workgroups of 512 threads (eight
// waves, two per SIMD) walk the (chunk, key head) units. Units 0 .. 2g-1
// go out statically (g = grid size), the rest through an atomic counter, so
// a workgroup on a CU that runs slow simply takes fewer units; the launch's
// last workgroup resets the counter. Per unit:
//   gates of both value heads (waves 0, 1; lane = token) -> LDS and out;
//   conv + SiLU + L2 norm of q and k (wave = 8 tokens, lane = 2 channels)
//       -> LDS as bf16 hi / lo;
//   K K^T (waves 0-3), one 16-row tile each, then A of both heads into LDS;
//       K Q^T (waves 4-7), one query tile each over every key tile, whose
//       accumulators are P's operand blocks: P of both heads (decay and
//       mask applied) straight from registers to global; the next unit's
//       inputs are requested here;
//   K image and Q blocks out;
//   T = (I + A)^-1 of both heads: the eight diagonal blocks by forward
//       substitution (one wave each), the off-diagonal blocks by six waves
//       walking their column block down on fp32 MFMAs;
//   T blocks out.
// Global loads are issued before the stores of the same unit (vmcnt counts
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
    float* Tm = reinterpret_cast<float*>(smem + kOffQ);   // [2][64][65]
    float* Am = reinterpret_cast<float*>(smem + kOffA);   // [2][64][65]
    float* Scr = reinterpret_cast<float*>(smem + kOffS);
    float* Gs = reinterpret_cast<float*>(smem + kOffG);   // [hh][64]
    float* Bs = Gs + 2 * kC;                              // [hh][64]

    int u = blockIdx.x, un = blockIdx.x + grid;
    UnitIn<IN_DT> in;
    fetch_unit<IN_DT>(in, u, T, qkv, a, b, a_log, dt_bias, conv_w, threadIdx.x >> 6, threadIdx.x & 63);
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
    const int rt = wave & 3, role = wave >> 2;   // MFMA row tile; K K^T or Q K^T
    int c, kh;
    unit_coords(u, c, kh);
    const int t0 = c * kC;
    const int nv = min(kC, T - t0);
    const int tw = t0 + 8 * wave;                  // this wave's first token

    // gates (deltanet.metal:250-280), waves 0 and 1 one value head each:
    // log g = -e^{A_log} softplus(a + dt_bias), beta = sigmoid(b); G =
    // inclusive prefix sum over the chunk. Padded tokens have log g = 0 and
    // beta = 0, so they change nothing (and G_63 = G_C).
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
        const float gc = __shfl(x, 63, 64);
        const float eg = __builtin_amdgcn_exp2f(x * kLog2e);
        Gs[hh * kC + lane] = x;
        Bs[hh * kC + lane] = beta;
        float* go = out.gates + (static_cast<size_t>(c) * 32 + 2 * kh + hh) * kGates;
        go[lane] = beta;
        go[kC + lane] = beta * eg;
        go[2 * kC + lane] = __builtin_amdgcn_exp2f((gc - x) * kLog2e);
        go[3 * kC + lane] = eg;
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
            uint32_t hh, ll;
            split_bf16x2(y[i][0] * sc, y[i][1] * sc, hh, ll);
            const int o = (8 * wave + i) * kLD + 2 * lane;
            *reinterpret_cast<uint32_t*>(dh + o) = hh;
            *reinterpret_cast<uint32_t*>(dl + o) = ll;
        }
    };
    {
        float y[8][2];
        conv(0, y);
        norm_store(y, 0.08838834764831845f, Qh, Ql);   // 1 / sqrt(128)
        conv(1, y);
        norm_store(y, 1.0f, Kh, Kl);
    }
    __syncthreads();
    // ---- beta V of both value heads (conv + SiLU of the v channels times the
    // token's beta), stored in the state pass's order: per 16-channel block
    // cb and token tile tt, lane n + 16g holds tokens 16tt + 4g .. +3 of
    // channel 16cb + n
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        float y[8][2];
        conv(2 + hh, y);
        float* bo = out.bv + (static_cast<size_t>(c) * 32 + 2 * kh + hh) * kBV;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int ch = 2 * lane + cc;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int tok = 8 * wave + 4 * hf;
                const float4 bt = *reinterpret_cast<const float4*>(Bs + hh * kC + tok);
                const int o = (((ch >> 4) * 4 + (tok >> 4)) * 64 + (ch & 15) + 16 * ((tok & 15) >> 2)) * 4;
                *reinterpret_cast<f32x4_t*>(bo + o) =
                    f32x4_t{bt.x * y[4 * hf][cc], bt.y * y[4 * hf + 1][cc], bt.z * y[4 * hf + 2][cc],
                            bt.w * y[4 * hf + 3][cc]};
            }
        }
    }
    // grabbed now, published at the end of the unit, when it has long arrived
    unsigned grabbed = 0;
    if (t == 0) grabbed = atomicAdd(sched, 1u);
    int unn;

    // ---- waves 0-3: K K^T -> A of both heads (strictly lower, scaled), row
    // tile rt; waves 4-7: K Q^T for query tile rt over every key tile, whose
    // accumulators are already P's MFMA A operands (lane (n, g) of key tile
    // kt holds P[16 rt + n][16 kt + 4g + i]: elements 4(kt & 1) + i of the
    // block (query tile rt, k step kt / 2)), so the P blocks of both heads
    // (lower incl. diagonal, decay applied) go out from registers
    if (role == 0) {
        f32x4_t acc[1][4];
#pragma unroll
        for (int cj = 0; cj < 4; ++cj) acc[0][cj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<128, 1, 4, false>(acc, Kh, Kl, kLD, 16 * rt, Kh, Kl, kLD, 0, lane);
        // the next unit's inputs (the unit index is clamped, so the loads
        // stay in bounds when the queue has run out)
        unn = s_next;
        fetch_unit<IN_DT>(in, un < units ? un : u, T, qkv, a, b, a_log, dt_bias, conv_w, wave, lane);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const float* G = Gs + hh * kC;
            const float* Bt = Bs + hh * kC;
            float gi[4], bi[4], gj[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                gi[ii] = G[16 * rt + 4 * kb + ii] * kLog2e;
                bi[ii] = Bt[16 * rt + 4 * kb + ii];
                gj[ii] = G[16 * ii + n] * kLog2e;
            }
#pragma unroll
            for (int cj = 0; cj < 4; ++cj) {
                // A is read only on and below its diagonal blocks
                if (cj > rt) continue;
                const int j = 16 * cj + n;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int i = 16 * rt + 4 * kb + ii;
                    // e^{G_i - G_j}; for j > i the product is discarded by the select
                    const float v = __builtin_amdgcn_exp2f(gi[ii] - gj[cj]) * acc[0][cj][ii];
                    Am[hh * kC * 65 + i * 65 + j] = j < i ? bi[ii] * v : 0.0f;
                }
            }
        }
    } else {
        f32x4_t acc[4][1];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) acc[kt][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        mma_block_x3<128, 4, 1, false>(acc, Kh, Kl, kLD, 0, Qh, Ql, kLD, 16 * rt, lane);
        unn = s_next;
        fetch_unit<IN_DT>(in, un < units ? un : u, T, qkv, a, b, a_log, dt_bias, conv_w, wave, lane);
        const int i = 16 * rt + n;   // this lane's query token
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const float* G = Gs + hh * kC;
            const float gi = G[i] * kLog2e;
            uint16_t* po = out.pop + (static_cast<size_t>(c) * 32 + 2 * kh + hh) * kPOp + 8 * lane;
#pragma unroll
            for (int sj = 0; sj < 2; ++sj) {
                if (sj > (rt >> 1)) continue;   // blocks tblk(rt, sj), sj <= rt / 2
                float pv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int kt = 2 * sj + (e >> 2), r = e & 3;
                    const int j = 16 * kt + 4 * kb + r;
                    const float v = __builtin_amdgcn_exp2f(gi - G[j] * kLog2e) * acc[kt][0][r];
                    pv[e] = j <= i ? v : 0.0f;
                }
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) split_bf16x2(pv[2 * q], pv[2 * q + 1], hw[q], lw[q]);
                uint16_t* pb = po + tblk(rt, sj) * kBlk;
                *reinterpret_cast<u32x4_t*>(pb) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
                *reinterpret_cast<u32x4_t*>(pb + 6 * kBlk) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
            }
        }
    }
    __syncthreads();
    // ---- K image and Q blocks (bf16 hi, lo) out ----------------------------------
    {
        uint16_t* ko = out.kimg + (static_cast<size_t>(c) * 16 + kh) * kKImg;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int pc = t + kLocalThreads * i;   // [hi, lo][row][physical piece]
            const int hl = pc >> 10, row = (pc >> 4) & 63, p = pc & 15;
            const int q = p ^ (row & 15);
            const int k0 = 32 * (q >> 2) + 4 * (q & 3);
            const uint16_t* src = (hl ? Kl : Kh) + row * kLD;
            const u32x2_t x0 = *reinterpret_cast<const u32x2_t*>(src + k0);
            const u32x2_t x1 = *reinterpret_cast<const u32x2_t*>(src + k0 + 16);
            *reinterpret_cast<u32x4_t*>(ko + 8 * pc) = u32x4_t{x0[0], x0[1], x1[0], x1[1]};
        }
        uint16_t* qo = out.qop + (static_cast<size_t>(c) * 16 + kh) * kQOp;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int pc = t + kLocalThreads * i;   // [block tt * 4 + j][lane]
            const int blk = pc >> 6, l = pc & 63;
            const int row = 16 * (blk >> 2) + (l & 15), k0 = 32 * (blk & 3) + 4 * (l >> 4);
            const u32x2_t h0 = *reinterpret_cast<const u32x2_t*>(Qh + row * kLD + k0);
            const u32x2_t h1 = *reinterpret_cast<const u32x2_t*>(Qh + row * kLD + k0 + 16);
            const u32x2_t l0 = *reinterpret_cast<const u32x2_t*>(Ql + row * kLD + k0);
            const u32x2_t l1 = *reinterpret_cast<const u32x2_t*>(Ql + row * kLD + k0 + 16);
            *reinterpret_cast<u32x4_t*>(qo + 8 * pc) = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
            *reinterpret_cast<u32x4_t*>(qo + 16 * kBlk + 8 * pc) = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
        }
    }
    __syncthreads();   // Q consumed: its region holds T from here on
    // ---- T = (I + A)^-1 (lower unitriangular) in 16x16 blocks, fp32 ------------
    // diagonal block bi of head hh by forward substitution (lanes 0-15, lane =
    // column), the blocks right of it zeroed by the whole wave
    {
        const int hh = wave >> 2, bi = wave & 3;
        const float* A = Am + hh * kC * 65;
        float* Th = Tm + hh * kC * 65;
        for (int idx = lane; idx < 16 * (48 - 16 * bi); idx += 64) {
            const int i = idx / (48 - 16 * bi), j = 16 * (bi + 1) + idx % (48 - 16 * bi);
            Th[(16 * bi + i) * 65 + j] = 0.0f;
        }
        if (lane < 16) {
            float tc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < i; ++j) ac[j & 3] = fmaf(A[(16 * bi + i) * 65 + 16 * bi + j], tc[j], ac[j & 3]);
                tc[i] = (i == lane ? 1.0f : 0.0f) - ((ac[0] + ac[1]) + (ac[2] + ac[3]));
                Th[(16 * bi + i) * 65 + 16 * bi + lane] = tc[i];
            }
        }
    }
    __syncthreads();
    // off-diagonal: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, wave (hh, bj)
    // walking column block bj downwards (fp32 MFMA 16x16x4)
    if (wave < 6) {
        const int hh = wave / 3, bj = wave % 3;
        const float* A = Am + hh * kC * 65;
        float* Th = Tm + hh * kC * 65;
        float* scr = Scr + wave * (16 * 17);
        for (int bi = bj + 1; bi < 4; ++bi) {
            f32x4_t ac = f32x4_t{0.f, 0.f, 0.f, 0.f};
            for (int bk = bj; bk < bi; ++bk)
                ac = mm16_f32(A + (16 * bi) * 65 + 16 * bk, 65, Th + (16 * bk) * 65 + 16 * bj, 65, ac, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) scr[(4 * kb + ii) * 17 + n] = ac[ii];
            __builtin_amdgcn_wave_barrier();
            const f32x4_t res = mm16_f32(Th + (16 * bi) * 65 + 16 * bi, 65, scr, 17,
                                         f32x4_t{0.f, 0.f, 0.f, 0.f}, lane);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) Th[(16 * bi + 4 * kb + ii) * 65 + 16 * bj + n] = -res[ii];
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
    // ---- T blocks out (bf16 hi / lo) --------------------------------------------
    for (int pc = t; pc < 2 * 6 * 64; pc += kLocalThreads) {   // [hh][block][lane]
        const int hh = pc / 384, blk = (pc >> 6) % 6, l = pc & 63;
        const int tt = blk < 2 ? blk : 2 + ((blk - 2) >> 1), j = blk < 2 ? 0 : (blk - 2) & 1;
        const int row = 16 * tt + (l & 15), k0 = 32 * j + 4 * (l >> 4);
        const float* src = Tm + hh * kC * 65 + row * 65 + k0;
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int kk = 2 * (e & 1) + 16 * (e >> 1);
            split_bf16x2(src[kk], src[kk + 1], hw[e], lw[e]);
        }
        uint16_t* to = out.top + (static_cast<size_t>(c) * 32 + 2 * kh + hh) * kTOp + 8 * (pc % 384);
        *reinterpret_cast<u32x4_t*>(to) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
        *reinterpret_cast<u32x4_t*>(to + 6 * kBlk) = u32x4_t{lw[0], lw[1], lw[2], lw[3]};
    }
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

// bf16 hi / lo halves of 8 fp32 values (two accumulator tiles, pq order).
__device__ __forceinline__ void split8(const f32x4_t& a, const f32x4_t& b, u32x4_t& hi, u32x4_t& lo) {
    uint32_t h[4], l[4];
    split_bf16x2(a[0], a[1], h[0], l[0]);
    split_bf16x2(a[2], a[3], h[1], l[1]);
    split_bf16x2(b[0], b[1], h[2], l[2]);
    split_bf16x2(b[2], b[3], h[3], l[3]);
    hi = u32x4_t{h[0], h[1], h[2], h[3]};
    lo = u32x4_t{l[0], l[1], l[2], l[3]};
}
__device__ __forceinline__ u32x4_t pack_f16x8(const f32x4_t& a, const f32x4_t& b) {
    return u32x4_t{pack_f16x2(a[0], a[1]), pack_f16x2(a[2], a[3]), pack_f16x2(b[0], b[1]), pack_f16x2(b[2], b[3])};
}
// acc += a b with bf16x3 operands
__device__ __forceinline__ f32x4_t mma_x3(u32x4_t ah, u32x4_t al, u32x4_t bh, u32x4_t bl, f32x4_t acc) {
    acc = mfma_16x16x32_bf16(al, bh, acc);
    acc = mfma_16x16x32_bf16(ah, bl, acc);
    return mfma_16x16x32_bf16(ah, bh, acc);
}

// LDS of the state pass: two stages of chunk operands (filled by the helper
// waves one chunk ahead) and the pieces the chain waves exchange.
struct StateSmem {
    uint16_t kimg[2][kKImg];        // [stage] K hi | lo image
    u32x4_t st[3][4][2][64];        // [chunk % 3][k step][hi, lo][lane] S^T bf16 B operands
    uint32_t yop[2][2][64][4];      // [k step][hi, lo][lane][tile parity x 2] Y bf16 B operands
    uint32_t uop[2][2][64][4];      // [k step][hi, lo][lane][...] e^{G_C - G} U bf16 B operands
    uint32_t uf[2][2][2][64][4];    // [chunk parity][k step][hi, lo][lane][...] U bf16 B operands
    unsigned sync;                  // arrivals of the chain waves at their own barriers
};

// Barrier of the four chain waves only (the helper waves keep running): lane
// 0 counts the wave in once its LDS writes have completed, then the wave
// waits for the count of the barrier's round. Every chain wave arrives at
// every round, so every wait ends.
__device__ __forceinline__ void chain_sync(unsigned* cnt, unsigned target, int lane) {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes done
    if (lane == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
        __builtin_amdgcn_s_sleep(1);
}

// One workgroup of 512 threads per (16-row block cb of the state, value head
// h), a 1-D grid of 256. Workgroups go to the 8 XCDs round-robin by linear
// id; the id -> (head, block) map puts both value heads of two key heads on
// each XCD, so its L2 serves the K image all 16 blocks of a key head share.
// Lane l = (n, g) = (l % 16, l / 16): state row 16 cb + n.
//
// Chain waves 0-3 (w, one per SIMD) split every product of a chunk step four
// ways, so each reads a quarter of its LDS operands (a wave draws ~1 KB per
// 30 cycles from LDS, and one wave reading all of them was the bound). Wave
// w holds S^T for keys 32w .. 32w+31 (key tiles 2w, 2w+1, S^T[16 kt + 4g +
// i][n]) and owns token tile w; the chunk data only it reads (its T blocks,
// beta V, gate factors) come from L2 into registers a chunk ahead, so only
// the K image, which all four read, goes through LDS. Per chunk c:
//   (a) X_w = K[tokens of tile w, :] S^T over all four k steps: A = K image
//       rows from LDS, B = the S^T operands the four waves published at the
//       end of chunk c - 1; Y_w = beta V - D X_w, split bf16 hi / lo and
//       published as its half of Y's k-step operand;
//   [C1: the chain waves only]
//   (b) U_w = T[tile w, :] Y (k steps j <= w / 2); U_w and e^{G_C - G} U_w
//       published as bf16 hi / lo operand halves (for the output and for
//       (c));
//   [C2: the chain waves only]
//   (c) S^T[keys of w] = e^{G_C} S^T + K^T diag(e^{G_C - G}) U: A = K^T through
//       the LDS transpose read of the image, B = the scaled U operands; the
//       new S^T published as bf16 hi / lo operands (slot (c + 1) % 3).
//   [B0 of chunk c + 1: the whole workgroup]
// Helper waves 4-7 (hw, token tile hw) meet the chain only at B0. Between
// B0(c) and B0(c + 1): the output rows of chunk c - 1, O = diag(e^G) Q S^T +
// P U, as bf16x3 products like the chain's (Q, P blocks in registers, loaded
// a chunk earlier; S^T of chunk c - 1 stays published until the end of step
// c + 1, hence three slots), stored as the fp32 pre-norm output that the
// gated RMSNorm pass reads; a quarter of chunk c + 1's K image into the free
// stage from registers loaded a chunk earlier; the loads of chunk c + 2.
constexpr int kStateThreads = 512;

__global__ __launch_bounds__(kStateThreads) void dn_chunk_state_kernel(int T, qff_dn_bufs in,
                                                                      float* __restrict__ ssm_state,
                                                                      float* __restrict__ po) {
    const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
    const int kh = 2 * xcd + (slot >> 4), h = 2 * kh + ((slot >> 3) & 1), cb = slot & 7;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int nch = (T + kC - 1) / kC;

    __shared__ StateSmem sm;
    if (t == 0) sm.sync = 0;   // published by the first B0

    if (wave < 4) {
        // ---- chain waves ----------------------------------------------------
        const int w = wave;
        float* Sg = ssm_state + (static_cast<size_t>(h) * 128 + 16 * cb + n) * 128 + 32 * w + 4 * g;
        f32x4_t sT[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) sT[k2] = *reinterpret_cast<const f32x4_t*>(Sg + 16 * k2);
        auto publish_state = [&](int slot3) {
            u32x4_t bh, bl;
            split8(sT[0], sT[1], bh, bl);
            sm.st[slot3][w][0][lane] = bh;
            sm.st[slot3][w][1][lane] = bl;
        };
        publish_state(0);
        // this wave's own chunk operands, loaded from L2 a chunk ahead: T
        // blocks tblk(w, 0 .. 1) (hi, lo), beta V of token tile w, D and
        // e^{G_C - G} of its tokens and e^{G_C}
        struct ChainIn {
            u32x4_t t[2][2];
            f32x4_t bv, d4, e4;
            float gam;
        };
        const int tb0 = w < 2 ? w : 2 * w - 2, tb1 = w < 2 ? tb0 : tb0 + 1;
        auto load_in = [&](ChainIn& r, int cc) {
            const uint16_t* tg = in.top + (static_cast<size_t>(cc) * 32 + h) * kTOp + 8 * lane;
            r.t[0][0] = *reinterpret_cast<const u32x4_t*>(tg + tb0 * kBlk);
            r.t[0][1] = *reinterpret_cast<const u32x4_t*>(tg + 6 * kBlk + tb0 * kBlk);
            r.t[1][0] = *reinterpret_cast<const u32x4_t*>(tg + tb1 * kBlk);
            r.t[1][1] = *reinterpret_cast<const u32x4_t*>(tg + 6 * kBlk + tb1 * kBlk);
            r.bv = *reinterpret_cast<const f32x4_t*>(in.bv + (static_cast<size_t>(cc) * 32 + h) * kBV +
                                                     (cb * 4 + w) * 256 + 4 * lane);
            const float* gg = in.gates + (static_cast<size_t>(cc) * 32 + h) * kGates;
            r.d4 = *reinterpret_cast<const f32x4_t*>(gg + kC + 16 * w + 4 * g);
            r.e4 = *reinterpret_cast<const f32x4_t*>(gg + 2 * kC + 16 * w + 4 * g);
            r.gam = gg[3 * kC + kC - 1];
        };
        auto step = [&](int c, const ChainIn& ci, ChainIn& next) {
            const int s = c & 1, s3 = c % 3;
            __syncthreads();   // B0(c): stage s holds chunk c; S_c published
            load_in(next, min(c + 1, nch - 1));
            const uint16_t* kh_ = sm.kimg[s];
            const uint16_t* kl_ = sm.kimg[s] + kC * 128;
            // (a) X_w over all keys, then Y_w
            u32x4_t ka[4][2], sb[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int o = kimg_off(16 * w + n, 4 * j + g);
                ka[j][0] = *reinterpret_cast<const u32x4_t*>(kh_ + o);
                ka[j][1] = *reinterpret_cast<const u32x4_t*>(kl_ + o);
                sb[j][0] = sm.st[s3][j][0][lane];
                sb[j][1] = sm.st[s3][j][1][lane];
            }
            f32x4_t xa = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) xa = mma_x3(ka[j][0], ka[j][1], sb[j][0], sb[j][1], xa);
            const f32x4_t y = ci.bv - ci.d4 * xa;
            {
                uint32_t h0, l0, h1, l1;
                split_bf16x2(y[0], y[1], h0, l0);
                split_bf16x2(y[2], y[3], h1, l1);
                uint32_t* yh = sm.yop[w >> 1][0][lane] + 2 * (w & 1);
                uint32_t* yl = sm.yop[w >> 1][1][lane] + 2 * (w & 1);
                *reinterpret_cast<u32x2_t*>(yh) = u32x2_t{h0, h1};
                *reinterpret_cast<u32x2_t*>(yl) = u32x2_t{l0, l1};
            }
            chain_sync(&sm.sync, 8 * c + 4, lane);   // C1(c)
            // (b) U_w = T[tile w, :] Y
            f32x4_t ua = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j <= (w >> 1))
                    ua = mma_x3(ci.t[j][0], ci.t[j][1], *reinterpret_cast<const u32x4_t*>(sm.yop[j][0][lane]),
                                *reinterpret_cast<const u32x4_t*>(sm.yop[j][1][lane]), ua);
            }
            {
                uint32_t h0, l0, h1, l1;
                split_bf16x2(ua[0], ua[1], h0, l0);
                split_bf16x2(ua[2], ua[3], h1, l1);
                *reinterpret_cast<u32x2_t*>(sm.uf[s][w >> 1][0][lane] + 2 * (w & 1)) = u32x2_t{h0, h1};
                *reinterpret_cast<u32x2_t*>(sm.uf[s][w >> 1][1][lane] + 2 * (w & 1)) = u32x2_t{l0, l1};
                const f32x4_t us = ua * ci.e4;
                split_bf16x2(us[0], us[1], h0, l0);
                split_bf16x2(us[2], us[3], h1, l1);
                *reinterpret_cast<u32x2_t*>(sm.uop[w >> 1][0][lane] + 2 * (w & 1)) = u32x2_t{h0, h1};
                *reinterpret_cast<u32x2_t*>(sm.uop[w >> 1][1][lane] + 2 * (w & 1)) = u32x2_t{l0, l1};
            }
            // the transposed K operands of (c), requested before the barrier
            u32x4_t kt_[2][2][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // source lane n of group g points at token 32j + 4g + n/4 (+16),
                // keys 16 kt + 4 (n % 4) .. +3 of key tile kt = 2w + k2
                const int r = 32 * j + 4 * g + (n >> 2);
                const int o = kimg_off(r, 4 * w + (n & 3));
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const int ok = o + 4 * k2;
                    const u32x2_t h0 = lds_read_tr16(kh_ + ok), h1 = lds_read_tr16(kh_ + ok + 16 * 128);
                    const u32x2_t l0 = lds_read_tr16(kl_ + ok), l1 = lds_read_tr16(kl_ + ok + 16 * 128);
                    kt_[j][k2][0] = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
                    kt_[j][k2][1] = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
                }
            }
            const float gam = ci.gam;
            chain_sync(&sm.sync, 8 * c + 8, lane);   // C2(c)
            // (c) S^T[keys of w] = e^{G_C} S^T + K^T (e^{G_C - G} U)
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) sT[k2] *= gam;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const u32x4_t uh = *reinterpret_cast<const u32x4_t*>(sm.uop[j][0][lane]);
                const u32x4_t ul = *reinterpret_cast<const u32x4_t*>(sm.uop[j][1][lane]);
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) sT[k2] = mma_x3(kt_[j][k2][0], kt_[j][k2][1], uh, ul, sT[k2]);
            }
            publish_state((c + 1) % 3);
        };
        ChainIn ia, ib;
        load_in(ia, 0);
        int c = 0;
        for (; c + 1 < nch; c += 2) {
            step(c, ia, ib);
            step(c + 1, ib, ia);
        }
        if (c < nch) step(c, ia, ib);
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) *reinterpret_cast<f32x4_t*>(Sg + 16 * k2) = sT[k2];
        __syncthreads();   // B0(nch): the helpers form the last chunk's output
    } else {
        // ---- helper waves ---------------------------------------------------
        const int hw = wave - 4;   // token tile and operand quarter
        // this wave's quarter of a chunk's K image: blocks 8hw .. +7 of 32
        // (hi then lo); P blocks pb, pb + 1 (token tile hw uses tblk(hw, 0) =
        // pb and, for hw >= 2, tblk(hw, 1) = pb + 1)
        const int pb = hw < 2 ? hw : 2 * hw - 2;
        struct Stage {
            u32x4_t k[8];
        } hs;
        struct Out {
            u32x4_t q[4][2];   // Q blocks (hw, j), hi / lo
            u32x4_t p[2][2];   // P blocks pb, pb + 1, hi / lo
            f32x4_t eg;        // e^G of the tile's tokens
        } ho;
        // every helper load is unconditional (a load under a divergent branch
        // makes the compiler wait for all outstanding loads at the join)
        auto load_stage = [&](int cc) {
            const uint16_t* kg = in.kimg + (static_cast<size_t>(cc) * 16 + kh) * kKImg + hw * (8 * kBlk);
#pragma unroll
            for (int i = 0; i < 8; ++i) hs.k[i] = *reinterpret_cast<const u32x4_t*>(kg + i * kBlk + 8 * lane);
        };
        auto store_stage = [&](int s) {
            uint16_t* kd = sm.kimg[s] + hw * (8 * kBlk);
#pragma unroll
            for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4_t*>(kd + i * kBlk + 8 * lane) = hs.k[i];
        };
        auto load_out = [&](int cc) {
            const uint16_t* qg = in.qop + (static_cast<size_t>(cc) * 16 + kh) * kQOp + 4 * hw * kBlk + 8 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ho.q[i][0] = *reinterpret_cast<const u32x4_t*>(qg + i * kBlk);
                ho.q[i][1] = *reinterpret_cast<const u32x4_t*>(qg + 16 * kBlk + i * kBlk);
            }
            const uint16_t* pg = in.pop + (static_cast<size_t>(cc) * 32 + h) * kPOp + pb * kBlk + 8 * lane;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ho.p[i][0] = *reinterpret_cast<const u32x4_t*>(pg + i * kBlk);
                ho.p[i][1] = *reinterpret_cast<const u32x4_t*>(pg + 6 * kBlk + i * kBlk);
            }
            ho.eg = *reinterpret_cast<const f32x4_t*>(in.gates + (static_cast<size_t>(cc) * 32 + h) * kGates + 3 * kC +
                                                      16 * hw + 4 * g);
        };
        // the output rows of chunk cc: lane (n, g) holds state row 16 cb + n of
        // tokens cc * 64 + 16 hw + 4 g + i
        auto output = [&](int cc) {
            const int par = cc & 1, s3 = cc % 3;
            f32x4_t o = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o = mma_x3(ho.q[j][0], ho.q[j][1], sm.st[s3][j][0][lane], sm.st[s3][j][1][lane], o);
            o *= ho.eg;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j == 0 || hw >= 2)
                    o = mma_x3(ho.p[j][0], ho.p[j][1], *reinterpret_cast<const u32x4_t*>(sm.uf[par][j][0][lane]),
                               *reinterpret_cast<const u32x4_t*>(sm.uf[par][j][1][lane]), o);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = cc * kC + 16 * hw + 4 * g + i;
                if (tok < T) po[static_cast<size_t>(tok) * 4096 + 128 * h + 16 * cb + n] = o[i];
            }
        };
        load_stage(0);
        store_stage(0);
        if (nch > 1) load_stage(1);
        load_out(0);
        for (int c = 0; c < nch; ++c) {
            __syncthreads();   // B0(c)
            // chunk c - 1's S^T and U stay published until the chain's (c) and
            // (b) of chunk c + 1
            if (c > 0) {
                output(c - 1);
                load_out(c);
            }
            if (c + 1 < nch) store_stage((c + 1) & 1);
            if (c + 2 < nch) load_stage(c + 2);
        }
        __syncthreads();   // B0(nch)
        output(nch - 1);
    }
}

hipError_t launch_deltanet_chunked(qff_ctx* ctx, hipStream_t stream, const qff_deltanet_params* p,
                                   const void* qkv, qff_dtype in_dtype, const float* a, const float* b,
                                   const float* conv_state, float* ssm_state, int T) {
    const int nch = (T + kC - 1) / kC;
    const bool bf = in_dtype == QFF_BF16;
    {
        ProfScope prof(ctx, stream, "dn_chunk_local");
        const int units = nch * 16;   // (chunk, key head)
        const int grid = std::min(units, std::max(ctx->num_cu, 1));
        unsigned* sched = ctx->sched + 2 * kSchedChunkLocal;
        if (bf)
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
