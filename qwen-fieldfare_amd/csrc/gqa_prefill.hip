// gqa_prefill.hip -- causal full-attention prefill (16 q heads on 2 kv heads,
// head dim 256) for T consecutive tokens of one sequence on gfx950.
//
// The reference has no prefill kernel: each prompt token runs the decode
// path at its position (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561,
// 1076-1150), so token t attends to positions 0 .. start+t. This file
// computes all T rows at once:
//   prep   one wave per token: head RMSNorm + partial RoPE of the
//          16 q heads (fp16, softmax scale folded in, to workspace: the
//          reference also rounds q to half, Runner:1119-1126) and of the 2 k
//          heads (appended to the cache, bf16 or fp16, together with v; a
//          bf16 cache's new rows also go to its fp16 copy in workspace, whose
//          older rows kv16_copy fills).
//   attn   flash attention. A workgroup owns 16 query tokens x the 8 q heads
//          of one kv head (128 rows; four wave pairs of 32 rows = 4 tokens
//          x 8 heads, each wave scoring half of a tile's positions and
//          accumulating half of the output dims, so accumulators and q stay
//          in VGPRs and two waves share each SIMD) and walks 64-position
//          K/V tiles copied from the fp16 cache (or the fp16 copy of a bf16
//          one: exact for the cache's values) straight into LDS
//          (double-buffered, XOR-swizzled rows, no registers),
//          so both products run on fp16 operands: S^T = K Q^T on 16x16x32
//          fp16 MFMAs (q keeps the 11-bit significand the reference gives
//          it, where bf16 q puts rare outputs beyond the output tolerance
//          once logits reach ~15); softmax in
//          base 2 (q carries scale * log2 e), with the running max raised
//          only when a tile exceeds it by more than 2^8, so the O rescale is
//          rare; causal masking only on the tiles that reach past the
//          block's first token. O += P V with 16x16x32 fp16 MFMAs (P in
//          fp16, 8x finer than bf16) whose 32-deep k
//          runs over the tile's positions in the order the S^T registers
//          hold them; the V operand comes from the row-major tile through the
//          LDS transpose read. The eight waves run as two groups one phase
//          apart (MFMA phase / softmax phase, see the kernel). Query blocks
//          are issued last-first so the longest rows start earliest. The
//          epilogue divides by the row sums and applies the sigmoid gate.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kPfQB = 16;       // query tokens per workgroup
constexpr int kPfKT = 64;       // K/V positions per tile

// One wave per token, 8 per workgroup: the token's 32 RoPE angles are
// evaluated once (lane i < 32: cos, sin of pos * f[i]) and shuffled to the
// lanes that rotate, then the 18 head slots (0-15 the q heads, 16-17 the kv
// heads) go in three rounds of six with each round's loads issued together.
// Lane l holds dims 4l .. 4l+3: the RMS is one wave reduction, and the RoPE
// partner of dim d < 32 (d + 32) sits 8 lanes up.
constexpr int kPrepWaves = 8;
constexpr int kPrepRound = 6;

template <int IN_DT, int KV_F16>
__global__ __launch_bounds__(64 * kPrepWaves) void gqa_prefill_prep_kernel(
    const void* __restrict__ q_gate, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w, RopeFreqs rf, float scale,
    float eps, int start, int T, uint16_t* __restrict__ qb, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, uint16_t* __restrict__ k16, uint16_t* __restrict__ v16) {
    const int lane = threadIdx.x & 63;
    const int tok = blockIdx.x * kPrepWaves + (threadIdx.x >> 6);
    if (tok >= T) return;
    const int pos = start + tok;
    float cs, sn;
    {
        const float ang = static_cast<float>(pos) * rf.f[lane & 31];
        cs = cosf(ang);
        sn = sinf(ang);
    }
    // (cos, sin) of this lane's four dims (d & 31 = (4 lane + i) & 31)
    float ci[4], si[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ci[i] = __shfl(cs, (4 * lane + i) & 31, 64);
        si[i] = __shfl(sn, (4 * lane + i) & 31, 64);
    }
    float qw[4], kw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qw[i] = q_norm_w[4 * lane + i];
        kw[i] = k_norm_w[4 * lane + i];
    }
    const float qs = scale * 1.44269504088896341f;
#pragma unroll
    for (int r0 = 0; r0 < 18; r0 += kPrepRound) {
        float x[kPrepRound][4];
#pragma unroll
        for (int j = 0; j < kPrepRound; ++j) {
            const int hs = r0 + j;
            const size_t src = hs < 16 ? (static_cast<size_t>(tok) * 16 + hs) * 512 + 4 * lane
                                       : (static_cast<size_t>(tok) * 2 + (hs - 16)) * 256 + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] = elem<IN_DT>::load(hs < 16 ? q_gate : k, src + i);
        }
        float vv[2][4];
        if (r0 + kPrepRound > 16) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    vv[j][i] = elem<IN_DT>::load(v, (static_cast<size_t>(tok) * 2 + j) * 256 + 4 * lane + i);
        }
#pragma unroll
        for (int j = 0; j < kPrepRound; ++j) {
            const int hs = r0 + j;
            const bool is_q = hs < 16;
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) ss += x[j][i] * x[j][i];
            ss = group_sum<64>(ss);
            const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = x[j][i] * inv * (is_q ? qw[i] : kw[i]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float up = __shfl_down(y[i], 8, 64), dn = __shfl_up(y[i], 8, 64);
                const int d = 4 * lane + i;
                if (d < 64) y[i] = (d < 32) ? y[i] * ci[i] + (-up) * si[i] : y[i] * ci[i] + dn * si[i];
            }
            if (is_q) {
                *reinterpret_cast<u32x2_t*>(qb + (static_cast<size_t>(tok) * 16 + hs) * 256 + 4 * lane) =
                    u32x2_t{pack_f16x2(y[0] * qs, y[1] * qs), pack_f16x2(y[2] * qs, y[3] * qs)};
            } else {
                const int kvh = hs - 16;
                const size_t off = (static_cast<size_t>(pos) * 2 + kvh) * 256 + 4 * lane;
                if (KV_F16) {
                    *reinterpret_cast<u32x2_t*>(k_cache + off) =
                        u32x2_t{pack_f16x2(y[0], y[1]), pack_f16x2(y[2], y[3])};
                    *reinterpret_cast<u32x2_t*>(v_cache + off) =
                        u32x2_t{pack_f16x2(vv[kvh][0], vv[kvh][1]), pack_f16x2(vv[kvh][2], vv[kvh][3])};
                } else {
                    // the bf16 entries, and their fp16 copy for the attention kernel
                    const u32x2_t kw2 = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
                    const u32x2_t vw2 = u32x2_t{pack_bf16x2(vv[kvh][0], vv[kvh][1]), pack_bf16x2(vv[kvh][2], vv[kvh][3])};
                    *reinterpret_cast<u32x2_t*>(k_cache + off) = kw2;
                    *reinterpret_cast<u32x2_t*>(v_cache + off) = vw2;
                    *reinterpret_cast<u32x2_t*>(k16 + off) = u32x2_t{bf16x2_to_f16x2(kw2[0]), bf16x2_to_f16x2(kw2[1])};
                    *reinterpret_cast<u32x2_t*>(v16 + off) = u32x2_t{bf16x2_to_f16x2(vw2[0]), bf16x2_to_f16x2(vw2[1])};
                }
            }
        }
    }
}

// The fp16 copy of bf16 cache rows 0 .. n-1 (both kv heads, K and V): one
// 16-byte piece of each per thread.
__global__ __launch_bounds__(256) void kv16_copy_kernel(const uint16_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ vc, uint16_t* __restrict__ k16,
                                                        uint16_t* __restrict__ v16, int pieces) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const size_t o = static_cast<size_t>(i) * 8;
    *reinterpret_cast<u32x4_t*>(k16 + o) = bf16x8_to_f16x8(*reinterpret_cast<const u32x4_t*>(kc + o));
    *reinterpret_cast<u32x4_t*>(v16 + o) = bf16x8_to_f16x8(*reinterpret_cast<const u32x4_t*>(vc + o));
}

constexpr int kPfThreads = 512;

// K and V tiles in LDS: 64 rows of 256 fp16 (512 B) without padding, the
// 16-byte pieces of row r XOR-permuted by swz(r): piece j of the row sits at
// j ^ swz(r). A K operand read (16 rows x one piece) and a V transpose read
// (16 rows x 2 pieces per 32 lanes) then each meet every bank group equally.
__device__ __forceinline__ int kv_swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// One wave's 1-KB chunk c (rows 2c, 2c + 1) of a 64-row tile, copied from
// the fp16 cache rows p0 + 2c, p0 + 2c + 1 straight into LDS: lane l fills
// LDS piece l % 32 of row 2c + h (h = l / 32) with global piece
// (l % 32) ^ swz(2c + h) = (l % 32) ^ 2h ^ U(c), U(c) = swz(2c) (2c is even,
// so swz(2c + h) = swz(2c) + 2h with bit 1 of swz(2c) clear): a lane term
// XORed with a uniform one, added to the uniform row base. Only the tile
// that reaches kv_end (tail) clamps rows at kv_end - 1 (finite data; their
// scores are masked).
template <bool TAIL>
__device__ __forceinline__ void kv_chunk_to_lds(const uint16_t* __restrict__ src, int kvh, int p0, int kv_end,
                                                uint16_t* tile, int c, int lane) {
    const int h = lane >> 5;
    // (redefined for the compiler at each chunk, so the offsets of all the
    // chunks are not formed ahead and held in registers)
    unsigned lt = 1024u * h + 16u * ((lane & 31) ^ (2 * h));
    asm volatile("" : "+v"(lt));
    const unsigned poff = lt ^ (16u * kv_swz(2 * c));
    const char* g;
    if constexpr (TAIL) {
        const int p = min(p0 + 2 * c + h, kv_end - 1);
        g = reinterpret_cast<const char*>(src) + (static_cast<size_t>(p) * 2 + kvh) * 512 + (poff & 1023u);
    } else {
        g = reinterpret_cast<const char*>(src) + (static_cast<size_t>(p0 + 2 * c) * 2 + kvh) * 512 + poff;
    }
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                     (__attribute__((address_space(3))) void*)(tile + 512 * c), 16, 0, 0);
}

// Chunks c0, c0 + step, ... (n of them) of the tile at rows p0 .. p0 + 63.
template <int N>
__device__ __forceinline__ void kv_tile_to_lds(const uint16_t* __restrict__ src, int kvh, int p0, int kv_end,
                                               uint16_t* tile, int c0, int step, int lane) {
    if (p0 + kPfKT > kv_end) {
#pragma unroll
        for (int i = 0; i < N; ++i) kv_chunk_to_lds<true>(src, kvh, p0, kv_end, tile, c0 + step * i, lane);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) kv_chunk_to_lds<false>(src, kvh, p0, kv_end, tile, c0 + step * i, lane);
    }
}

// A workgroup barrier between two phases of a wave's schedule; nothing
// (MFMAs included, which touch no memory) is moved across it.
__device__ __forceinline__ void phase_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
}

// grid (ceil(T/16), 2 kv heads), 512 threads: four wave pairs, pair pr
// owning the 32 rows of tokens t0 + 4 pr .. t0 + 4 pr + 3 (x the 8 q heads)
// as two 16-row tiles. Wave e of a pair scores positions 32e .. 32e + 31 of
// each K tile for both row tiles (each K operand read from LDS feeds two
// MFMAs), the pair meets once for the row maxima and once for the P
// operands (through LDS), and wave e accumulates output dims
// 128e .. 128e + 127 over all 64 positions (each V operand feeds two MFMAs):
// 34 KB of LDS reads per wave and tile instead of the 64 KB a wave of 16
// rows scoring every position and accumulating every dim would need.
//
// Schedule: two phases per tile between workgroup barriers -- M(j), on the
// MFMAs: S^T of tile j+1 interleaved with O += P V of tile j (20
// independent accumulator chains, operands read two steps ahead); V(j+1),
// on the VALU: the softmax of tile j+1 -- with waves 4-7 (group 1) one
// phase behind waves 0-3 (group 0): group 1 passes one barrier more at the
// start, group 0 one more at the end. Waves w and w + 4 share a SIMD, so
// while one issues MFMAs the other runs its softmax. Slots: group 0
// computes S_j in slot 2j and P V_j in slot 2j+2, group 1 one slot later, so
// K_j is read in slots 2j, 2j+1 and V_j in 2j+2, 2j+3. The tiles go from the
// fp16 cache (or its fp16 copy) straight into LDS, requested by group 1 in
// its V(m) (slot 2m+2): K_{m+2} into the buffer whose K_m was last read in
// 2m+1, V_{m+1} into the one whose V_{m-1} was last read in 2m+1; group 1
// waits for them at the end of its next M phase (slot 2m+3), before both
// are first read (slot 2m+4).
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(kPfThreads) void gqa_prefill_attn_kernel(
    const uint16_t* __restrict__ qb, const void* __restrict__ q_gate, const uint16_t* __restrict__ k16,
    const uint16_t* __restrict__ v16, int start, int T, void* __restrict__ out) {
    __shared__ __attribute__((aligned(1024))) uint16_t Ks[2][kPfKT * 256];
    __shared__ __attribute__((aligned(1024))) uint16_t Vs[2][kPfKT * 256];
    __shared__ float xrow[kPfThreads / 64][2][16];                              // per wave, row tile, row
    __shared__ __attribute__((aligned(16))) u32x4_t xp[kPfThreads / 64][2][64];  // per wave, row tile, lane
    const int nqb = (T + kPfQB - 1) / kPfQB;
    const int q_blk = nqb - 1 - static_cast<int>(blockIdx.x);
    const int kvh = blockIdx.y;
    const int t0 = q_blk * kPfQB;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int pr = wave >> 1, e = wave & 1, partner = wave ^ 1;
    const int wv = __builtin_amdgcn_readfirstlane(wave);   // the same, known uniform
    const int grp = wv >> 2;
    constexpr float kLazy = 8.0f;   // raise the running max only past 2^8

    // this lane's q rows: row tile rt = token t0 + 4 pr + 2 rt + n/8, head n%8
    u32x4_t qreg[2][8];
    int lim[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int tok_q = min(t0 + 4 * pr + 2 * rt + (n >> 3), T - 1);
        lim[rt] = start + tok_q;
        const uint16_t* qrow = qb + (static_cast<size_t>(tok_q) * 16 + kvh * 8 + (n & 7)) * 256;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) qreg[rt][jj] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * jj + 8 * kb);
        // consumed here (no instruction) so the loads are not sunk into the loop
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) asm volatile("" ::"v"(qreg[rt][jj]));
    }
    const int kv_end = start + min(T, t0 + kPfQB);
    const int ntiles = (kv_end + kPfKT - 1) / kPfKT;
    const int first_masked = (start + t0) / kPfKT;   // tiles before this need no causal mask

    float m_run[2] = {-INFINITY, -INFINITY}, d_run[2] = {0.0f, 0.0f};
    f32x4_t oacc[2][8];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int jd = 0; jd < 8; ++jd) oacc[rt][jd] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // K_0, V_0 and K_1 by every wave (32 chunks each, 4 a wave)
    kv_tile_to_lds<4>(k16, kvh, 0, kv_end, Ks[0], wv, 8, lane);
    kv_tile_to_lds<4>(v16, kvh, 0, kv_end, Vs[0], wv, 8, lane);
    if (ntiles > 1) kv_tile_to_lds<4>(k16, kvh, kPfKT, kv_end, Ks[1], wv, 8, lane);
    // every load so far (q included) has landed
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (grp) phase_barrier();   // group 1 runs one phase behind

    const int kp = 32 * e;      // the wave's first scored position in a tile
    f32x4_t s[2][2];            // S^T of the tile whose softmax comes next
    u32x4_t pa[2];              // the wave's P operands of the current tile

    // S^T = K Q^T of tile kt for the wave's two 16-position tiles x both row
    // tiles (32 dims a step), optionally interleaved with O += P V of tile
    // kt - 1 (four MFMAs of each a step); the masked row maxima of the
    // wave's 32 positions go to the partner
    auto mphase = [&](auto with_s, auto with_pv, int kt) {
        constexpr bool WS = decltype(with_s)::value, WPV = decltype(with_pv)::value;
        // the lane's K rows kp + 16pt + n (swz = kv_swz(n)), piece 4st + kb:
        // element (kp + n) 256 + 8 ((kb ^ swz) ^ 4st) = kidx ^ 32st
        const uint16_t* kbuf = Ks[kt & 1];
        const int kidx = (kp + n) * 256 + 8 * (kb ^ kv_swz(n));
        // PV of tile kt - 1: B operand through the LDS transpose read, lane
        // s of group kb at position 32c + 16h + 4kb + s/4, dims 128e + 16jd +
        // 4(s%4); A = the wave's own P (c = e), then the partner's (c = 1-e)
        // (rows 4kb + n/4 + 16h + 32c all permute by vr = kv_swz(4kb + n/4); the
        // lane's 4 dims are piece 16e + 2jd + (n%4)/2, half n%2 of it)
        // element (4kb + n/4) 256 + 128e + 8 (vx ^ 2jd) + 4 (n%2) = vidx ^ 16jd
        const uint16_t* vbuf = Vs[(kt + 1) & 1];
        const int vidx = (4 * kb + (n >> 2)) * 256 + 128 * e + 4 * (n & 1) +
                         8 * (((n & 3) >> 1) ^ kv_swz(4 * kb + (n >> 2)));
        u32x4_t A1[2];   // the partner's P operands, read for PV steps 4 .. 7
        auto load_a1 = [&]() {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) A1[rt] = xp[partner][rt][lane];
        };
        // S step st: dims 32st .. 32st + 31; PV step st: c = st / 4 (the wave's
        // own P, then the partner's), dims 16jd, jd = 2 (st % 4) + 0, 1. Each
        // operand is read kLead steps before its MFMAs, into rings of kLead + 1.
        // (The lane indices are redefined, as far as the compiler knows, at
        // every step, so each step's XOR is formed next to its reads instead
        // of all of them being held in registers across the loop.)
        constexpr int kLead = 3, kRing = kLead + 1;
        u32x4_t ka[kRing][2];
        u32x2_t va[kRing][4];
        auto load_k = [&](int st) {
            int ki = kidx;
            asm volatile("" : "+v"(ki));
            ki ^= 32 * st;
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
                ka[st % kRing][pt] = *reinterpret_cast<const u32x4_t*>(kbuf + ki + 16 * pt * 256);
        };
        auto load_v = [&](int st) {
            const int cc = st >> 2, jd0 = 2 * (st & 3);
            const uint16_t* vb = vbuf + 32 * (cc == 0 ? e : 1 - e) * 256;
            int vi = vidx;
            asm volatile("" : "+v"(vi));
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int o = vi ^ (16 * (jd0 + jj));
                va[st % kRing][2 * jj] = lds_read_tr16(vb + o);
                va[st % kRing][2 * jj + 1] = lds_read_tr16(vb + 16 * 256 + o);
            }
        };
        auto mfma_s = [&](int st) {
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) s[rt][pt] = mfma_16x16x32_f16(ka[st % kRing][pt], qreg[rt][st], s[rt][pt]);
        };
        auto mfma_pv = [&](int st) {
            const int cc = st >> 2, jd0 = 2 * (st & 3);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const u32x4_t B = u32x4_t{va[st % kRing][2 * jj][0], va[st % kRing][2 * jj][1], va[st % kRing][2 * jj + 1][0],
                                          va[st % kRing][2 * jj + 1][1]};
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    oacc[rt][jd0 + jj] = mfma_16x16x32_f16(cc == 0 ? pa[rt] : A1[rt], B, oacc[rt][jd0 + jj]);
            }
        };
        // masked row maxima of S^T over the wave's 32 positions, to the partner
        auto row_max = [&]() {
            if (kt >= first_masked) {   // (uniform) the tiles that reach the block's first token
                const int p0 = kt * kPfKT;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (p0 + kp + 16 * pt + 4 * kb + i > lim[rt]) s[rt][pt][i] = -INFINITY;
            }
            // over the lanes n, n + 16, n + 32, n + 48 on the permlane swaps
            // (VALU; an LDS permute would queue behind the operand reads)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                float tm = fmaxf(fmaxf(fmaxf(s[rt][0][0], s[rt][0][1]), fmaxf(s[rt][0][2], s[rt][0][3])),
                                 fmaxf(fmaxf(s[rt][1][0], s[rt][1][1]), fmaxf(s[rt][1][2], s[rt][1][3])));
                const auto h16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(tm), __float_as_uint(tm), false, false);
                tm = fmaxf(__uint_as_float(h16[0]), __uint_as_float(h16[1]));
                const auto h32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(tm), __float_as_uint(tm), false, false);
                tm = fmaxf(__uint_as_float(h32[0]), __uint_as_float(h32[1]));
                if (kb == 0) xrow[wave][rt][n] = tm;
            }
        };
        if constexpr (WS) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int pt = 0; pt < 2; ++pt) s[rt][pt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (WS && WPV) {
            // step u: S_u (u < 8) and PV_{u-2} (u >= 2), so S is done two steps
            // before the end and its row maxima run beside the last PV MFMAs;
            // K of S_{u+3} and V of PV_{u+1} are read at step u
#pragma unroll
            for (int st = 0; st < kLead; ++st) load_k(st);
            load_v(0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * kLead + 4, 0);
#pragma unroll
            for (int u = 0; u < 10; ++u) {
                if (u + kLead < 8) load_k(u + kLead);
                if (u + 1 < 8) load_v(u + 1);
                if (u == 4) load_a1();
                if (u < 8) mfma_s(u);
                if (u >= 2) mfma_pv(u - 2);
                if (u == 4) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
                else if (u + kLead < 8) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
                else if (u + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                if (u < 2 || u >= 8) __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                else __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                if (u == 8) row_max();
            }
        } else {
            // a single product: operands kLead steps ahead
            if constexpr (WPV) load_a1();
#pragma unroll
            for (int st = 0; st < kLead; ++st) {
                if constexpr (WS) load_k(st);
                if constexpr (WPV) load_v(st);
            }
#pragma unroll
            for (int st = 0; st < 8; ++st) {
                if (st + kLead < 8) {
                    if constexpr (WS) load_k(st + kLead);
                    if constexpr (WPV) load_v(st + kLead);
                }
                if constexpr (WS) mfma_s(st);
                if constexpr (WPV) mfma_pv(st);
            }
            if constexpr (WS) row_max();
        }
        // group 1's tile requests of its last V phase have landed (group 0
        // has none in flight)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    // softmax (base 2) of tile kt's S^T into the wave's P operands (to the
    // partner too); group 1 then requests K_{kt+2} and V_{kt+1}
    auto vphase = [&](bool with_softmax, int kt) {
        if (with_softmax) {
            // both waves of the pair take the same maxima and so keep the
            // same running max (the lazy rule sees the same values in both)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                float tm = fmaxf(xrow[wave][rt][n], xrow[partner][rt][n]);
                if (__any(tm > m_run[rt] + kLazy)) {
                    const float m_new = tm > m_run[rt] + kLazy ? tm : m_run[rt];
                    const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_new);
                    m_run[rt] = m_new;
                    d_run[rt] *= alpha;
                    float al[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
                    for (int jd = 0; jd < 8; ++jd)
#pragma unroll
                        for (int i = 0; i < 4; ++i) oacc[rt][jd][i] *= al[i];
                }
            }
            // k = 8kb + j of the A operand <-> position kp + 16(j/4) + 4kb + j%4
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                float pe[2][4];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        pe[h][i] = __builtin_amdgcn_exp2f(s[rt][h][i] - m_run[rt]);
                        d_run[rt] += pe[h][i];
                    }
                pa[rt] = u32x4_t{pack_f16x2(pe[0][0], pe[0][1]), pack_f16x2(pe[0][2], pe[0][3]),
                                 pack_f16x2(pe[1][0], pe[1][1]), pack_f16x2(pe[1][2], pe[1][3])};
                xp[wave][rt][lane] = pa[rt];
            }
        }
        if (grp) {
            // K_{kt+2} over K_kt and V_{kt+1} over V_{kt-1}: 32 chunks each, 8 a wave
            if (kt + 2 < ntiles) kv_tile_to_lds<8>(k16, kvh, (kt + 2) * kPfKT, kv_end, Ks[kt & 1], wv - 4, 4, lane);
            if (kt + 1 < ntiles) kv_tile_to_lds<8>(v16, kvh, (kt + 1) * kPfKT, kv_end, Vs[(kt + 1) & 1], wv - 4, 4, lane);
        }
    };

    mphase(std::true_type{}, std::false_type{}, 0);
    phase_barrier();
    vphase(true, 0);
    phase_barrier();
    for (int kt = 1; kt < ntiles; ++kt) {
        mphase(std::true_type{}, std::true_type{}, kt);
        phase_barrier();
        vphase(true, kt);
        phase_barrier();
    }
    mphase(std::false_type{}, std::true_type{}, ntiles);
    phase_barrier();
    if (!grp) phase_barrier();   // group 0 passes group 1's last barrier

    // epilogue: O / d * sigmoid(gate), d the pair's row sums;
    // oacc[rt][jd][i] = O[row 4kb+i of row tile rt][dim 128e + 16jd + n]
    float dt[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        float d = d_run[rt];
        d += __shfl_xor(d, 16, 64);
        d += __shfl_xor(d, 32, 64);
        dt[rt] = d;
        if (kb == 0) xrow[wave][rt][n] = d;
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const float d = dt[rt] + xrow[partner][rt][n];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * kb + i;
            const float inv_d = 1.0f / __shfl(d, row, 64);
            const int tok = t0 + 4 * pr + 2 * rt + (row >> 3);
            if (tok >= T) continue;
            const int h = kvh * 8 + (row & 7);
            const size_t qi = static_cast<size_t>(tok) * 16 + h;
#pragma unroll
            for (int jd = 0; jd < 8; ++jd) {
                const int dim = 128 * e + 16 * jd + n;
                const float g = elem<IN_DT>::load(q_gate, qi * 512 + 256 + dim);
                elem<OUT_DT>::store(out, qi * 256 + dim, oacc[rt][jd][i] * inv_d * sigmoid(g));
            }
        }
    }
}

hipError_t launch_gqa_prefill(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                              const void* q_gate, const void* k, const void* v, qff_dtype in_dtype,
                              void* k_cache, void* v_cache, int start_pos, void* out,
                              qff_dtype out_dtype, int T, int) {
    // the fp16 q rows [T][16][256] (workspace)
    uint16_t* qb = ctx->gqa_qb;
    uint16_t* kc = static_cast<uint16_t*>(k_cache);
    uint16_t* vc = static_cast<uint16_t*>(v_cache);
    const RopeFreqs rf = rope_freqs(p->rope_theta);
    // the attention kernel reads fp16 K and V: an fp16 cache itself, else
    // the fp16 copy in workspace ([max_ctx][2][256] K, then V), which the
    // prep kernel extends by the new rows and kv16_copy fills below start_pos
    uint16_t* k16 = p->kv_f16 ? kc : ctx->gqa_kv16;
    uint16_t* v16 = p->kv_f16 ? vc : ctx->gqa_kv16 + static_cast<size_t>(ctx->cfg.max_ctx) * 512;
    if (!p->kv_f16 && start_pos > 0) {
        ProfScope prof(ctx, stream, "gqa_prefill_kv16");
        const int pieces = start_pos * 64;
        kv16_copy_kernel<<<(pieces + 255) / 256, 256, 0, stream>>>(kc, vc, k16, v16, pieces);
    }
    {
        ProfScope prof(ctx, stream, "gqa_prefill_prep");
        const int pgrid = (T + kPrepWaves - 1) / kPrepWaves;
#define QFF_PREP(I, F)                                                                                           \
    gqa_prefill_prep_kernel<I, F><<<pgrid, 64 * kPrepWaves, 0, stream>>>(q_gate, k, v, p->q_norm_w, p->k_norm_w, \
                                                                        rf, p->scale, p->eps, start_pos, T, qb, \
                                                                        kc, vc, k16, v16)
        if (p->kv_f16) {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 1); else QFF_PREP(0, 1);
        } else {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 0); else QFF_PREP(0, 0);
        }
#undef QFF_PREP
    }
    const dim3 grid((T + kPfQB - 1) / kPfQB, 2);
    ProfScope prof(ctx, stream, "gqa_prefill_attn");
#define QFF_PFA(I, O) \
    gqa_prefill_attn_kernel<I, O><<<grid, kPfThreads, 0, stream>>>(qb, q_gate, k16, v16, start_pos, T, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_PFA(1, 1); else QFF_PFA(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_PFA(0, 1); else QFF_PFA(0, 0);
    }
#undef QFF_PFA
    return hipGetLastError();
}

}  // namespace qff
