// gqa_prefill.hip -- causal full-attention prefill (16 q heads on 2 kv heads,
// head dim 256) for T consecutive tokens of one sequence on gfx950.
//
// The reference has no prefill kernel: each prompt token runs the decode
// path at its position (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561,
// 1076-1150), so token t attends to positions 0 .. start+t. This file
// computes all T rows in two launches:
//   prep   one wave per token: head RMSNorm + partial RoPE of the
//          16 q heads (fp16, softmax scale folded in, to workspace: the
//          reference also rounds q to half, Runner:1119-1126) and of the 2 k
//          heads (appended to the cache, bf16 or fp16, together with v; a
//          bf16 cache's new k rows also go to its fp16 copy in workspace).
//          The same launch's other workgroups write the transposed fp16
//          copy of V (per kv head and 64-position tile, dims x positions,
//          so that the attention's V operand is one 16-byte LDS read per
//          lane) and a bf16 cache's older k rows into the fp16 copy.
//   attn   flash attention. A workgroup owns 16 query tokens x the 8 q heads
//          of one kv head (128 rows; four wave pairs of 32 rows = 4 tokens
//          x 8 heads, each wave running its own flash attention over half of
//          every tile's positions with O^T over all 256 dims, the pair's
//          halves merged once at the end, so accumulators and q stay in
//          VGPRs and two waves share each SIMD) and walks 64-position
//          tiles of K (from the fp16 cache, or the fp16 copy of a bf16 one:
//          exact for the cache's values) and of V^T, copied straight into
//          LDS (double-buffered, XOR-swizzled rows, no registers), so both
//          products run on fp16 operands in the transposed orientation on
//          32x32x16 MFMAs: S^T = K Q^T (q keeps the 11-bit significand the
//          reference gives it, where bf16 q puts rare outputs beyond the
//          output tolerance once logits reach ~15) and O^T = V^T P^T (P in
//          fp16, 8x finer than bf16), each lane owning one q row of both.
//          Softmax in base 2 (q carries scale * log2 e), with the running
//          max raised only when a tile exceeds it by more than 2^8, so the
//          O rescale is rare; causal masking only on the tiles that reach
//          past the block's first token. One barrier per tile; the next
//          tiles' copies are requested inside the MFMA stream. Query blocks
//          are issued last-first so the longest rows start earliest. The
//          epilogue merges each pair's halves, divides by the row sums and
//          applies the sigmoid gate.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kPfQB = 16;       // query tokens per workgroup
constexpr int kPfKT = 64;       // K/V positions per tile

// The transposed fp16 copy of V, per kv head and 64-position tile a
// [256 dims][64 slots] block (the tile's 32 KB contiguous, tiles of one kv
// head ntile_stride apart). Within each 16 slots, slot 8h + 4j + i holds
// position 8j + 4h + i (bits 2 and 3 swapped): the order in which the
// attention's O^T = V^T P^T operand runs over positions, so a lane's eight
// positions are one 16-byte piece. Positions before start come from the
// cache, start .. start + T - 1 from the step's v (rounded to the cache's
// type first, exactly as the prep workgroups store them, so the copy holds
// the cache's values), later ones are zero. A workgroup of 512 threads
// stages one tile through LDS.
__device__ __forceinline__ int vt_slot_row(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }

template <int IN_DT, int KV_F16>
__device__ __forceinline__ void vt_tile_copy(const void* __restrict__ v, const uint16_t* __restrict__ vc,
                                             uint16_t* __restrict__ vt, int tl, int kvh, int start, int n,
                                             int ntile_stride) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[64][264];   // positions x dims (+8 pad)
    const int t = threadIdx.x;
    const int p0 = tl * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = t + 512 * i, row = q >> 5, pc = q & 31, p = p0 + row;
        u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
        if (p < start) {
            w = *reinterpret_cast<const u32x4_t*>(vc + (static_cast<size_t>(p) * 2 + kvh) * 256 + 8 * pc);
            if (!KV_F16) w = bf16x8_to_f16x8(w);
        } else if (p < n) {
            const size_t src = (static_cast<size_t>(p - start) * 2 + kvh) * 256 + 8 * pc;
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = elem<IN_DT>::load(v, src + e);
            if (KV_F16) {
                w = u32x4_t{pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]),
                            pack_f16x2(f[6], f[7])};
            } else {
                w = bf16x8_to_f16x8(u32x4_t{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                            pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])});
            }
        }
        *reinterpret_cast<u32x4_t*>(&tile[row][8 * pc]) = w;
    }
    __syncthreads();
    uint16_t* dst = vt + (static_cast<size_t>(kvh) * ntile_stride + tl) * (256 * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = t + 512 * i, d = q >> 3, sp = q & 7;   // dim d, slots 8 sp .. 8 sp + 7
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = static_cast<uint32_t>(tile[vt_slot_row(8 * sp + 2 * k)][d]) |
                   (static_cast<uint32_t>(tile[vt_slot_row(8 * sp + 2 * k + 1)][d]) << 16);
        *reinterpret_cast<u32x4_t*>(dst + d * 64 + 8 * sp) = u32x4_t{w[0], w[1], w[2], w[3]};
    }
}

// Launch layout of the prep kernel: vt_blocks workgroups of transposed-V
// tiles (two per 64-position tile, one per kv head), then k16_blocks
// workgroups copying a bf16 cache's K rows before start into the fp16 copy
// (512 16-byte pieces each), then one workgroup per 8 tokens of the prep
// proper. None depends on another: the copies read only rows the prep does
// not write, or the step's inputs.
struct PrepGrid {
    int vt_blocks, k16_blocks, vt_stride;
};

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
    uint16_t* __restrict__ v_cache, uint16_t* __restrict__ k16, uint16_t* __restrict__ vt, PrepGrid pg) {
    int blk = static_cast<int>(blockIdx.x);
    if (blk < pg.vt_blocks) {
        vt_tile_copy<IN_DT, KV_F16>(v, v_cache, vt, blk >> 1, blk & 1, start, start + T, pg.vt_stride);
        return;
    }
    blk -= pg.vt_blocks;
    if (blk < pg.k16_blocks) {
        // the fp16 copy of bf16 K cache rows 0 .. start - 1 (both kv heads)
        const int i = blk * 512 + static_cast<int>(threadIdx.x);
        if (i < start * 64) {
            const size_t o = static_cast<size_t>(i) * 8;
            *reinterpret_cast<u32x4_t*>(k16 + o) = bf16x8_to_f16x8(*reinterpret_cast<const u32x4_t*>(k_cache + o));
        }
        return;
    }
    blk -= pg.k16_blocks;
    const int lane = threadIdx.x & 63;
    const int tok = blk * kPrepWaves + (threadIdx.x >> 6);
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
                    // the bf16 entries, and the k entries' fp16 copy for the attention kernel
                    const u32x2_t kw2 = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
                    *reinterpret_cast<u32x2_t*>(k_cache + off) = kw2;
                    *reinterpret_cast<u32x2_t*>(v_cache + off) =
                        u32x2_t{pack_bf16x2(vv[kvh][0], vv[kvh][1]), pack_bf16x2(vv[kvh][2], vv[kvh][3])};
                    *reinterpret_cast<u32x2_t*>(k16 + off) = u32x2_t{bf16x2_to_f16x2(kw2[0]), bf16x2_to_f16x2(kw2[1])};
                }
            }
        }
    }
}

constexpr int kPfThreads = 512;

// K tiles in LDS: 64 rows of 256 fp16 (512 B) without padding, piece j
// (16 bytes) of row r at j ^ k_swz(r); V^T tiles: 256 rows (dims) of 64
// slots (128 B), piece j of row d at j ^ vt_swz(d). A K operand read (32
// rows x one piece per 32 lanes) and a V^T operand read (32 rows x one
// piece) then each meet every bank group equally.
// A b128 read at a 32-bit LDS byte address; a ^ x in one VALU instruction
// that the compiler neither hoists nor merges.
__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(static_cast<uintptr_t>(a));
}
__device__ __forceinline__ uint32_t lds_xor(uint32_t a, uint32_t x) {
    uint32_t r;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "s"(x), "v"(a));
    return r;
}

__device__ __forceinline__ int k_swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
__device__ __forceinline__ int vt_swz(int d) { return (d >> 1) & 7; }

// One wave's 1-KB chunk c (rows 2c, 2c + 1) of a 64-row K tile, copied from
// the fp16 cache rows p0 + 2c, p0 + 2c + 1 straight into LDS: lane l fills
// LDS piece l % 32 of row 2c + h (h = l / 32) with global piece
// (l % 32) ^ k_swz(2c + h) = (l % 32) ^ 2h ^ k_swz(2c) (bit 1 of k_swz(2c) is
// clear): a lane term XORed with a uniform one (one VALU instruction), as
// the 32-bit offset from a uniform row base. Only the tile that reaches
// kv_end (tail) clamps rows at kv_end - 1 (finite data; their scores are
// masked).
template <bool TAIL>
__device__ __forceinline__ void k_chunk_to_lds(const uint16_t* __restrict__ src, int kvh, int p0, int kv_end,
                                               uint16_t* tile, int c, int lane) {
    const int h = lane >> 5;
    const uint32_t lt = 1024u * h + 16u * ((lane & 31) ^ (2 * h));
    const uint32_t poff = lds_xor(lt, 16u * k_swz(2 * c));
    if constexpr (TAIL) {
        const int p = min(p0 + 2 * c + h, kv_end - 1);
        dma16(reinterpret_cast<const char*>(src) + (static_cast<size_t>(p0) * 2 + kvh) * 512,
              static_cast<uint32_t>(p - p0) * 1024u + (poff & 1023u), lds_addr(tile + 512 * c));
    } else {
        dma16(reinterpret_cast<const char*>(src) + (static_cast<size_t>(p0 + 2 * c) * 2 + kvh) * 512, poff,
              lds_addr(tile + 512 * c));
    }
}

// Chunks c0, c0 + step, ... (N of them) of the K tile at rows p0 .. p0 + 63.
template <int N>
__device__ __forceinline__ void k_tile_to_lds(const uint16_t* __restrict__ src, int kvh, int p0, int kv_end,
                                              uint16_t* tile, int c0, int step, int lane) {
    if (p0 + kPfKT > kv_end) {
#pragma unroll
        for (int i = 0; i < N; ++i) k_chunk_to_lds<true>(src, kvh, p0, kv_end, tile, c0 + step * i, lane);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) k_chunk_to_lds<false>(src, kvh, p0, kv_end, tile, c0 + step * i, lane);
    }
}

// Chunk c (dims 8c .. 8c + 7) of the V^T tile at src (32 KB), copied
// straight into LDS: lane l fills LDS piece
// l % 8 of row 8c + l / 8 with global piece (l % 8) ^ vt_swz(8c + l / 8) =
// (l % 8) ^ (l / 16) ^ 4 (c % 2). The copy is whole (rows past the cache
// end are zero), so no clamping.
__device__ __forceinline__ void vt_chunk_to_lds(const uint16_t* __restrict__ src, uint16_t* tile, int c, int lane) {
    const uint32_t lt = 128u * (lane >> 3) + 16u * ((lane & 7) ^ (lane >> 4));
    dma16(reinterpret_cast<const char*>(src) + 1024 * c, lds_xor(lt, 64u * (c & 1)), lds_addr(tile + 512 * c));
}

// A workgroup barrier that nothing (MFMAs included, which touch no memory)
// is moved across.
__device__ __forceinline__ void phase_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
}

// grid (ceil(T/16), 2 kv heads), 512 threads: four wave pairs, pair pr
// owning the 32 q rows r = 8 tt + hh (token t0 + 4 pr + tt, head hh of the
// kv head's 8). Lane l holds row l % 32 throughout. Wave e of a pair runs
// flash attention on its own over positions 32e .. 32e + 31 of every tile
// (its own running max and row sum, O^T over all 256 dims), and the pair
// merges its two halves once, at the end. Per tile a wave computes
// S^T = K Q^T on 32x32x16 fp16 MFMAs (A = 32 K rows x 16 dims from LDS, B
// = the row's q in registers; 16 steps) and O^T += V^T P^T (A = 32 dims x
// 16 positions of the V^T tile, B = P^T straight from the S^T accumulator:
// a lane's S^T and O^T registers belong to its one q row, so neither the
// softmax nor the rescale needs a lane exchange beyond the permlane swap
// of the two 16-position halves; 8 dim tiles x 2 steps). Each K or V
// operand read feeds 32 rows: 32 KB of LDS reads per wave and tile.
//
// Schedule: one workgroup barrier per tile. Iteration kt runs S^T of tile
// kt interleaved step by step with O^T += V^T P^T of tile kt - 1 (operands
// read kLead steps ahead; the wave at a raised priority), then the softmax
// of tile kt; it reads K_kt and V_{kt-1}, and during the first half of its
// MFMA stream (one request per step) every wave requests its share of
// K_{kt+1} (into the buffer K_{kt-1} left) and of V_kt (into the one
// V_{kt-2} left), straight into LDS, waiting for them before the next
// barrier. All eight waves run the same schedule, two per SIMD, so one
// wave's operand reads and softmax overlap the other's MFMAs.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(kPfThreads) void gqa_prefill_attn_kernel(
    const uint16_t* __restrict__ qb, const void* __restrict__ q_gate, const uint16_t* __restrict__ k16,
    const uint16_t* __restrict__ vt, int vt_stride, int start, int T, void* __restrict__ out) {
    // K tiles 0, 1 and V^T tiles 0, 1 (kvs[2], kvs[3]); after the loop,
    // each wave's 16 KB hand-over of O^T to its partner
    __shared__ __attribute__((aligned(1024))) uint16_t kvs[4][kPfKT * 256];
    __shared__ float xm[kPfThreads / 64][32], xd[kPfThreads / 64][32];   // per wave, q row
    const int nqb = (T + kPfQB - 1) / kPfQB;
    const int q_blk = nqb - 1 - static_cast<int>(blockIdx.x);
    const int kvh = blockIdx.y;
    const int t0 = q_blk * kPfQB;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wv = __builtin_amdgcn_readfirstlane(wave);   // the same, known uniform
    const int r = lane & 31, h = lane >> 5;
    const int pr = wave >> 1, e = wave & 1, partner = wave ^ 1;
    constexpr float kLazy = 8.0f;   // raise the running max only past 2^8

    // the lane's q row: token t0 + 4 pr + r / 8, head r % 8; B operand of S
    // step s = dims 16s + 8h .. +7
    const int tok_q = min(t0 + 4 * pr + (r >> 3), T - 1);
    const int lim = start + tok_q;
    u32x4_t qreg[16];
    {
        const uint16_t* qrow = qb + (static_cast<size_t>(tok_q) * 16 + kvh * 8 + (r & 7)) * 256 + 8 * h;
#pragma unroll
        for (int s = 0; s < 16; ++s) qreg[s] = *reinterpret_cast<const u32x4_t*>(qrow + 16 * s);
        // consumed here (no instruction) so the loads are not sunk into the loop
#pragma unroll
        for (int s = 0; s < 16; ++s) asm volatile("" ::"v"(qreg[s]));
    }
    const int kv_end = start + min(T, t0 + kPfQB);
    const int ntiles = (kv_end + kPfKT - 1) / kPfKT;
    const int first_masked = (start + t0) / kPfKT;   // tiles before this need no causal mask

    float m_run = -INFINITY, d_run = 0.0f;   // of the lane's row (the same in lanes r, r + 32)
    f32x16_t oacc[8];                        // O^T tile dt: dims 32dt + 8(i/4) + 4h + i%4
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.0f;

    // this kv head's V^T tiles (64 x 256 fp16 each)
    const uint16_t* __restrict__ vth = vt + static_cast<size_t>(kvh) * vt_stride * (kPfKT * 256);
    // K_0 by every wave (32 chunks, 4 a wave); every load so far (q
    // included) has landed at the first barrier
    k_tile_to_lds<4>(k16, kvh, 0, kv_end, kvs[0], wv, 8, lane);
    __builtin_amdgcn_s_waitcnt(0);

    const int kp = 32 * e;   // the wave's first position in a tile
    f32x16_t sacc;           // S^T: position kp + 8(i/4) + 4h + i%4
    u32x4_t pa[2];           // P^T operands of the previous tile (positions kp + 16m ..)

    // iteration kt: S^T of tile kt (WS) and O^T += V^T P^T of tile kt - 1
    // (WPV, step v: m = v / 8, dt = v % 8), then the softmax of tile kt
    auto iter = [&](auto with_s, auto with_pv, int kt) {
        constexpr bool WS = decltype(with_s)::value, WPV = decltype(with_pv)::value;
        phase_barrier();
        // K_{kt+1} (K_{ntiles-1} again in the last iteration, into the free
        // buffer) and V_kt: 32 chunks each, 4 a wave, one request per MFMA
        // step in the first half of the stream, so the requests queue while
        // the MFMAs run (the lane terms derived anew each time from an
        // opaque copy of the lane index, rather than held in registers
        // across the loop; the K rows clamped at kv_end - 1 in every tile,
        // so no branch splits the stream)
        int ln = static_cast<int>(threadIdx.x);
        asm volatile("" : "+v"(ln));
        ln &= 63;
        // the stream at a raised wave priority, the softmax at the normal one
        // (the SIMD's other wave then takes the MFMA issue slots it leaves)
        __builtin_amdgcn_s_setprio(1);
        const int kn = min(kt + 1, ntiles - 1);
        auto dma = [&](int i) {
            if constexpr (WS) {
                const int c = wv + 8 * (i >> 1);
                if (i & 1) vt_chunk_to_lds(vth + kt * (kPfKT * 256), kvs[2 + (kt & 1)], c, ln);
                else k_chunk_to_lds<true>(k16, kvh, kn * kPfKT, kv_end, kvs[(kt + 1) & 1], c, ln);
            }
        };
        // K operand of step s: row kp + r, piece 2s + h -> element
        // (kp + r) 256 + 8 ((h ^ k_swz(r)) ^ 2s) = kidx ^ 16s
        const int kidx = (kp + r) * 256 + 8 * (h ^ k_swz(r));
        // V^T operand of PV step (m, dt): row (dim) 32dt + r, slots
        // kp + 16m + 8h .. +7 (positions kp + 16m + 8j + 4h + i for
        // k = 8h + 4j + i), piece 4e + 2m + h permuted by vt_swz(r) ->
        // element (vidx ^ (kp + 16m)) + 2048 dt
        const int vidx = r * 64 + 8 * (h ^ vt_swz(r));
        constexpr int kLead = 2, kRing = kLead + 1;
        u32x4_t ka[kRing];
        u32x4_t va[kRing];
        // (the buffers are 1-KB aligned, so XOR of an element offset's low
        // bits is XOR of the LDS byte address's; each K step's XOR is one
        // VALU instruction, formed next to its read in an asm statement the
        // compiler cannot hoist, instead of all of them being held in
        // registers across the loop)
        const uint32_t kaddr = lds_addr(kvs[kt & 1] + kidx);
        const uint32_t vaddr = lds_addr(kvs[2 + ((kt + 1) & 1)] + vidx) ^ (64u * e);
        auto load_k = [&](int st) { ka[st % kRing] = lds_read_b128(lds_xor(kaddr, 32 * st)); };
        auto load_v = [&](int v) {
            const int m = v >> 3, dt = v & 7;
            va[v % kRing] = lds_read_b128((m ? (vaddr ^ 32u) : vaddr) + 4096 * dt);
        };
        auto mfma_s = [&](int st) { sacc = mfma_32x32x16_f16(ka[st % kRing], qreg[st], sacc); };
        auto mfma_pv = [&](int v) {
            const int m = v >> 3, dt = v & 7;
            oacc[dt] = mfma_32x32x16_f16(va[v % kRing], pa[m], oacc[dt]);
        };
        if constexpr (WS) {
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[i] = 0.0f;
        }
        if constexpr (WS && WPV) {
#pragma unroll
            for (int st = 0; st < kLead; ++st) {
                load_k(st);
                load_v(st);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * kLead, 0);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const bool ld = u + kLead < 16;
                if (ld) {
                    load_k(u + kLead);
                    load_v(u + kLead);
                }
                if (u < 8) dma(u);
                mfma_s(u);
                mfma_pv(u);
                if (ld) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            }
        } else {
            // a single product: operands kLead steps ahead
#pragma unroll
            for (int st = 0; st < kLead; ++st) {
                if constexpr (WS) load_k(st);
                if constexpr (WPV) load_v(st);
            }
#pragma unroll
            for (int st = 0; st < 16; ++st) {
                if (st + kLead < 16) {
                    if constexpr (WS) load_k(st + kLead);
                    if constexpr (WPV) load_v(st + kLead);
                }
                if (st < 8) dma(st);
                if constexpr (WS) mfma_s(st);
                if constexpr (WPV) mfma_pv(st);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        if constexpr (WS) {
            // softmax (base 2) of tile kt's S^T, masked, into the P^T operands
            if (kt >= first_masked) {   // (uniform) the tiles that reach the block's first token
                const int rel = lim - (kt * kPfKT + kp + 4 * h);
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (8 * (i >> 2) + (i & 3) > rel) sacc[i] = -INFINITY;
            }
            float tm = sacc[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) tm = fmaxf(tm, sacc[i]);
            // with the other 16 positions (lane r + 32) on the permlane swap
            const auto h32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(tm), __float_as_uint(tm), false, false);
            tm = fmaxf(__uint_as_float(h32[0]), __uint_as_float(h32[1]));
            // a row whose positions so far are all masked keeps m_run = -inf
            // and alpha 1 (its O^T and sum are zero), its P entries exp2(-inf)
            if (__any(tm > m_run + kLazy)) {
                const bool up = tm > m_run + kLazy;
                const float alpha = up ? __builtin_amdgcn_exp2f(m_run - tm) : 1.0f;
                if (up) m_run = tm;
                d_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
            }
            const float mb = m_run == -INFINITY ? 0.0f : m_run;
            // chunk m: k = 8h + 4j + i of the B operand <-> S^T element
            // 8m + 4j + i (position kp + 16m + 8j + 4h + i)
            float pe[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                pe[i] = __builtin_amdgcn_exp2f(sacc[i] - mb);
                d_run += pe[i];
            }
#pragma unroll
            for (int m = 0; m < 2; ++m)
                pa[m] = u32x4_t{pack_f16x2(pe[8 * m], pe[8 * m + 1]), pack_f16x2(pe[8 * m + 2], pe[8 * m + 3]),
                                pack_f16x2(pe[8 * m + 4], pe[8 * m + 5]), pack_f16x2(pe[8 * m + 6], pe[8 * m + 7])};
        }
        // this iteration's tile requests have landed (the softmax stays
        // ahead of the wait, which it would otherwise follow)
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };

    iter(std::true_type{}, std::false_type{}, 0);
    for (int kt = 1; kt < ntiles; ++kt) iter(std::true_type{}, std::true_type{}, kt);
    iter(std::false_type{}, std::true_type{}, ntiles);

    // epilogue: merge the pair's halves, O = (O_0 f_0 + O_1 f_1) / (d_0 f_0 +
    // d_1 f_1) with f_e = exp2(m_e - max(m_0, m_1)), d_e the row sums (the
    // lane's 16 positions plus lane r + 32's), then * sigmoid(gate). Wave e
    // finishes dims 128e .. 128e + 127 and hands the other half of its O^T
    // (dim tiles 4(1 - e) ..) to the partner through LDS (lane-major, one
    // 16-byte piece per lane and index).
    {
        const auto h32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(d_run), __float_as_uint(d_run), false, false);
        const float d = __uint_as_float(h32[0]) + __uint_as_float(h32[1]);
        if (h == 0) {
            xm[wave][r] = m_run;
            xd[wave][r] = d;
        }
        f32x4_t* const xo = reinterpret_cast<f32x4_t*>(kvs[0]) + wave * 1024;   // 16 KB a wave
        phase_barrier();   // every wave is done with the tiles
        auto hand_over = [&](auto ev) {
            constexpr int E = decltype(ev)::value;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xo[(4 * c + j) * 64 + lane] = f32x4_t{oacc[4 * (1 - E) + c][4 * j], oacc[4 * (1 - E) + c][4 * j + 1],
                                                         oacc[4 * (1 - E) + c][4 * j + 2],
                                                         oacc[4 * (1 - E) + c][4 * j + 3]};
        };
        if (e == 0) hand_over(std::integral_constant<int, 0>{});
        else hand_over(std::integral_constant<int, 1>{});
        __syncthreads();
        const float mp = xm[partner][r], dp = xd[partner][r];
        const float mx = fmaxf(m_run, mp);
        const float fo = __builtin_amdgcn_exp2f(m_run - mx), fp = __builtin_amdgcn_exp2f(mp - mx);
        const float inv_d = 1.0f / (d * fo + dp * fp);
        const float so = fo * inv_d, sp = fp * inv_d;
        const f32x4_t* const xq = reinterpret_cast<const f32x4_t*>(kvs[0]) + partner * 1024;
        const int tok = t0 + 4 * pr + (r >> 3);
        auto finish = [&](auto ev) {
            constexpr int E = decltype(ev)::value;
            if (tok >= T) return;
            const size_t qi = static_cast<size_t>(tok) * 16 + kvh * 8 + (r & 7);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int dim = 128 * E + 32 * c + 8 * j + 4 * h;
                    const f32x4_t po = xq[(4 * c + j) * 64 + lane];
                    float g[4], y[4];
                    if constexpr (IN_DT == 1) {
                        const u32x2_t w = *reinterpret_cast<const u32x2_t*>(
                            static_cast<const uint16_t*>(q_gate) + qi * 512 + 256 + dim);
                        g[0] = __uint_as_float(w[0] << 16);
                        g[1] = __uint_as_float(w[0] & 0xffff0000u);
                        g[2] = __uint_as_float(w[1] << 16);
                        g[3] = __uint_as_float(w[1] & 0xffff0000u);
                    } else {
                        const f32x4_t w = *reinterpret_cast<const f32x4_t*>(
                            static_cast<const float*>(q_gate) + qi * 512 + 256 + dim);
#pragma unroll
                        for (int i = 0; i < 4; ++i) g[i] = w[i];
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        y[i] = (oacc[4 * E + c][4 * j + i] * so + po[i] * sp) * sigmoid(g[i]);
                    if constexpr (OUT_DT == 1) {
                        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(out) + qi * 256 + dim) =
                            u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
                    } else {
                        *reinterpret_cast<f32x4_t*>(static_cast<float*>(out) + qi * 256 + dim) =
                            f32x4_t{y[0], y[1], y[2], y[3]};
                    }
                }
        };
        if (e == 0) finish(std::integral_constant<int, 0>{});
        else finish(std::integral_constant<int, 1>{});
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
    // the attention kernel reads fp16 K (an fp16 cache itself, else the fp16
    // copy in workspace, [max_ctx][2][256]) and the transposed fp16 copy of V
    // ([2][max_ctx / 64][256][64] in workspace), both written by the prep
    // launch
    uint16_t* k16 = p->kv_f16 ? kc : ctx->gqa_kv16;
    {
        // one launch: the transposed V copy (cache rows before start_pos and
        // the step's v), the fp16 copy of a bf16 cache's K rows before
        // start_pos, and the per-token prep (q to workspace, k / v appended,
        // a bf16 cache's new k rows also to the fp16 copy)
        ProfScope prof(ctx, stream, "gqa_prefill_prep");
        PrepGrid pg;
        pg.vt_stride = (ctx->cfg.max_ctx + kPfKT - 1) / kPfKT;   // tiles per kv head
        pg.vt_blocks = 2 * ((start_pos + T + kPfKT - 1) / kPfKT);
        pg.k16_blocks = p->kv_f16 ? 0 : (start_pos * 64 + 511) / 512;
        const int grid = pg.vt_blocks + pg.k16_blocks + (T + kPrepWaves - 1) / kPrepWaves;
#define QFF_PREP(I, F)                                                                                      \
    gqa_prefill_prep_kernel<I, F><<<grid, 64 * kPrepWaves, 0, stream>>>(q_gate, k, v, p->q_norm_w,          \
                                                                       p->k_norm_w, rf, p->scale, p->eps, \
                                                                       start_pos, T, qb, kc, vc, k16,     \
                                                                       ctx->gqa_vt, pg)
        if (p->kv_f16) {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 1); else QFF_PREP(0, 1);
        } else {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 0); else QFF_PREP(0, 0);
        }
#undef QFF_PREP
    }
    const int vt_stride = (ctx->cfg.max_ctx + kPfKT - 1) / kPfKT;
    const dim3 grid((T + kPfQB - 1) / kPfQB, 2);
    ProfScope prof(ctx, stream, "gqa_prefill_attn");
#define QFF_PFA(I, O) \
    gqa_prefill_attn_kernel<I, O><<<grid, kPfThreads, 0, stream>>>(qb, q_gate, k16, ctx->gqa_vt, vt_stride, \
                                                                   start_pos, T, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) QFF_PFA(1, 1); else QFF_PFA(1, 0);
    } else {
        if (out_dtype == QFF_BF16) QFF_PFA(0, 1); else QFF_PFA(0, 0);
    }
#undef QFF_PFA
    return hipGetLastError();
}

}  // namespace qff
