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
//          heads (appended to the cache, bf16 or fp16, together with v).
//   attn   flash attention. A workgroup owns 16 query tokens x the 8 q heads
//          of one kv head (128 rows; four wave pairs of 32 rows = 4 tokens
//          x 8 heads, each wave scoring half of a tile's positions and
//          accumulating half of the output dims, so accumulators and q stay
//          in VGPRs and two waves share each SIMD) and walks 64-position
//          K/V tiles staged in LDS
//          row-major (double-buffered; the next tile's global loads are in
//          flight while the current one computes), converted from a bf16
//          cache to fp16 as they are staged (exact for the cache's values;
//          an fp16 cache, the reference's, is staged as it is),
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
//          LDS transpose read. Query blocks are issued last-first so the
//          longest rows start earliest. The epilogue divides by the row sums
//          and applies the sigmoid gate.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kPfQB = 16;       // query tokens per workgroup
constexpr int kPfKT = 64;       // K/V positions per tile
constexpr int kKStride = 264;   // fp16 per K row in LDS: 256 + 8 pad (528 B)

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
    uint16_t* __restrict__ v_cache) {
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
                    *reinterpret_cast<u32x2_t*>(k_cache + off) =
                        u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
                    *reinterpret_cast<u32x2_t*>(v_cache + off) =
                        u32x2_t{pack_bf16x2(vv[kvh][0], vv[kvh][1]), pack_bf16x2(vv[kvh][2], vv[kvh][3])};
                }
            }
        }
    }
}

constexpr int kPfThreads = 512;
constexpr int kPfPieces = kPfKT * 32 / kPfThreads;   // 16-B pieces of K (and of V) per thread

struct TileRegs {
    u32x4_t k[kPfPieces];
    u32x4_t v[kPfPieces];
};

// Thread t loads 16-byte pieces t + 512i of the K and V tile rows p0 ..
// p0+kPfKT-1 (row = piece / 32, dims 8 (piece % 32) .. +7); rows at or past
// kv_end read row kv_end - 1 instead (finite data; their scores are masked).

__device__ __forceinline__ void tile_load(TileRegs& r, const uint16_t* __restrict__ kc,
                                          const uint16_t* __restrict__ vc, int kvh, int p0, int kv_end,
                                          int t) {
#pragma unroll
    for (int i = 0; i < kPfPieces; ++i) {
        const int q = t + kPfThreads * i;
        const int p = min(p0 + (q >> 5), kv_end - 1);
        const size_t o = (static_cast<size_t>(p) * 2 + kvh) * 256 + 8 * (q & 31);
        r.k[i] = *reinterpret_cast<const u32x4_t*>(kc + o);
        r.v[i] = *reinterpret_cast<const u32x4_t*>(vc + o);
    }
}

// ... and stores them to LDS as fp16 (an fp16 cache's pieces as they are).
template <int KV_F16>
__device__ __forceinline__ void tile_store(const TileRegs& r, uint16_t* __restrict__ ks, uint16_t* __restrict__ vs,
                                           int t) {
#pragma unroll
    for (int i = 0; i < kPfPieces; ++i) {
        const int q = t + kPfThreads * i;
        const int o = (q >> 5) * kKStride + 8 * (q & 31);
        *reinterpret_cast<u32x4_t*>(ks + o) = KV_F16 ? r.k[i] : bf16x8_to_f16x8(r.k[i]);
        *reinterpret_cast<u32x4_t*>(vs + o) = KV_F16 ? r.v[i] : bf16x8_to_f16x8(r.v[i]);
    }
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
template <int IN_DT, int OUT_DT, int KV_F16>
__global__ __launch_bounds__(kPfThreads) void gqa_prefill_attn_kernel(
    const uint16_t* __restrict__ qb, const void* __restrict__ q_gate, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int start, int T, void* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kPfKT * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kPfKT * kKStride];
    __shared__ float xrow[kPfThreads / 64][2][16];                              // per wave, row tile, row
    __shared__ __attribute__((aligned(16))) u32x4_t xp[kPfThreads / 64][2][64];  // per wave, row tile, lane
    const int nqb = (T + kPfQB - 1) / kPfQB;
    const int q_blk = nqb - 1 - static_cast<int>(blockIdx.x);
    const int kvh = blockIdx.y;
    const int t0 = q_blk * kPfQB;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int pr = wave >> 1, e = wave & 1, partner = wave ^ 1;
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

    TileRegs regs;
    tile_load(regs, k_cache, v_cache, kvh, 0, kv_end, t);
    tile_store<KV_F16>(regs, Ks[0], Vs[0], t);
    // every load before the loop (q included) has landed: without this the
    // loop's waits would also cover the next tile's loads each iteration
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int kp = 32 * e;   // the wave's first scored position in a tile
    for (int kt = 0; kt < ntiles; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ntiles;
        if (more) tile_load(regs, k_cache, v_cache, kvh, (kt + 1) * kPfKT, kv_end, t);
        const int p0 = kt * kPfKT;
        // S^T = K Q^T for the wave's two 16-position tiles x both row tiles,
        // 32 dims at a time: the K operands of the next 32 dims are read
        // while the four independent MFMAs of these run
        f32x4_t s[2][2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int pt = 0; pt < 2; ++pt) s[rt][pt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        u32x4_t ka[2][2];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
            ka[0][pt] = *reinterpret_cast<const u32x4_t*>(&Ks[cur][(kp + 16 * pt + n) * kKStride + 8 * kb]);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            if (jj + 1 < 8) {
#pragma unroll
                for (int pt = 0; pt < 2; ++pt)
                    ka[(jj + 1) & 1][pt] = *reinterpret_cast<const u32x4_t*>(
                        &Ks[cur][(kp + 16 * pt + n) * kKStride + 32 * (jj + 1) + 8 * kb]);
            }
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) s[rt][pt] = mfma_16x16x32_f16(ka[jj & 1][pt], qreg[rt][jj], s[rt][pt]);
        }
        // softmax (base 2); lane holds q row n of each row tile, positions
        // p0 + kp + 16pt + 4kb + i; the pair's maxima over all 64 positions
        const bool masked = kt >= first_masked;
        float tm[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            tm[rt] = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (masked && p0 + kp + 16 * pt + 4 * kb + i > lim[rt]) s[rt][pt][i] = -INFINITY;
                    tm[rt] = fmaxf(tm[rt], s[rt][pt][i]);
                }
            tm[rt] = fmaxf(tm[rt], __shfl_xor(tm[rt], 16, 64));
            tm[rt] = fmaxf(tm[rt], __shfl_xor(tm[rt], 32, 64));
            if (kb == 0) xrow[wave][rt][n] = tm[rt];
        }
        __syncthreads();
        // both waves of the pair take the same maxima and so keep the same
        // running max (the lazy rule sees the same values in both)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            tm[rt] = fmaxf(tm[rt], xrow[partner][rt][n]);
            if (__any(tm[rt] > m_run[rt] + kLazy)) {
                const float m_new = tm[rt] > m_run[rt] + kLazy ? tm[rt] : m_run[rt];
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
        // P of the wave's 32 positions: the A operand of O += P V for that
        // 32-position chunk, k = 8kb + j <-> position kp + 16(j/4) + 4kb + j%4
        u32x4_t pa[2];
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
        __syncthreads();
        // O += P V for dims 128e .. 128e + 127: the wave's own chunk (pa),
        // then the partner's (its P operands, read back lane for lane); B
        // operand through the LDS transpose read: lane s of group kb points at
        // position 32c + 16h + 4kb + s/4, dims 128e + 16jd + 4(s%4)
        const uint16_t* vbase = &Vs[cur][(4 * kb + (n >> 2)) * kKStride + 4 * (n & 3) + 128 * e];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            u32x4_t A[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) A[rt] = cc == 0 ? pa[rt] : xp[partner][rt][lane];
            const uint16_t* vb = vbase + 32 * (cc == 0 ? e : 1 - e) * kKStride;
#pragma unroll
            for (int j0 = 0; j0 < 8; j0 += 4) {
                u32x2_t v0[4], v1[4];
#pragma unroll
                for (int jd = 0; jd < 4; ++jd) {
                    v0[jd] = lds_read_tr16(vb + 16 * (j0 + jd));
                    v1[jd] = lds_read_tr16(vb + 16 * kKStride + 16 * (j0 + jd));
                }
#pragma unroll
                for (int jd = 0; jd < 4; ++jd) {
                    const u32x4_t B = u32x4_t{v0[jd][0], v0[jd][1], v1[jd][0], v1[jd][1]};
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) oacc[rt][j0 + jd] = mfma_16x16x32_f16(A[rt], B, oacc[rt][j0 + jd]);
                }
            }
        }
        if (more) tile_store<KV_F16>(regs, Ks[cur ^ 1], Vs[cur ^ 1], t);
        __syncthreads();
    }

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
    {
        ProfScope prof(ctx, stream, "gqa_prefill_prep");
        const int pgrid = (T + kPrepWaves - 1) / kPrepWaves;
#define QFF_PREP(I, F)                                                                                           \
    gqa_prefill_prep_kernel<I, F><<<pgrid, 64 * kPrepWaves, 0, stream>>>(q_gate, k, v, p->q_norm_w, p->k_norm_w, \
                                                                        rf, p->scale, p->eps, start_pos, T, qb, \
                                                                        kc, vc)
        if (p->kv_f16) {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 1); else QFF_PREP(0, 1);
        } else {
            if (in_dtype == QFF_BF16) QFF_PREP(1, 0); else QFF_PREP(0, 0);
        }
#undef QFF_PREP
    }
    const dim3 grid((T + kPfQB - 1) / kPfQB, 2);
    ProfScope prof(ctx, stream, "gqa_prefill_attn");
#define QFF_PFA(I, O, F) \
    gqa_prefill_attn_kernel<I, O, F><<<grid, kPfThreads, 0, stream>>>(qb, q_gate, kc, vc, start_pos, T, out)
#define QFF_PFA_IO(F)                                                     \
    if (in_dtype == QFF_BF16) {                                           \
        if (out_dtype == QFF_BF16) QFF_PFA(1, 1, F); else QFF_PFA(1, 0, F); \
    } else {                                                              \
        if (out_dtype == QFF_BF16) QFF_PFA(0, 1, F); else QFF_PFA(0, 0, F); \
    }
    if (p->kv_f16) {
        QFF_PFA_IO(1)
    } else {
        QFF_PFA_IO(0)
    }
#undef QFF_PFA_IO
#undef QFF_PFA
    return hipGetLastError();
}

}  // namespace qff
