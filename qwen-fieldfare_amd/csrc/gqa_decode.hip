// gqa_decode.hip -- full-attention decode (16 q heads on 2 kv heads, head dim
// 256, bf16 or fp16 token-major KV cache) for a batch of sequences on gfx950.
//
// Reference: QwenQ4ActiveExpertStreamingRunner.swift:1076-1150 runs split
// q/gate, head RMSNorm, host RoPE tables + RoPE, the f16 KV append, a cast of
// q to half, Attention.encodeFull (split-KV partial + combine,
// attention.metal:134-224, 342-377; geometry Attention.swift:129-157) and the
// gate (deltanet.metal:700-708), one q head per threadgroup.
//
// Here the eight q heads that share a kv head run in the same wave, so every
// K/V byte is read from HBM once, and both products run on the matrix cores:
//   partial  one single-wave workgroup per (sequence, kv head, chunk) unit
//            (four-wave workgroups of four chunks and a persistent grid on an
//            atomic queue were measured no faster and slower). The wave
//            normalises and rotates the 8 q heads into LDS (bf16, softmax
//            scale and log2 e folded in); the one whose chunk holds the new
//            token also normalises/rotates k, appends k and v to the cache
//            and keeps both in LDS for its own use. It then walks 16-position
//            tiles with the next tile's K and V rows already in flight (two
//            register stages): S^T = K Q^T with 8 MFMA 16x16x32
//            (K rows straight from HBM, 16 B per lane; q as bf16 hi + lo
//            in the two 8-column halves of the MFMA's 16 columns, so the
//            scores see ~16 bits of q, more than the reference's fp16 q),
//            base-2 online softmax
//            per head whose running max is raised only past 2^8 (so O is
//            rarely rescaled), the V tile copied row-major into LDS and read
//            back as MFMA B operands with the gfx950 transpose read
//            (ds_read_b64_tr_b16), O += P V with 16 MFMA 16x16x16 (P as
//            bf16 hi + lo in the two 8-row halves), and one
//            (m, d, o[8][256]) partial per chunk (m in base-2 units).
//   combine  grid (q head, sequence): merges the chunk partials and applies
//            out = attn * sigmoid(gate).
// With an fp16 cache (the reference's, Runner:731-732) the same kernel runs
// its products on fp16 MFMAs (KV_F16): q and P become fp16 hi + lo pairs
// (~22 bits) and the appended k, v are rounded to fp16; K and V are exact
// in either MFMA type.
// Lengths come from the device `positions` array, so no host sync is needed;
// waves past a sequence's last chunk exit at once.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

constexpr int kDecTile = 16;          // positions per MFMA tile
constexpr int kVRowStride = 264;      // bf16 per V row in LDS: 256 + 8 pad (528 B)


struct DecTile {
    u32x4_t k[8], v[8];
};

// Wave-local LDS of one partial unit.
struct DecLds {
    uint16_t qs[8][256];                      // normed, rotated, scaled q: hi part (cache's type)
    uint16_t ql[8][256];                      // ... and lo part (q = hi + lo to ~2^-16 / 2^-22)
    uint16_t vs[kDecTile * kVRowStride];      // the current V tile, row-major
    uint16_t knew[256], vnew[256];            // the new token's k, v
    float2 rcs[32];                           // (cos, sin) of pos * f[i]
};

// Orders one wave's LDS stores before its later LDS loads by other lanes:
// a wave's LDS accesses complete in issue order, so only the compiler has to
// be kept from moving them (no s_barrier: waves of one workgroup run
// different units).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// One partial unit: chunk c (positions c * chunk_len ..) of sequence seq and
// kv head kvh, run by one wave on its own LDS. The wave normalises and
// rotates the 8 q heads; if the chunk holds the new token it also
// normalises / rotates k, appends k and v to the cache and keeps both in
// LDS for its own use. It then walks 16-position tiles: S^T = K Q^T with 8
// MFMA 16x16x32 (K rows straight from HBM, 16 B per lane; q as bf16 hi +
// lo in columns 0-7 / 8-15), base-2 online softmax per head whose running
// max is raised only past 2^8 (so O is rarely rescaled), the V tile copied
// row-major into LDS and read back as MFMA B operands with the gfx950
// transpose read (ds_read_b64_tr_b16), O += P V with 16 MFMA 16x16x16 (P as
// bf16 hi + lo in rows 0-7 / 8-15, added at the end), and writes one (m, d, o[8][256]) partial (m in base-2 units). The next
// tile's loads are in flight while a tile computes (two register stages).
template <int IN_DT, int KV_F16>
__device__ __forceinline__ void gqa_partial_unit(
    DecLds& L, int seq, int kvh, int c, int pos, int lane, const void* __restrict__ q_gate,
    const void* __restrict__ k_new, const void* __restrict__ v_new, const float* __restrict__ q_norm_w,
    const float* __restrict__ k_norm_w, const float* freqs, float scale, float eps,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int max_ctx, int chunk_len, int cstride,
    float* __restrict__ pm, float* __restrict__ pd, float* __restrict__ po) {
    const int p_start = c * chunk_len;
    const int p_end = min(pos + 1, p_start + chunk_len);
    const bool has_new = pos >= p_start && pos < p_end;   // then p_end - 1 == pos
    const size_t seq_base = static_cast<size_t>(seq) * max_ctx * 512 + kvh * 256;
    const int n = lane & 15, kb = lane >> 4;
    const uint16_t* Kb = k_cache + seq_base;
    const uint16_t* Vb = v_cache + seq_base;

    // K rows p0 + n (A of 16x16x32) and V rows p0 + 2i + lane/32 (dims
    // 8*(lane%32) .. +7). Rows past the chunk end re-read its last row: their
    // scores are masked to -inf, so they enter P V with probability 0 times
    // finite data (the cache past the sequence may hold any bit pattern, NaN
    // included, and is never read). Every row that lands on the new token's
    // position takes the LDS copy instead, so tiles may be loaded before the
    // append. The loads are unconditional so the compiler's vmcnt bookkeeping
    // stays exact across the two stages, and non-temporal (`nt`): every cache
    // byte is read once per step, so the stream does not displace the caches'
    // other contents (config 4 at B = 16 and 32K: 3.23 against 3.56 ms).
    // (the row addresses are rebuilt from an opaque copy of the lane index
    // each tile: kept live across the tile loop they would spill)
    auto load = [&](DecTile& tl, int p0) {
        int l = lane;
        asm volatile("" : "+v"(l));
        const uint16_t* krow = Kb + static_cast<size_t>(min(p0 + (l & 15), p_end - 1)) * 512;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            tl.k[jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(krow + 32 * jj + 8 * (l >> 4)));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int vp = min(p0 + 2 * i + (l >> 5), p_end - 1);
            tl.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Vb + static_cast<size_t>(vp) * 512 + 8 * (l & 31)));
        }
    };
    // ---- q: head RMSNorm + partial RoPE + scale, bf16 into LDS ---------------
    // (deltanet.metal:599-651; RoPE angles as QwenQ4ActiveExpertStreamingRunner
    // .swift:1090-1099 with host-computed inverse frequencies). Lane -> head
    // u/32, dims 8*(u%32) .. +7 for u = lane + 64 it; the RoPE pair (d, d^32)
    // of dims < 64 sits in lanes 4 apart. The q rows and norm weights are
    // requested first and the first tile's K/V rows right behind them, so
    // the q work waits for its own loads only.
    float xq[4][8], qw[8];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int u = 64 * it + lane;
        const size_t qbase = (static_cast<size_t>(seq) * 16 + kvh * 8 + (u >> 5)) * 512 + 8 * (u & 31);
#pragma unroll
        for (int i = 0; i < 8; ++i) xq[it][i] = elem<IN_DT>::load(q_gate, qbase + i);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) qw[i] = q_norm_w[8 * (lane & 31) + i];
    __builtin_amdgcn_sched_barrier(0);
    DecTile ta, tb;
    load(ta, p_start);
    __builtin_amdgcn_sched_barrier(0);
    if (lane < 32) {
        const float ang = static_cast<float>(pos) * freqs[lane];
        L.rcs[lane] = make_float2(cosf(ang), sinf(ang));
    }
    wave_lds_sync();
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int u = 64 * it + lane;
        const int hl = u >> 5, j = u & 31;
        float* x = xq[it];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
        ss = group_sum<32>(ss);
        const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = x[i] * inv * qw[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = 8 * j + i;
            const float partner = __shfl_xor(x[i], 4, 64);   // d +- 32 (used when d < 64)
            if (d < 64) {
                const float2 r = L.rcs[d & 31];
                x[i] = (d < 32) ? x[i] * r.x + (-partner) * r.y : x[i] * r.x + partner * r.y;
            }
        }
        const float qscale = scale * 1.44269504088896341f;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            uint32_t hi, lo;
            if (KV_F16) split_f16x2(x[i] * qscale, x[i + 1] * qscale, hi, lo);
            else split_bf16x2(x[i] * qscale, x[i + 1] * qscale, hi, lo);
            *reinterpret_cast<uint32_t*>(&L.qs[hl][8 * j + i]) = hi;
            *reinterpret_cast<uint32_t*>(&L.ql[hl][8 * j + i]) = lo;
        }
    }
    // ---- the new token (only the unit whose chunk holds it): k norm + RoPE,
    // append k and v to the cache (deltanet.metal:670-689), keep both in LDS
    // so the wave never reads back its own global stores.
    if (has_new) {
        const size_t kb0 = (static_cast<size_t>(seq) * 2 + kvh) * 256 + 4 * lane;
        float kx[4], vx[4], ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kx[i] = elem<IN_DT>::load(k_new, kb0 + i);
            vx[i] = elem<IN_DT>::load(v_new, kb0 + i);
            ss += kx[i] * kx[i];
        }
        ss = group_sum<64>(ss);
        const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
        for (int i = 0; i < 4; ++i) kx[i] = kx[i] * inv * k_norm_w[4 * lane + i];
        // dims 4*lane .. +3; RoPE partner of dim d < 32 is d + 32 = lane + 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float up = __shfl_down(kx[i], 8, 64), dn = __shfl_up(kx[i], 8, 64);
            const int d = 4 * lane + i;
            if (d < 64) {
                const float2 r = L.rcs[d & 31];
                kx[i] = (d < 32) ? kx[i] * r.x + (-up) * r.y : kx[i] * r.x + dn * r.y;
            }
        }
        const uint32_t k01 = KV_F16 ? pack_f16x2(kx[0], kx[1]) : pack_bf16x2(kx[0], kx[1]);
        const uint32_t k23 = KV_F16 ? pack_f16x2(kx[2], kx[3]) : pack_bf16x2(kx[2], kx[3]);
        const uint32_t v01 = KV_F16 ? pack_f16x2(vx[0], vx[1]) : pack_bf16x2(vx[0], vx[1]);
        const uint32_t v23 = KV_F16 ? pack_f16x2(vx[2], vx[3]) : pack_bf16x2(vx[2], vx[3]);
        *reinterpret_cast<u32x2_t*>(&L.knew[4 * lane]) = u32x2_t{k01, k23};
        *reinterpret_cast<u32x2_t*>(&L.vnew[4 * lane]) = u32x2_t{v01, v23};
        const size_t off = seq_base + static_cast<size_t>(pos) * 512 + 4 * lane;
        *reinterpret_cast<u32x2_t*>(k_cache + off) = u32x2_t{k01, k23};
        *reinterpret_cast<u32x2_t*>(v_cache + off) = u32x2_t{v01, v23};
    }
    wave_lds_sync();

    // q^T (B of 16x16x32): col n = head n & 7, its hi part for n < 8 and
    // lo part for n >= 8 (the columns a group of 8 heads leaves free), k =
    // dims 32jj + 8kb .. +7, read from LDS per tile (registers are kept for
    // the two tile stages)
    const uint16_t* qrow = n < 8 ? &L.qs[n][8 * kb] : &L.ql[n - 8][8 * kb];
    uint16_t* vsw = L.vs;
    constexpr float kLazy = 8.0f;   // raise the running max only past 2^8

    float m_run = -INFINITY, d_run = 0.0f;
    f32x4_t oacc[16];
#pragma unroll
    for (int jd = 0; jd < 16; ++jd) oacc[jd] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](DecTile& tl, int p0) {
        // (the opaque copy keeps the compiler from folding the LDS read into
        // the tile load as one flat load through a selected pointer)
        if (has_new && p0 + n >= pos) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                u32x4_t kv = *reinterpret_cast<const u32x4_t*>(&L.knew[32 * jj + 8 * kb]);
                asm volatile("" : "+v"(kv));
                tl.k[jj] = kv;
            }
        }
        // S^T = K Q^T, q as hi + lo (K is exact in the cache's type): the
        // scores carry ~16 (bf16) or ~22 (fp16) significant bits of q, finer
        // than the reference's fp16 q.
        // Column n scores against head n & 7's hi (n < 8) or lo (n >= 8)
        // part; lanes n and n ^ 8 (DPP row rotate by 8) add the two, so
        // both hold head n & 7's scores from here on.
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const u32x4_t qop = *reinterpret_cast<const u32x4_t*>(qrow + 32 * jj);
            s = KV_F16 ? mfma_16x16x32_f16(tl.k[jj], qop, s) : mfma_16x16x32_bf16(tl.k[jj], qop, s);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] += dpp_mov<0x128>(s[i]);
        // V tile row-major into LDS (the new token's row from LDS as well)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 2 * i + (lane >> 5);
            u32x4_t v = tl.v[i];
            if (has_new && p0 + r >= pos) {   // rows clamped to the new token's position
                v = *reinterpret_cast<const u32x4_t*>(&L.vnew[8 * (lane & 31)]);
                asm volatile("" : "+v"(v));
            }
            *reinterpret_cast<u32x4_t*>(&vsw[r * kVRowStride + 8 * (lane & 31)]) = v;
        }
        // online softmax (base 2); lane holds head n, positions p0 + 4kb + i
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (p0 + 4 * kb + i >= p_end) s[i] = -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        if (__any(tmax > m_run + kLazy)) {
            const float m_new = tmax > m_run + kLazy ? tmax : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            d_run *= alpha;
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
            for (int jd = 0; jd < 16; ++jd)
#pragma unroll
                for (int i = 0; i < 4; ++i) oacc[jd][i] *= al[i];
        }
        float pe[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pe[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
            d_run += pe[i];
        }
        // A of O += P V (16x16x16): row n = head n & 7, k = positions 4kb ..
        // +3, P's hi part in rows 0-7 and lo part in rows 8-15 (V is exact
        // in the cache's type), so rows h and h + 8 of O sum to head h's output
        uint32_t ph0, pl0, ph1, pl1;
        if (KV_F16) {
            split_f16x2(pe[0], pe[1], ph0, pl0);
            split_f16x2(pe[2], pe[3], ph1, pl1);
        } else {
            split_bf16x2(pe[0], pe[1], ph0, pl0);
            split_bf16x2(pe[2], pe[3], ph1, pl1);
        }
        const u32x2_t pa = n < 8 ? u32x2_t{ph0, ph1} : u32x2_t{pl0, pl1};
        // B = V^T block straight from the row-major tile with a transpose read:
        // source lane (group kb, s = n) points at row 4kb + n/4, dims
        // 16jd + 4(n%4) .. +3, and receives V[4kb + k][16jd + n], k = 0..3.
        wave_lds_sync();
        const uint16_t* vsrc = &vsw[(4 * kb + (n >> 2)) * kVRowStride + 4 * (n & 3)];
#pragma unroll
        for (int jd = 0; jd < 16; ++jd) {
            const u32x2_t vb = lds_read_tr16(vsrc + 16 * jd);
            oacc[jd] = KV_F16 ? mfma_16x16x16_f16(pa, vb, oacc[jd]) : mfma_16x16x16_bf16(pa, vb, oacc[jd]);
        }
        wave_lds_sync();
    };
    // (issuing both stages before the q work was measured slower: 254
    // VGPRs and a longer issue stall ahead of the q loads)
    int p0 = p_start;
    for (; p0 + kDecTile < p_end; p0 += 2 * kDecTile) {
        load(tb, p0 + kDecTile);
        compute(ta, p0);
        load(ta, p0 + 2 * kDecTile);
        compute(tb, p0 + kDecTile);
    }
    if (p0 < p_end) compute(ta, p0);
    // ---- partial (m, d, o) of this chunk; oacc[jd][i] = O[row 4kb+i][dim 16jd+n],
    // rows 0-7 (lanes 0-31) the hi parts and rows 8-15 (lanes 32-63) the lo
    // parts of heads 0-7
    d_run += __shfl_xor(d_run, 16, 64);
    d_run += __shfl_xor(d_run, 32, 64);
    const size_t pbase = (static_cast<size_t>(seq) * 2 + kvh) * cstride + c;
    if (lane < 8) {
        pm[pbase * 8 + lane] = m_run;
        pd[pbase * 8 + lane] = d_run;
    }
#pragma unroll
    for (int jd = 0; jd < 16; ++jd)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(oacc[jd][i]),
                                                            __float_as_uint(oacc[jd][i]), false, false);
            oacc[jd][i] = __uint_as_float(h[0]) + __uint_as_float(h[1]);
        }
    if (kb < 2) {
        float* orow = po + pbase * 8 * 256;
#pragma unroll
        for (int jd = 0; jd < 16; ++jd)
#pragma unroll
            for (int i = 0; i < 4; ++i) orow[(4 * kb + i) * 256 + 16 * jd + n] = oacc[jd][i];
    }
}

// ---- split of a call's positions into chunks ----------------------------------
//
// Every workgroup of the partial and combine launches derives the same split
// from the device `positions` (no host sync, no atomics): the chunk length
// ch (a multiple of 32 positions, at least 32) makes about `target` chunks
// per kv head out of the batch's total attended length P = sum_b L_b,
// whatever the individual lengths, and at most `cap` chunks per sequence;
// sequence b takes nc_b = ceil(L_b / ch) chunks, numbered from
// first_b = sum_{b' < b} nc_b'. A sequence whose position lies outside the
// cache has length 0 (no chunks; its outputs are NaN).
__device__ __forceinline__ int gqa_len(const int32_t* __restrict__ positions, int b, int max_ctx) {
    const int pos = positions[b];
    return (pos >= 0 && pos < max_ctx) ? pos + 1 : 0;
}

// The split as seen by one wave: chunk length ch (every lane) and, for
// global chunk index g, its (sequence, chunk), or seq = -1 past the last
// chunk, and that sequence's length len = position + 1.
// Lane l reads positions l, l + 64, ...; batches up to 64 read them
// once. The K/V streams of a partial workgroup wait for this, so the
// reductions and the prefix run on DPP moves, not LDS permutes.
__device__ __forceinline__ void gqa_split(const int32_t* __restrict__ positions, int batch, int max_ctx, int target,
                                          int cap, int g, int lane, int& ch, int& seq, int& c, int& len) {
    const int L0 = lane < batch ? gqa_len(positions, lane, max_ctx) : 0;
    long long P = wave_sum_int(L0);
    int maxL = wave_max_int(L0);
    for (int b0 = 64; b0 < batch; b0 += 64) {
        const int L = b0 + lane < batch ? gqa_len(positions, b0 + lane, max_ctx) : 0;
        P += wave_sum_int(L);
        maxL = max(maxL, wave_max_int(L));
    }
    const int by_total = static_cast<int>((P + target - 1) / target), by_cap = (maxL + cap - 1) / cap;
    ch = (max(max(by_total, by_cap), 1) + 31) / 32 * 32;
    seq = -1;
    c = 0;
    len = 0;
    int base = 0;
    for (int b0 = 0; b0 < batch; b0 += 64) {
        const int L = b0 == 0 ? L0 : (b0 + lane < batch ? gqa_len(positions, b0 + lane, max_ctx) : 0);
        const int nc = (L + ch - 1) / ch;
        const int incl = base + wave_inclusive_scan_int(nc);   // chunks of sequences b0 .. b0 + lane
        // the first lane whose inclusive count exceeds g holds chunk g
        const unsigned long long hit = __ballot(incl > g);
        if (hit) {
            const int src = static_cast<int>(__builtin_ctzll(hit));
            seq = b0 + src;
            c = g - (__builtin_amdgcn_readlane(incl, src) - __builtin_amdgcn_readlane(nc, src));
            len = __builtin_amdgcn_readlane(L, src);
            return;
        }
        base = __builtin_amdgcn_readlane(incl, 63);
    }
}

// grid 2 x (target + batch), one wave each: workgroup u takes kv head u & 1
// of global chunk u >> 1 of the split above (workgroups past the last chunk
// exit at once). The kv head is the fastest-varying index, so the two heads'
// workgroups of a chunk are dispatched together and stream the interleaved
// halves of the same cache records at the same time. Two single-wave
// workgroups per SIMD stay resident, each with its next tile in flight.
template <int IN_DT, int KV_F16>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
void gqa_decode_partial_kernel(
    const void* __restrict__ q_gate, const void* __restrict__ k_new, const void* __restrict__ v_new,
    const float* __restrict__ q_norm_w, const float* __restrict__ k_norm_w, RopeFreqs rf, float scale,
    float eps, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ positions, int batch, int max_ctx, int target, int cstride,
    float* __restrict__ pm, float* __restrict__ pd, float* __restrict__ po) {
    const int lane = threadIdx.x & 63;
    const int kvh = blockIdx.x & 1;
    int chunk_len, seq, c, len;
    gqa_split(positions, batch, max_ctx, target, cstride, static_cast<int>(blockIdx.x >> 1), lane, chunk_len, seq, c,
              len);
    // past the last chunk; sequences whose position lies outside the cache
    // (the caller's error) have no chunks: the combine writes NaN for them
    if (seq < 0) return;
    const int pos = len - 1;
    __shared__ __attribute__((aligned(16))) DecLds lds;
    __shared__ float freqs[32];
    if (lane < 32) freqs[lane] = rf.f[lane];
    wave_lds_sync();
    gqa_partial_unit<IN_DT, KV_F16>(lds, seq, kvh, c, pos, lane, q_gate, k_new, v_new, q_norm_w, k_norm_w, freqs,
                                    scale, eps, k_cache, v_cache, max_ctx, chunk_len, cstride, pm, pd, po);
}

// grid (16 q heads x DS dim blocks, batch), 512 threads: attention.metal
// :342-377 merge, then the gate of deltanet.metal:700-708, for 256 / DS dims
// per workgroup (DS = 4 at small batches, so more than 16 workgroups share
// the partial reads). Chunk weights are formed one thread per chunk; the
// 8 DS chunk streams (stream s sums chunks s, s + 8 DS, ...; 64 / DS lanes
// per stream, a float4 of dims per lane) add their chunks in order, and
// their sums are added in LDS in a fixed order. The loads form a short
// chain: the (m, d) of every slot of the (sequence, kv head) and the gate
// are requested with the positions the split reads, and each stream's first
// four partial rows as soon as the split gives the chunk count, before the
// maxima and weights are known. Every load is unconditional, its index
// clamped to the workspace's slots or the call's chunks (a clamped row gets
// no weight): a load under a branch makes the compiler wait for all loads
// in flight where the branch ends. (Requesting the rows before the split,
// clamped to the workspace's slots, was slower: slots past the call's
// chunks hold rows this call did not write, which come from HBM.)
template <int IN_DT, int OUT_DT, int DS>
__global__ __launch_bounds__(512) void gqa_decode_combine_kernel(
    const void* __restrict__ q_gate, const int32_t* __restrict__ positions, int batch, int max_ctx, int target,
    int cstride, const float* __restrict__ pm, const float* __restrict__ pd, const float* __restrict__ po,
    void* __restrict__ out) {
    constexpr int kDims = 256 / DS, kLanes = 64 / DS, kStreams = 8 * DS, kRound = 4;
    __shared__ float es[kGqaMaxChunks], red[16];
    __shared__ __attribute__((aligned(16))) float osum[kStreams][kDims];
    const int h = blockIdx.x / DS, dblk = blockIdx.x % DS, seq = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int kvh = h >> 3, hl = h & 7;
    const int d0 = dblk * kDims;
    const size_t qi = (static_cast<size_t>(seq) * 16 + h);
    const size_t base = (static_cast<size_t>(seq) * 2 + kvh) * cstride;
    // every slot of this (sequence, kv head) lies in the workspace (cstride
    // <= 512 threads); slots past the call's chunk count are masked below
    const int ts = min(t, cstride - 1);
    const float m_slot = pm[(base + ts) * 8 + hl];
    const float d_slot = pd[(base + ts) * 8 + hl];
    const float gate = elem<IN_DT>::load(q_gate, qi * 512 + 256 + d0 + min(t, kDims - 1));
    const int pos = positions[seq];
    if (pos < 0 || pos >= max_ctx) {
        if (t < kDims) elem<OUT_DT>::store(out, qi * 256 + d0 + t, __builtin_nanf(""));
        return;
    }
    int chunk_len, unused_seq, unused_c, unused_len;
    gqa_split(positions, batch, max_ctx, target, cstride, 0, lane, chunk_len, unused_seq, unused_c, unused_len);
    const int L = pos + 1;
    const int nc = (L + chunk_len - 1) / chunk_len;   // <= cstride
    const int sid = wave * DS + lane / kLanes, f = lane % kLanes;
    // chunk c of this head at pr[c * 512]
    const float4* pr = reinterpret_cast<const float4*>(po + (base * 8 + hl) * 256 + d0) + f;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 v[kRound];
#pragma unroll
    for (int u = 0; u < kRound; ++u) v[u] = pr[static_cast<size_t>(min(sid + kStreams * u, nc - 1)) * 512];
    const float m = t < nc ? m_slot : -INFINITY;
    const float d = t < nc ? d_slot : 0.0f;
    const float wmax = group_max<64>(m);
    if (lane == 0) red[wave] = wmax;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) M = fmaxf(M, red[w]);
    const float e = t < nc ? __builtin_amdgcn_exp2f(m - M) : 0.0f;   // m are base-2 maxima
    if (t < kGqaMaxChunks) es[t] = e;
    const float wd = group_sum<64>(d * e);
    if (lane == 0) red[8 + wave] = wd;
    __syncthreads();
    float4 acc = zero;
    for (int c = sid; c < nc; c += kRound * kStreams) {
        float4 cur[kRound];
#pragma unroll
        for (int u = 0; u < kRound; ++u) cur[u] = v[u];
        // the next round's rows, requested before this round's sums
#pragma unroll
        for (int u = 0; u < kRound; ++u)
            v[u] = pr[static_cast<size_t>(min(c + kStreams * (kRound + u), nc - 1)) * 512];
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            const int cc = c + kStreams * u;
            const float w = es[min(cc, kGqaMaxChunks - 1)];
            if (cc < nc) {
                acc.x += cur[u].x * w; acc.y += cur[u].y * w; acc.z += cur[u].z * w; acc.w += cur[u].w * w;
            }
        }
    }
    reinterpret_cast<float4*>(osum[sid])[f] = acc;
    __syncthreads();
    if (t < kDims) {
        float D = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) D += red[8 + w];
#pragma unroll
        for (int s2 = 0; s2 < kStreams; ++s2) O += osum[s2][t];
        elem<OUT_DT>::store(out, qi * 256 + d0 + t, (O / D) * sigmoid(gate));
    }
}

// Chunks per (sequence, kv head) available to a call of this batch: the
// workspace's partial slots spread over the batch, at most kGqaMaxChunks.
int gqa_chunk_cap(const qff_ctx_cfg& cfg, int batch) {
    const int cap = gqa_slots(cfg) / (2 * batch);
    return cap < kGqaMaxChunks ? cap : kGqaMaxChunks;
}

// Chunks per kv head a call aims for: half a round of resident one-wave
// workgroups (two per SIMD, 8 per CU) over both kv heads. Measured at
// context 8192 with random lengths and config 4: 2 x CUs beat 4 x (batch 8
// 26.6 vs 28.9 us, config 4 at batch 16 3.72 vs 3.81 ms) and 8 x. A single
// sequence takes 1 x CUs: half the partials for the combine to merge
// (config 4 at batch 1 and 64K: 999-1000 against 1014-1016 us per step;
// 0.5 x: 1099 us); at context 8192 both give 32-position chunks.
static int gqa_target_chunks(int num_cu, int batch) {
    const int n = num_cu > 0 ? num_cu : 256;
    return batch == 1 ? n : 2 * n;
}

hipError_t launch_gqa_decode(qff_ctx* ctx, hipStream_t stream, const qff_gqa_params* p,
                             const void* q_gate, const void* k_new, const void* v_new,
                             qff_dtype in_dtype, void* k_cache, void* v_cache,
                             const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                             int max_ctx) {
    const GqaPartials ws{ctx->gqa_m, ctx->gqa_d, ctx->gqa_o, gqa_chunk_cap(ctx->cfg, batch), ctx->num_cu};
    return launch_gqa_decode_into(ctx, ws, stream, p, q_gate, k_new, v_new, in_dtype, k_cache, v_cache, positions,
                                  out, out_dtype, batch, max_ctx);
}

hipError_t launch_gqa_decode_into(qff_ctx* ctx, const GqaPartials& ws, hipStream_t stream,
                                  const qff_gqa_params* p, const void* q_gate, const void* k_new,
                                  const void* v_new, qff_dtype in_dtype, void* k_cache, void* v_cache,
                                  const int32_t* positions, void* out, qff_dtype out_dtype, int batch,
                                  int max_ctx) {
    const int cap = ws.cap;
    // the split is derived from the device positions inside the kernels; at
    // most target + batch chunks per kv head (rounding up adds at most one
    // per sequence), so the grid covers every chunk of any length mix
    const int target = gqa_target_chunks(ws.num_cu, batch);
    const int units = 2 * (target + batch);
    const RopeFreqs rf = rope_freqs(p->rope_theta);
    uint16_t* kc = static_cast<uint16_t*>(k_cache);
    uint16_t* vc = static_cast<uint16_t*>(v_cache);
    {
        ProfScope prof(ctx, stream, "gqa_decode_partial");
#define QFF_PART(I, F)                                                                                           \
    gqa_decode_partial_kernel<I, F><<<units, 64, 0, stream>>>(q_gate, k_new, v_new, p->q_norm_w, p->k_norm_w, rf, \
                                                             p->scale, p->eps, kc, vc, positions, batch, max_ctx, \
                                                             target, cap, ws.m, ws.d, ws.o)
        if (p->kv_f16) {
            if (in_dtype == QFF_BF16) QFF_PART(1, 1); else QFF_PART(0, 1);
        } else {
            if (in_dtype == QFF_BF16) QFF_PART(1, 0); else QFF_PART(0, 0);
        }
#undef QFF_PART
    }
    // small batches split each head's 256 dims over 4 workgroups
    const int ds = batch <= 8 ? 4 : 1;
    const dim3 cgrid(16 * ds, batch);
    ProfScope prof(ctx, stream, "gqa_decode_combine");
#define QFF_COMB(I, O)                                                                                      \
    if (ds == 4)                                                                                            \
        gqa_decode_combine_kernel<I, O, 4><<<cgrid, 512, 0, stream>>>(q_gate, positions, batch, max_ctx,   \
                                                                      target, cap, ws.m, ws.d, ws.o, out);  \
    else                                                                                                    \
        gqa_decode_combine_kernel<I, O, 1><<<cgrid, 512, 0, stream>>>(q_gate, positions, batch, max_ctx,   \
                                                                      target, cap, ws.m, ws.d, ws.o, out)
    if (in_dtype == QFF_BF16) {
        if (out_dtype == QFF_BF16) { QFF_COMB(1, 1); } else { QFF_COMB(1, 0); }
    } else {
        if (out_dtype == QFF_BF16) { QFF_COMB(0, 1); } else { QFF_COMB(0, 0); }
    }
#undef QFF_COMB
    return hipGetLastError();
}

}  // namespace qff
