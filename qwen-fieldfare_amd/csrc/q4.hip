// q4.hip -- MLX affine-Q4 (group 64) dequant and matmul on gfx950.
//
// Format (QwenQ4ActiveExpertStreamingRunner.swift:899-922,
// deltanet.metal:809-861): element c of row r is nibble c % 8 (lowest first)
// of uint32 word w[r * cols/8 + c/8]; W[r,c] = nibble * scale[r, c/64] +
// bias[r, c/64].
//
// Matmul: y[m, r] = sum_c W[r, c] x[m, c]. The reference accumulates the
// factored form scale * sum(q x) + bias * sum(x) per group on the vector
// units, one SIMD group per row (deltanet.metal:1838-1895). Here the group
// products run on the matrix cores: a nibble q becomes the exact bf16 value
// 128 + q by OR-ing it into the mantissa of 0x4300 (128.0), so an MFMA over
// those operands yields P = sum (128 + q) x, and
//   sum_c W x = s * P + (b - 128 s) * sum(x)       (per group, per row)
// with sum(x) over the same bf16-rounded x the MFMA saw. Two kernels:
// q4_gemv_kernel for decode batches (<= 32 tokens), streaming each weight row
// once with the K dimension split over a workgroup's waves, and
// q4_gemm_kernel for many tokens (prefill projections), tiled 128 x 128.
#include "common.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace qff {

// One uint32 word (8 nibbles) per thread -> 8 fp32 values.
template <int SB_DT>
__global__ __launch_bounds__(256) void q4_dequant_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         float* __restrict__ out, int rows, int cols) {
    const size_t words = static_cast<size_t>(rows) * (cols / 8);
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const int r = static_cast<int>(i / (cols / 8));
    const int c0 = static_cast<int>(i % (cols / 8)) * 8;
    const size_t gi = static_cast<size_t>(r) * (cols / 64) + c0 / 64;
    const float s = elem<SB_DT>::load(scales, gi);
    const float b = elem<SB_DT>::load(biases, gi);
    const uint32_t word = w[i];
    float v[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) v[n] = static_cast<float>((word >> (4 * n)) & 0xFu) * s + b;
    float4* o = reinterpret_cast<float4*>(out + static_cast<size_t>(r) * cols + c0);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

constexpr int kQ4MaxGroups = 64;  // cols <= 4096

// 8 nibbles -> bf16 128 + q in the k order (c0, c4, c1, c5, c2, c6, c3, c7):
// dword j = ((w >> 4j) & 0x000F000F) | 0x43004300, two instructions each.
__device__ __forceinline__ u32x4_t q4_to_bf16_interleaved(uint32_t w) {
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = ((w >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
    return r;
}

// 8 bf16 (x0 .. x7 in 4 dwords) -> (x0 x4, x1 x5, x2 x6, x3 x7)
__device__ __forceinline__ u32x4_t interleave8(u32x4_t v) {
    return u32x4_t{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                   __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
}

// ---- decode-shaped product (batch <= 32) ---------------------------------------
//
// One workgroup per 16 RT weight rows, cols/512 waves (at least one), each
// wave taking 8 of the row's 64-column groups. The workgroup first streams
// its rows' weight words into LDS with 16-B loads that cover whole rows
// (consecutive threads, consecutive bytes: full cache lines per
// instruction), together with the scales and folded biases; each lane has
// meanwhile issued the loads of its x values (16 per group and token tile).
// Per group: the lane reads its 8 B of each row tile from LDS, P = sum
// (128 + q) x on the matrix cores, the group sum of x from the same
// registers (plus two shuffles), acc += s P + (b - 128 s) sum(x) in fp32.
// The waves' partial sums meet in LDS. RT = 4 reads x a quarter as often
// per weight byte (several tokens over long matrices); RT = 1 gives the most
// workgroups (batch 1, short matrices).
constexpr int kQ4GemvMaxWaves = 16;

// Q4Parts: the parts of one launch (a single product is one part):
// workgroups blk0[p] .. blk0[p+1]-1 take part p's row blocks.
struct Q4Parts {
    const uint32_t* w[QFF_Q4_MAX_PARTS];
    const uint16_t* s[QFF_Q4_MAX_PARTS];
    const uint16_t* b[QFF_Q4_MAX_PARTS];
    void* y[QFF_Q4_MAX_PARTS];
    int rows[QFF_Q4_MAX_PARTS];
    int ybf16[QFF_Q4_MAX_PARTS];
    const void* res[QFF_Q4_MAX_PARTS];   // residual of y's dtype, or null
    int blk0[QFF_Q4_MAX_PARTS + 1];
    int n;
};

// The part of workgroup blk with its fields, read at kernel start in two
// scalar-memory round trips (the block boundaries, then the part's fields;
// selecting among all parts' fields read at once needs ~100 SGPRs and the
// compiler splits it into two batches anyway); the integer fields are
// pinned in registers: left to itself the compiler re-reads kernel
// arguments at a later use, and every such read is another round trip on
// the critical path of a launch that lasts a few microseconds.
struct Q4Part1 {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    void* y;
    const void* res;
    int rows, ybf16, blk0;
};
__device__ __forceinline__ Q4Part1 q4_part_of(const Q4Parts& parts, int blk) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < QFF_Q4_MAX_PARTS; ++i) p += blk >= parts.blk0[i];   // unused entries hold INT_MAX
    Q4Part1 r{parts.w[p], parts.s[p], parts.b[p], parts.y[p], parts.res[p], parts.rows[p], parts.ybf16[p], parts.blk0[p]};
    // (the pointers stay as read: through an asm operand they would lose
    // their global address space and every access would become a flat one)
    asm volatile("" : "+s"(r.rows), "+s"(r.ybf16), "+s"(r.blk0));
    return r;
}

// The residual of elements i .. i+3 of part p (0 without one), read early,
// when ok (i a multiple of 4, so the loads are aligned): one 8-B (bf16) and
// one 16-B (fp32) load. Both dtypes are loaded unconditionally, each from an
// in-bounds address (the part's weights stand in for the one not needed),
// and selected: a branch around a load would make the compiler wait for
// every load in flight at the join.
__device__ __forceinline__ f32x4_t q4_res4(const Q4Parts& parts, int p, size_t i, bool ok) {
    const bool has = ok && parts.res[p] != nullptr, bf = parts.ybf16[p] != 0;
    const u32x2_t* r16 = has && bf ? reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(parts.res[p]) + i)
                                   : reinterpret_cast<const u32x2_t*>(parts.w[p]);
    const u32x4_t* r32 = has && !bf ? reinterpret_cast<const u32x4_t*>(static_cast<const float*>(parts.res[p]) + i)
                                    : reinterpret_cast<const u32x4_t*>(parts.w[p]);
    const u32x2_t a = *r16;
    const u32x4_t b = *r32;
    const f32x4_t r = bf ? f32x4_t{__uint_as_float(a[0] << 16), __uint_as_float(a[0] & 0xffff0000u),
                                   __uint_as_float(a[1] << 16), __uint_as_float(a[1] & 0xffff0000u)}
                         : f32x4_t{__uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]),
                                   __uint_as_float(b[3])};
    return has ? r : f32x4_t{0.f, 0.f, 0.f, 0.f};
}
// y[i] of part p = v, in the part's output dtype
__device__ __forceinline__ void q4_put(const Q4Parts& parts, int p, size_t i, float v) {
    if (parts.ybf16[p]) elem<1>::store(parts.y[p], i, v);
    else elem<0>::store(parts.y[p], i, v);
}

// y[i] of part p = v (+ residual[i]), in the part's output dtype
__device__ __forceinline__ void q4_store(const Q4Parts& parts, int p, size_t i, float v) {
    const bool bf = parts.ybf16[p];
    if (parts.res[p]) v += bf ? elem<1>::load(parts.res[p], i) : elem<0>::load(parts.res[p], i);
    if (bf) elem<1>::store(parts.y[p], i, v);
    else elem<0>::store(parts.y[p], i, v);
}

// N consecutive RMSNorm weights from column c (N a multiple of 8, c of 8),
// f32 or bf16 without a branch on the dtype (a branch around loads makes the
// compiler wait for every load in flight at the join): per 8 weights two
// 16-B loads, the second a repeat of the first for bf16, and selects.
// The two halves: the raw 16-B pieces of 8 weights at column c, and their
// values (so callers can issue other loads before any of these is used).
struct Q4NormRaw {
    u32x4_t lo, hi;
};
__device__ __forceinline__ Q4NormRaw q4_norm_weights_raw(const Q4Norm& nrm, int c) {
    const bool bf = nrm.wbf16;
    const char* base = static_cast<const char*>(nrm.w) + static_cast<size_t>(c) * (bf ? 2 : 4);
    return Q4NormRaw{*reinterpret_cast<const u32x4_t*>(base), *reinterpret_cast<const u32x4_t*>(base + (bf ? 0 : 16))};
}
__device__ __forceinline__ void q4_norm_weights_finish(const Q4Norm& nrm, const Q4NormRaw& r, float* wn) {
    const bool bf = nrm.wbf16;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t f = e < 4 ? r.lo[e] : r.hi[e - 4];
        const uint32_t h = (e & 1) ? (r.lo[e >> 1] & 0xffff0000u) : (r.lo[e >> 1] << 16);
        wn[e] = __uint_as_float(bf ? h : f);
    }
}
template <int N>
__device__ __forceinline__ void q4_norm_weights(const Q4Norm& nrm, int c, float (&wn)[N]) {
#pragma unroll
    for (int q = 0; q < N / 8; ++q) q4_norm_weights_finish(nrm, q4_norm_weights_raw(nrm, c + 8 * q), wn + 8 * q);
}

// Groups per wave: 2 up to 2048 columns, 4 up to 4096 (at most 16 waves).
__host__ __device__ constexpr int q4_gemv_gpw(int cols) { return cols > 2048 ? 4 : 2; }
template <int GPW>
__host__ __device__ constexpr int q4_gemv_waves(int cols) { return (cols / 64 + GPW - 1) / GPW; }
__host__ __device__ constexpr int q4_lds_stride(int cols) { return cols / 8 + 8; }   // dwords per staged row

template <int RT, int NBT, int GPW>
__host__ __device__ constexpr int q4_gemv_lds_bytes(int cols) {
    return (16 * RT * q4_lds_stride(cols) * 4 + 16 * RT * (cols / 64) * 8) >
                   q4_gemv_waves<GPW>(cols) * RT * NBT * 64 * 16
               ? 16 * RT * q4_lds_stride(cols) * 4 + 16 * RT * (cols / 64) * 8
               : q4_gemv_waves<GPW>(cols) * RT * NBT * 64 * 16;
}

template <int SB_DT, int X_DT, int NBT, int RT, bool NORM, int GPW>
__global__ __launch_bounds__(64 * kQ4GemvMaxWaves) void q4_gemv_kernel(Q4Parts parts, const void* __restrict__ x,
                                                                       int cols, int batch, Q4Norm nrm) {
    constexpr int RW = 16 * RT;                     // rows per workgroup
    constexpr bool HILO = X_DT == 0 || NORM;        // x is not exactly bf16: hi + lo operands
    // per thread at most PPT weight pieces and SBT scale/bias entries:
    // RW * (cols / 32) / (64 nw) <= RW GPW / 32 with nw = ceil(G / GPW)
    constexpr int PPT = RW * GPW / 32, SBT = (RW * GPW + 63) / 64;
    const int G = cols / 64, W8 = cols / 8, S = q4_lds_stride(cols);
    const int nw = q4_gemv_waves<GPW>(cols), NT = 64 * nw;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    int p = 0;
#pragma unroll
    for (int i = 1; i < QFF_Q4_MAX_PARTS; ++i) p += (i < parts.n && static_cast<int>(blockIdx.x) >= parts.blk0[i]);
    const uint32_t* __restrict__ w = parts.w[p];
    const uint16_t* __restrict__ scales = parts.s[p];
    const uint16_t* __restrict__ biases = parts.b[p];
    const int rows = parts.rows[p];
    const int R0 = (blockIdx.x - parts.blk0[p]) * RW;

    // LDS: the rows' weight words [RW][S], then (s, b - 128 s) [RW][G]; after
    // the products the same bytes hold the waves' partial sums
    extern __shared__ __attribute__((aligned(16))) unsigned char q4lds[];
    uint32_t* wl = reinterpret_cast<uint32_t*>(q4lds);
    float2* sb = reinterpret_cast<float2*>(q4lds + RW * S * 4);
    f32x4_t* part = reinterpret_cast<f32x4_t*>(q4lds);

    // weight pieces (16 B): piece q -> row q / (W8/4), words 4 (q % (W8/4));
    // at most PPT per thread, clamped so every load is issued
    const int ppr = W8 / 4, npieces = RW * ppr;
    u32x4_t wp[PPT];
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int q = min(t + NT * i, npieces - 1);
        const int r = q / ppr, c4 = q - r * ppr;
        // weights stream through once a call: non-temporal loads (`nt`)
        wp[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(w + static_cast<size_t>(min(R0 + r, rows - 1)) * W8 + 4 * c4));
    }
    // scales/biases: at most SBT entries per thread
    float sreg[SBT], breg[SBT];
#pragma unroll
    for (int k = 0; k < SBT; ++k) {
        const int idx = min(t + NT * k, RW * G - 1);
        const size_t gi = static_cast<size_t>(min(R0 + idx / G, rows - 1)) * G + idx % G;
        sreg[k] = elem<SB_DT>::load(scales, gi);
        breg[k] = elem<SB_DT>::load(biases, gi);
    }
    // the weight and scale loads stay ahead of the x loads below, so the LDS
    // staging of the weights waits for them alone
    __builtin_amdgcn_sched_barrier(0);
    // the residuals of the outputs this wave stores at the end (its tile
    // wave of the RT x NBT output tiles, when it has one), requested now
    // (rows a multiple of 4 and a 16-B aligned residual, so each lane's four
    // rows are one aligned access; otherwise the store reads it itself)
    const bool res_ok = (rows & 3) == 0 && (reinterpret_cast<uintptr_t>(parts.res[p]) & 15) == 0;
    f32x4_t resv = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (RT * NBT <= kQ4GemvMaxWaves) {
        const int tile = min(wave, RT * NBT - 1), rt = tile / NBT, bt = tile % NBT;
        const int m = min(16 * bt + n, batch - 1), r = min(R0 + 16 * rt + 4 * kb, rows - 4);
        resv = q4_res4(parts, p, res_ok ? static_cast<size_t>(m) * rows + r : 0, res_ok);
    }
    // this lane's x (16 values per group and token tile): bf16 activations
    // for all GPW groups of its wave up front; fp32 ones (converted to bf16
    // as they arrive) group by group in the product loop. With NORM the
    // lane also sums the squares of its raw x over the row's groups and
    // takes bf16(x w_norm); the waves together cover the row, so their sums
    // meet in LDS and the row sums are scaled by each token's inverse RMS.
    const int g0 = wave * GPW, gn = min(GPW, G - g0);
    float ssq[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) ssq[bt] = 0.0f;
    // NORM: the norm weights go to LDS once per workgroup (fp32), staged
    // with the weights
    __shared__ __attribute__((aligned(16))) float wnl[NORM ? 64 * kQ4MaxGroups : 4];
    if (NORM) {
        for (int c8 = t; c8 < cols / 8; c8 += NT) {
            float w8[8];
            q4_norm_weights<8>(nrm, 8 * c8, w8);
            *reinterpret_cast<float4*>(&wnl[8 * c8]) = make_float4(w8[0], w8[1], w8[2], w8[3]);
            *reinterpret_cast<float4*>(&wnl[8 * c8 + 4]) = make_float4(w8[4], w8[5], w8[6], w8[7]);
        }
    }
    auto load_x = [&](int i, u32x4_t (&xo2)[NBT][2], u32x4_t (&xl2)[NBT][2]) {
        const int g = min(g0 + i, G - 1);
        float wn[16];
        if (NORM) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 f = *reinterpret_cast<const float4*>(&wnl[64 * g + 16 * kb + 4 * q]);
                wn[4 * q] = f.x;
                wn[4 * q + 1] = f.y;
                wn[4 * q + 2] = f.z;
                wn[4 * q + 3] = f.w;
            }
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            const size_t xo = static_cast<size_t>(min(16 * bt + n, batch - 1)) * cols + 64 * g + 16 * kb;
            if (NORM) {
                float v[16];
                if (X_DT == 1) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const u32x4_t u =
                            *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + xo + 8 * q);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[8 * q + 2 * e] = __uint_as_float(u[e] << 16);
                            v[8 * q + 2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
                        }
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 f = reinterpret_cast<const float4*>(static_cast<const float*>(x) + xo)[q];
                        v[4 * q] = f.x;
                        v[4 * q + 1] = f.y;
                        v[4 * q + 2] = f.z;
                        v[4 * q + 3] = f.w;
                    }
                }
                float s2 = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) s2 = fmaf(v[e], v[e], s2);
                ssq[bt] += i < gn ? s2 : 0.0f;
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        uint32_t hh, ll;
                        split_bf16x2(v[8 * q + 2 * e] * wn[8 * q + 2 * e], v[8 * q + 2 * e + 1] * wn[8 * q + 2 * e + 1],
                                     hh, ll);
                        xo2[bt][q][e] = hh;
                        xl2[bt][q][e] = ll;
                    }
            } else if (X_DT == 1) {
                xo2[bt][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + xo);
                xo2[bt][1] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + xo + 8);
            } else {
                const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(x) + xo);
                const float4 e0 = q[0], e1 = q[1], e2 = q[2], e3 = q[3];
                const float f[16] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w,
                                     e2.x, e2.y, e2.z, e2.w, e3.x, e3.y, e3.z, e3.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    uint32_t hh, ll;
                    split_bf16x2(f[2 * e], f[2 * e + 1], hh, ll);
                    xo2[bt][e >> 2][e & 3] = hh;
                    xl2[bt][e >> 2][e & 3] = ll;
                }
            }
        }
    };
    constexpr bool kPre = X_DT == 1 && !NORM;   // all of the wave's x up front
    constexpr int kXPre = kPre ? GPW : 1;
    u32x4_t xv[kXPre][NBT][2];
    if (kPre) {
        u32x4_t unused[NBT][2];
#pragma unroll
        for (int i = 0; i < kXPre; ++i) load_x(i, xv[i], unused);
    }
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int q = t + NT * i;
        if (q < npieces) {
            const int r = q / ppr, c4 = q - r * ppr;
            *reinterpret_cast<u32x4_t*>(wl + r * S + 4 * c4) = wp[i];
        }
    }
#pragma unroll
    for (int k = 0; k < SBT; ++k) {
        const int idx = t + NT * k;
        if (idx < RW * G) sb[idx] = make_float2(sreg[k], breg[k] - 128.0f * sreg[k]);
    }
    __syncthreads();
    // the preloaded x enters the computation only from here: work on it
    // placed above the barrier would make the barrier wait for the x loads
    if (kPre) {
#pragma unroll
        for (int i = 0; i < kXPre; ++i)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) asm volatile("" : "+v"(xv[i][bt][0]), "+v"(xv[i][bt][1]));
    }

    f32x4_t acc[RT][NBT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[rt][bt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // the wave's GPW groups unrolled (groups past the row end read group
    // G-1 and are masked), so the LDS reads, shuffles and MFMAs of different
    // groups overlap
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
        const int g = min(g0 + i, G - 1);
        const float keep = i < gn ? 1.0f : 0.0f;
        float xsum[NBT];
        u32x4_t xi[NBT][2], xil[NBT][2];
        u32x4_t (&xg)[NBT][2] = xv[kPre ? i : 0];
        u32x4_t xgl[NBT][2];
        if (!kPre) load_x(i, xg, xgl);
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            const u32x4_t x0 = xg[bt][0], x1 = xg[bt][1];
            float sx = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                sx += (__uint_as_float(x0[j] << 16) + __uint_as_float(x0[j] & 0xffff0000u)) +
                      (__uint_as_float(x1[j] << 16) + __uint_as_float(x1[j] & 0xffff0000u));
            if (HILO) {
                const u32x4_t l0 = xgl[bt][0], l1 = xgl[bt][1];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    sx += (__uint_as_float(l0[j] << 16) + __uint_as_float(l0[j] & 0xffff0000u)) +
                          (__uint_as_float(l1[j] << 16) + __uint_as_float(l1[j] & 0xffff0000u));
                xil[bt][0] = interleave8(l0);
                xil[bt][1] = interleave8(l1);
            }
            sx += __shfl_xor(sx, 16, 64);
            sx += __shfl_xor(sx, 32, 64);
            xsum[bt] = sx;
            xi[bt][0] = interleave8(x0);
            xi[bt][1] = interleave8(x1);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const u32x2_t wv = *reinterpret_cast<const u32x2_t*>(wl + (16 * rt + n) * S + 8 * g + 2 * kb);
            const u32x4_t a0 = q4_to_bf16_interleaved(wv[0]);
            const u32x4_t a1 = q4_to_bf16_interleaved(wv[1]);
            float2 svb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                svb[j] = sb[(16 * rt + 4 * kb + j) * G + g];
                svb[j].x *= keep;
                svb[j].y *= keep;
            }
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                f32x4_t P = f32x4_t{0.f, 0.f, 0.f, 0.f};
                P = mfma_16x16x32_bf16(a0, xi[bt][0], P);
                P = mfma_16x16x32_bf16(a1, xi[bt][1], P);
                if (HILO) {
                    P = mfma_16x16x32_bf16(a0, xil[bt][0], P);
                    P = mfma_16x16x32_bf16(a1, xil[bt][1], P);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[rt][bt][j] = fmaf(svb[j].x, P[j], fmaf(svb[j].y, xsum[bt], acc[rt][bt][j]));
            }
        }
    }
    // per-wave sums of squares of each token (the lanes of one n share a token)
    __shared__ float q4ss[NORM ? kQ4GemvMaxWaves * 32 : 1];
    if (NORM) {
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            float v = ssq[bt];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (kb == 0) q4ss[wave * 32 + 16 * bt + n] = v;
        }
    }
    __syncthreads();   // the staged weights are consumed; their bytes take the partial sums
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) part[(wave * RT * NBT + rt * NBT + bt) * 64 + lane] = acc[rt][bt];
    __syncthreads();
    for (int tile = wave; tile < RT * NBT; tile += nw) {
        const int rt = tile / NBT, bt = tile % NBT;
        f32x4_t v = part[tile * 64 + lane];
        for (int ww = 1; ww < nw; ++ww) v += part[(ww * RT * NBT + tile) * 64 + lane];
        const int m = 16 * bt + n;
        if (m < batch) {
            if (NORM) {
                float sq = 0.0f;
                for (int ww = 0; ww < nw; ++ww) sq += q4ss[ww * 32 + m];
                v *= rsqrtf(sq / static_cast<float>(cols) + nrm.eps);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = R0 + 16 * rt + 4 * kb + j;
                if (r < rows) {
                    const size_t i = static_cast<size_t>(m) * rows + r;
                    if (RT * NBT <= kQ4GemvMaxWaves && tile == wave && res_ok) q4_put(parts, p, i, v[j] + resv[j]);
                    else q4_store(parts, p, i, v[j]);
                }
            }
        }
    }
}

// ---- decode batches of 2-16 tokens, 4096 columns: split over 512-column slices
//
// The out-projection shape (2048 rows x 4096 columns, no norm) has too few
// rows for the decode-batch kernel above to amortise x: 128 workgroups of 16
// rows each read all 256 KB of fp32 x. Here one workgroup takes (64 rows,
// one 512-column slice): four waves of 16 rows, 32 KB of x, and the grid is
// tiles x 8 slices wide. The workgroup stages its slice of x once in LDS as
// bf16 operands (lane l of wave w takes word l of the slice for tokens w,
// w + 4, ..: hi, + lo when x is fp32, in the nibble conversion's pair order),
// the per-(group, token) sums of the staged values and the rows' (s, b - 128
// s). The weights go straight to registers: lane (row n, kb) loads the 16 B
// at words 4 kb .. 4 kb + 3 of each 128-column span (one access per row and
// 4 lanes), and one permlane32 swap of words 2, 3 between lanes kb and kb ^ 2
// leaves every lane two words of each of the span's two groups: with group
// parity h, lane kb holds words base(kb ^ 2h) + {0, 1} of the group,
// base(k) = 4 (k & 1) + 2 (k >> 1), and the B operand reads x for the same
// words, so each 16x16x32 MFMA stays inside one group and the group's scale
// applies to its result: y = sum_g s_g P_g + (b_g - 128 s_g) X_g as in the
// other paths. Each workgroup writes its (64 rows x 16 tokens) partial to the
// workspace; q4_sk_reduce_kernel, the next launch, adds each tile's partials
// in slice order and the residual and stores the rows. (Handing the partials
// to the tile's last workgroup inside one launch needs an agent-scope
// release per workgroup, which writes back the L2: measured 9x slower.
// Measured against the kernel above: 8.6-9.2 vs 10.1-12.3 us at 2048 x 4096,
// batch 4-16; the normed 2048-column in-projections ran slower split, 772
// small workgroups, and stay there.)
constexpr int kQ4SkCols = 512;     // columns per slice (8 groups)
constexpr int kQ4SkSplit = 8;      // slices per row (cols = 4096)
constexpr int kQ4SkRows = 64;      // rows per workgroup (four waves of 16)
constexpr int kQ4SkXStride = 17;   // LDS entries (16 B) per staged word: 16 tokens + 1 pad

__device__ __forceinline__ int q4_sk_word(int kb, int h, int s) {
    const int k = kb ^ (2 * h);
    return 4 * (k & 1) + 2 * (k >> 1) + s;
}

template <int SB_DT, int X_DT>
__global__ __launch_bounds__(256) void q4_gemv_sk_kernel(Q4Parts parts, const void* __restrict__ x, int batch,
                                                         float* __restrict__ wpart) {
    constexpr bool HILO = X_DT == 0;   // fp32 x: hi + lo operands
    constexpr int cols = kQ4SkCols * kQ4SkSplit, G = cols / 64, W8 = cols / 8;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int tile = static_cast<int>(blockIdx.x), split = static_cast<int>(blockIdx.y);
    const Q4Part1 P = q4_part_of(parts, tile);
    const int rows = P.rows;
    const int R0 = (tile - P.blk0) * kQ4SkRows;
    const int k0 = split * kQ4SkCols, gs = k0 / 64;

    __shared__ u32x4_t xh[64 * kQ4SkXStride];
    __shared__ u32x4_t xlo[HILO ? 64 * kQ4SkXStride : 1];
    __shared__ float xsum[8][16];
    __shared__ float2 sbl[kQ4SkRows * 8];

    // ---- requests: this wave's weight rows, the slice's x, the workgroup's
    // scales and biases; nothing is used before all are issued
    const size_t wrow = static_cast<size_t>(min(R0 + 16 * wave + n, rows - 1));
    u32x4_t wq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        wq[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(P.w + wrow * W8 + k0 / 8 + 16 * j + 4 * kb));
    // x: token 4 i + wave, columns k0 + 8 lane .. +7
    u32x4_t xr[4][HILO ? 2 : 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t xo = static_cast<size_t>(min(4 * i + wave, batch - 1)) * cols + k0 + 8 * lane;
        if (HILO) {
            xr[i][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(x) + xo);
            xr[i][HILO ? 1 : 0] = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(x) + xo + 4);
        } else {
            xr[i][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + xo);
        }
    }
    float sreg[2], breg[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int e = t + 256 * j, r = e >> 3, g = e & 7;
        const size_t gi = static_cast<size_t>(min(R0 + r, rows - 1)) * G + gs + g;
        sreg[j] = elem<SB_DT>::load(P.s, gi);
        breg[j] = elem<SB_DT>::load(P.b, gi);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x operands and group sums into LDS
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * i + wave;
        u32x4_t hv, lv;
        float sum = 0.0f;
        if (HILO) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t hh, ll;
                split_bf16x2(__uint_as_float(xr[i][0][e]), __uint_as_float(xr[i][HILO ? 1 : 0][e]), hh, ll);
                hv[e] = hh;
                lv[e] = ll;
                sum += (__uint_as_float(hh << 16) + __uint_as_float(ll << 16)) +
                       (__uint_as_float(hh & 0xffff0000u) + __uint_as_float(ll & 0xffff0000u));
            }
        } else {
            hv = interleave8(xr[i][0]);   // exact bf16 x, reordered to the pair order
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += __uint_as_float(hv[e] << 16) + __uint_as_float(hv[e] & 0xffff0000u);
        }
        xh[lane * kQ4SkXStride + m] = hv;
        if (HILO) xlo[lane * kQ4SkXStride + m] = lv;
        sum = group_sum<8>(sum);   // the 8 words of group lane / 8
        if ((lane & 7) == 0) xsum[lane >> 3][m] = sum;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) sbl[t + 256 * j] = make_float2(sreg[j], breg[j] - 128.0f * sreg[j]);
    __syncthreads();

    // ---- products: per 128-column span j, words 2, 3 swap with lane ^ 32
    const bool b5 = lane & 32;
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto s2 = __builtin_amdgcn_permlane32_swap(wq[j][2], wq[j][2], false, false);
        const auto s3 = __builtin_amdgcn_permlane32_swap(wq[j][3], wq[j][3], false, false);
        const uint32_t p2 = b5 ? s2[0] : s2[1], p3 = b5 ? s3[0] : s3[1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int g = 2 * j + h;
            const bool own = (kb < 2) == (h == 0);
            const uint32_t w0 = own ? wq[j][0] : p2, w1 = own ? wq[j][1] : p3;
            const int e0 = (8 * g + q4_sk_word(kb, h, 0)) * kQ4SkXStride + n;
            const int e1 = (8 * g + q4_sk_word(kb, h, 1)) * kQ4SkXStride + n;
            const u32x4_t a0 = q4_to_bf16_interleaved(w0), a1 = q4_to_bf16_interleaved(w1);
            f32x4_t pr = f32x4_t{0.f, 0.f, 0.f, 0.f};
            pr = mfma_16x16x32_bf16(a0, xh[e0], pr);
            pr = mfma_16x16x32_bf16(a1, xh[e1], pr);
            if (HILO) {
                pr = mfma_16x16x32_bf16(a0, xlo[e0], pr);
                pr = mfma_16x16x32_bf16(a1, xlo[e1], pr);
            }
            const float xs = xsum[g][n];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 sb = sbl[(16 * wave + 4 * kb + i) * 8 + g];
                acc[i] = fmaf(sb.x, pr[i], fmaf(sb.y, xs, acc[i]));
            }
        }
    }
    // this slice's partial: rows 16 wave + 4 kb .. +3 of token n
    const size_t slot = static_cast<size_t>(tile) * kQ4SkSplit + split;
    *reinterpret_cast<f32x4_t*>(wpart + slot * 16 * kQ4SkRows + n * kQ4SkRows + 16 * wave + 4 * kb) = acc;
}

// One workgroup per row tile: thread t -> token t % 16, rows 4 (t / 16) .. +3
// of the tile, the slices' partials and the residuals requested at once, the
// partials added in slice order.
__global__ __launch_bounds__(256) void q4_sk_reduce_kernel(Q4Parts parts, int batch, const float* __restrict__ wpart) {
    const int t = threadIdx.x, tile = static_cast<int>(blockIdx.x);
    const Q4Part1 P = q4_part_of(parts, tile);
    const int rows = P.rows, R0 = (tile - P.blk0) * kQ4SkRows;
    const int m = t & 15, r4 = 4 * (t >> 4);
    f32x4_t pv[kQ4SkSplit];
#pragma unroll
    for (int sp = 0; sp < kQ4SkSplit; ++sp)
        pv[sp] = *reinterpret_cast<const f32x4_t*>(wpart + (static_cast<size_t>(tile) * kQ4SkSplit + sp) * 16 *
                                                               kQ4SkRows + m * kQ4SkRows + r4);
    const size_t o0 = static_cast<size_t>(min(m, batch - 1)) * rows;
    const bool has_res = P.res != nullptr, ybf = P.ybf16 != 0;
    uint32_t rh[4], rf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t oi = o0 + min(R0 + r4 + i, rows - 1);
        rh[i] = *(has_res && ybf ? static_cast<const uint16_t*>(P.res) + oi : reinterpret_cast<const uint16_t*>(P.w));
        rf[i] = *(has_res && !ybf ? static_cast<const uint32_t*>(P.res) + oi : P.w);
    }
    f32x4_t y = pv[0];
#pragma unroll
    for (int sp = 1; sp < kQ4SkSplit; ++sp) y += pv[sp];
    if (m >= batch) return;
    uint32_t mask = has_res ? ~0u : 0u;   // opaque: no branch around the residual loads
    asm volatile("" : "+v"(mask));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = R0 + r4 + i;
        if (r < rows) {
            const float v = y[i] + __uint_as_float((ybf ? rh[i] << 16 : rf[i]) & mask);
            if (ybf) elem<1>::store(P.y, o0 + r, v);
            else elem<0>::store(P.y, o0 + r, v);
        }
    }
}

// ---- single-token product on the vector units ---------------------------------
//
// Batch 1 is latency bound, so this path streams the weights straight into
// registers (no LDS staging of weights): a wave takes kQ4VecRows whole rows,
// one 16-B load per lane per 2048 columns (lane l takes the 32-column piece
// l of each 2048), all rows' loads in flight from the first instruction.
// Meanwhile the workgroup prepares x once for its four waves: each thread
// converts 8 columns to bf16 (with NORM: x w_norm, plus its share of sum
// x^2), stores them in LDS in the pair order of the nibble conversion
// below, and the 32-column piece sums; one barrier. Values that are not
// exactly bf16 (fp32 x, and every normed x) go in as a bf16 hi + lo pair
// with x = hi + lo to ~2^-16, each taken by its own dot2 pass over the same
// nibbles, and the piece sums add hi + lo, so the product keeps fp32-class
// activations as the reference's fp32 row kernels do (deltanet.metal
// :1838-1895). Products run on the
// vector units: the nibbles of a word become four bf16 pairs 128 + q with
// one shift and one and-or each (pair h = columns h and h + 4 of the word),
// and v_dot2_f32_bf16 takes a pair of them against the matching pair of x,
// so per group and row sum_c W x = s P + (b - 128 s) X over the lane's half
// group (P = sum (128 + q) x, X = sum x). The row sums meet in a
// reduce-scatter over the wave (6 shuffles); with NORM they are scaled by
// the token's inverse RMS.
constexpr int kQ4VecRows = 4;      // rows per wave
constexpr int kQ4VecWaves = 4;     // waves per workgroup

typedef __bf16 q4_bf16x2_t __attribute__((ext_vector_type(2)));

// c + a.lo b.lo + a.hi b.hi (bf16 pairs), v_dot2_f32_bf16
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(q4_bf16x2_t, a), __builtin_bit_cast(q4_bf16x2_t, b),
                                           c, false);
}

template <int SB_DT, int X_DT, int KW, bool NORM>
__global__ __launch_bounds__(64 * kQ4VecWaves) void q4_gemv1_kernel(Q4Parts parts, const void* __restrict__ x,
                                                                    int cols, Q4Norm nrm) {
    constexpr bool HILO = X_DT == 0 || NORM;   // x is not exactly bf16: hi + lo
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const Q4Part1 P = q4_part_of(parts, static_cast<int>(blockIdx.x));
    const uint32_t* __restrict__ w = P.w;
    const uint16_t* __restrict__ scales = P.s;
    const uint16_t* __restrict__ biases = P.b;
    const int rows = P.rows;
    const int R0 = ((static_cast<int>(blockIdx.x) - P.blk0) * kQ4VecWaves + wave) * kQ4VecRows;
    const int G = cols / 64, W8 = cols / 8, npc = cols / 32;   // 32-column pieces per row

    // Every load of the workgroup is issued before any loaded value is used:
    // x (and the norm weights) first, the residual, then the weight rows, so
    // the preparation of x below waits for its own loads only while the
    // weight rows are still arriving. Slice i = columns 8i .. 8i+7 of x.
    constexpr int NS = KW * 256 / (64 * kQ4VecWaves);   // slices per thread
    u32x4_t xr[NS][2];
    Q4NormRaw nr[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int ic = min(t + 64 * kQ4VecWaves * k, W8 - 1);
        if (X_DT == 1) {
            xr[k][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + 8 * ic);
        } else {
            const u32x4_t* f = reinterpret_cast<const u32x4_t*>(static_cast<const float*>(x) + 8 * ic);
            xr[k][0] = f[0];
            xr[k][1] = f[1];
        }
        if (NORM) nr[k] = q4_norm_weights_raw(nrm, 8 * ic);
    }
    // the residual of the row this lane stores at the end (lanes
    // 64 j / kQ4VecRows store row R0 + j)
    const size_t ri = static_cast<size_t>(min(R0 + lane / (64 / kQ4VecRows), rows - 1));
    const bool has_res = P.res != nullptr, ybf = P.ybf16 != 0;
    const uint32_t rh = *(has_res && ybf ? static_cast<const uint16_t*>(P.res) + ri : reinterpret_cast<const uint16_t*>(w));
    const uint32_t rf = *(has_res && !ybf ? static_cast<const uint32_t*>(P.res) + ri : w);
    // weights and group constants of this wave's rows
    u32x4_t wq[kQ4VecRows][KW];
    float sv[kQ4VecRows][KW], bv[kQ4VecRows][KW];
#pragma unroll
    for (int r = 0; r < kQ4VecRows; ++r) {
        const size_t row = static_cast<size_t>(min(R0 + r, rows - 1));
#pragma unroll
        for (int k = 0; k < KW; ++k) {
            const int pc = min(lane + 64 * k, npc - 1);
            wq[r][k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(w + row * W8 + 4 * pc));   // read once: `nt`
            sv[r][k] = elem<SB_DT>::load(scales, row * G + pc / 2);
            bv[r][k] = elem<SB_DT>::load(biases, row * G + pc / 2);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    float v[NS][8], wn[NS][8];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        if (X_DT == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[k][2 * e] = __uint_as_float(xr[k][0][e] << 16);
                v[k][2 * e + 1] = __uint_as_float(xr[k][0][e] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[k][e] = __uint_as_float(xr[k][0][e]);
                v[k][4 + e] = __uint_as_float(xr[k][1][e]);
            }
        }
        if (NORM) q4_norm_weights_finish(nrm, nr[k], wn[k]);
    }

    // x once per workgroup: slice i -> xl[i] as the four bf16 pairs
    // (x0 x4, x1 x5, x2 x6, x3 x7); xsl[i / 4] = its 32-column piece's sum
    __shared__ u32x4_t xl[64 * KW * 4];
    __shared__ u32x4_t xll[HILO ? 64 * KW * 4 : 1];
    __shared__ float xsl[64 * KW];
    __shared__ float ssl[kQ4VecWaves];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int i = t + 64 * kQ4VecWaves * k;
        const bool live = i < W8;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = live ? v[k][e] : 0.0f;
        if (NORM) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                ss = fmaf(v[k][e], v[k][e], ss);
                v[k][e] *= wn[k][e];
            }
        }
        u32x4_t xb, xlb;
        float sum = 0.0f;
        if (HILO) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t hh, ll;
                split_bf16x2(v[k][e], v[k][e + 4], hh, ll);
                xb[e] = hh;
                xlb[e] = ll;
                sum += (__uint_as_float(hh << 16) + __uint_as_float(ll << 16)) +
                       (__uint_as_float(hh & 0xffff0000u) + __uint_as_float(ll & 0xffff0000u));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) xb[e] = pack_bf16x2(v[k][e], v[k][e + 4]);   // exact: bf16 x, no norm
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += __uint_as_float(xb[e] << 16) + __uint_as_float(xb[e] & 0xffff0000u);
        }
        sum = group_sum<4>(sum);
        if (live) {
            xl[i] = xb;
            if (HILO) xll[i] = xlb;
            if ((i & 3) == 0) xsl[i >> 2] = sum;
        }
    }
    if (NORM) {
        ss = group_sum<64>(ss);
        if (lane == 0) ssl[wave] = ss;
    }
    __syncthreads();

    float part[kQ4VecRows];
#pragma unroll
    for (int r = 0; r < kQ4VecRows; ++r) part[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
        const int pc = lane + 64 * k;
        const bool live = pc < npc;
        const int pcc = min(pc, npc - 1);
        u32x4_t xv[4], xw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[j] = xl[4 * pcc + j];
            if (HILO) xw[j] = xll[4 * pcc + j];
        }
        const float xs = live ? xsl[pcc] : 0.0f;
#pragma unroll
        for (int r = 0; r < kQ4VecRows; ++r) {
            float dq = 0.0f, dl = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t wd = wq[r][k][j];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t wp = ((wd >> (4 * h)) & 0x000F000Fu) | 0x43004300u;
                    dq = dot2_bf16(wp, xv[j][h], dq);
                    if (HILO) dl = dot2_bf16(wp, xw[j][h], dl);
                }
            }
            if (HILO) dq += dl;
            // pieces past the row end (cols < 2048) hold a copy: weight zero
            const float sk = live ? sv[r][k] : 0.0f, bk = live ? bv[r][k] : 0.0f;
            part[r] = fmaf(sk, dq, fmaf(fmaf(-128.0f, sk, bk), xs, part[r]));
        }
    }
    // reduce-scatter over the wave: with four rows the 32-lane halves swap
    // (permlane32) and lane ^ 16 (swizzle) halve them, with two rows the
    // swap alone; then the 16-lane groups sum on DPP moves. Lane
    // 64 j / kQ4VecRows ends with row j.
    const bool b5 = lane & 32, b4 = lane & 16;
    auto other_half = [&](float v) {
        const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(b5 ? h[0] : h[1]);
    };
    float q1;
    if (kQ4VecRows == 4) {
        float q2[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) q2[j] = (b5 ? part[2 + j] : part[j]) + other_half(b5 ? part[j] : part[2 + j]);
        q1 = (b4 ? q2[1] : q2[0]) + swizzle_xor16(b4 ? q2[0] : q2[1]);
    } else if (kQ4VecRows == 2) {
        q1 = (b5 ? part[kQ4VecRows - 1] : part[0]) + other_half(b5 ? part[0] : part[kQ4VecRows - 1]);
        q1 += swizzle_xor16(q1);
    } else {
        q1 = part[0] + other_half(part[0]);
        q1 += swizzle_xor16(q1);
    }
    q1 = group_sum<16>(q1);
    if (NORM) {
        float sq = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kQ4VecWaves; ++ww) sq += ssl[ww];
        q1 *= rsqrtf(sq / static_cast<float>(cols) + nrm.eps);
    }
    if ((lane & (64 / kQ4VecRows - 1)) == 0) {
        const int r = R0 + lane / (64 / kQ4VecRows);
        uint32_t mask = has_res ? ~0u : 0u;   // opaque: no branch around the residual loads
        asm volatile("" : "+v"(mask));
        const float y = q1 + __uint_as_float((ybf ? rh << 16 : rf) & mask);
        if (r < rows) {
            if (ybf) elem<1>::store(P.y, r, y);
            else elem<0>::store(P.y, r, y);
        }
    }
}

// ---- many-token GEMM (prefill projections) -----------------------------------
//
// y[m, r] = sum_c W[r, c] x[m, c] for batch >= kQ4GemmMinBatch, on fp16 matrix
// cores with fp32 accumulation:
//   W16[r, c] = fp16(2^8 (s q + b))     one fused fp16 FMA per element,
//                                      rounded once from the exact value
//   x16[m, c] = fp16(x'[m, c] 2^-e_m)  x' = x (or x w_norm), e_m the token's
//                                      binary exponent that puts max |x'| in
//                                      [2^13, 2^14)
//   y[m, r]   = f_m sum_c W16 x16,     f_m = 2^(e_m - 8) (times the token's
//                                      inverse RMS with the norm)
// The power-of-two shifts are exact and keep both operands inside fp16's
// normal range: x' of any fp32 magnitude down to 2^-141 (the shift is at
// most 2^127), W of magnitude 2^-22 .. 255. Both
// operands carry 11 significant bits (the bf16 activations of the factored
// form carried 8), so the product is the fp32 dot product to a few 2^-12
// relative; the bias is part of every W16 element, so no group sums are
// needed and the accumulators stay in the matrix cores for the whole K loop.
//
// q4_x16_kernel forms x16 and f_m (one wave per token). q4_gemm_kernel: one
// workgroup per 256 rows x 128 tokens, four waves of 64 rows x 128 tokens
// (2 x 4 tiles of 32x32x16 fp16 MFMAs, C rows = weight rows so each lane's
// four consecutive outputs are adjacent in y; a 32x32x16 MFMA runs long
// enough that the wave's next LDS operand reads issue under it). A wave loads
// its own rows' nibbles straight into registers (16 B per lane and row tile
// per group: it alone uses them) and converts them there; the token tile's
// x16 group goes through LDS, double-buffered, one barrier per group, loaded
// straight from global memory into LDS. The packed fp16 (256 s, 256 b) of
// the tile's rows sit in LDS for the whole K loop.
//
// Within each 8-column word the matrix-core k order is (c0, c4, c1, c5, c2,
// c6, c3, c7): dword j of the converted word is then the fp16 pair
// ((w >> 4j) & 0x000F000F) | 0x64006400 = (1024 + q_j, 1024 + q_j+4), exact,
// minus 1024 (exact), then the FMA; x16 is stored in the same order. The
// lanes of half h (k slots 8h .. 8h + 7) of a 16-deep MFMA step ks take word
// 4h + ks of the group, so a lane's four words of a group are one 16-byte
// load, and the x16 piece 4h + ks.
constexpr int kQ4GemmRows = 256;   // weight rows per workgroup
constexpr int kQ4GemmToks = 128;   // tokens per workgroup

// x16 and f_m of one token per wave: lane l holds 8-column blocks l, l + 64, ...
template <int X_DT, bool NORM>
__global__ __launch_bounds__(256) void q4_x16_kernel(const void* __restrict__ x, uint16_t* __restrict__ x16,
                                                     float* __restrict__ fm, int cols, int batch, Q4Norm nrm) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= batch) return;
    const int nb = cols / 8;
    constexpr int kMaxB = 4096 / 8 / 64;
    float v[kMaxB][8];
    float ss = 0.0f, mx = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxB; ++i) {
        const int b = lane + 64 * i;
        if (b < nb) {
            const size_t o = static_cast<size_t>(m) * cols + 8 * b;
            if (X_DT == 1) {
                const u32x4_t u = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + o);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[i][2 * j] = __uint_as_float(u[j] << 16);
                    v[i][2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
                }
            } else {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + o);
                const float4 a = p[0], c = p[1];
                v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
                v[i][4] = c.x; v[i][5] = c.y; v[i][6] = c.z; v[i][7] = c.w;
            }
            if (NORM) {
                float wn[8];
                q4_norm_weights<8>(nrm, 8 * b, wn);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    ss = fmaf(v[i][e], v[i][e], ss);
                    v[i][e] *= wn[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[i][e]));
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    // max |x'| in [2^(E-1), 2^E): x' 2^-(E-14) stays below 2^14. e >= -127
    // keeps 2^-e a finite fp32 for the smallest tokens (fp32 subnormals
    // included): their x16 then sits below 2^14 but stays in fp16's normal
    // range down to |x'| = 2^-141, and f_m >= 2^-135 keeps 14 bits.
    const int e = mx > 0.0f ? max(__builtin_amdgcn_frexp_expf(mx) - 14, -127) : 0;
    const float p = ldexpf(1.0f, -e);
#pragma unroll
    for (int i = 0; i < kMaxB; ++i) {
        const int b = lane + 64 * i;
        if (b < nb) {
            const u32x4_t h{pack_f16x2(v[i][0] * p, v[i][4] * p), pack_f16x2(v[i][1] * p, v[i][5] * p),
                            pack_f16x2(v[i][2] * p, v[i][6] * p), pack_f16x2(v[i][3] * p, v[i][7] * p)};
            *reinterpret_cast<u32x4_t*>(x16 + static_cast<size_t>(m) * cols + 8 * b) = h;
        }
    }
    if (NORM) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    }
    if (lane == 0) {
        const float rs = NORM ? rsqrtf(ss / static_cast<float>(cols) + nrm.eps) : 1.0f;
        fm[m] = ldexpf(rs, e - 8);
    }
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// One nibble word -> four fp16 pairs 256 (s q + b) in the k order above;
// sb = packed fp16 (256 s, 256 b); e1024 = 0x64006400 held in a VGPR, so the
// extraction of each pair is one v_and_or_b32 (its other constant the one
// scalar operand a VOP3 instruction may read) after the shift.
__device__ __forceinline__ u32x4_t q4_to_f16_scaled(uint32_t w, uint32_t sb, uint32_t e1024) {
    const f16x2_t sbv = __builtin_bit_cast(f16x2_t, sb);
    const f16x2_t s2 = {sbv[0], sbv[0]}, b2 = {sbv[1], sbv[1]};
    const f16x2_t k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t e;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(e) : "v"(w >> (4 * j)), "s"(0x000F000Fu), "v"(e1024));
        const f16x2_t q = __builtin_bit_cast(f16x2_t, e) - k1024;
        r[j] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s2, b2));
    }
    return r;
}

template <int SB_DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void q4_gemm_kernel(
    Q4Parts parts, const uint16_t* __restrict__ x16, const float* __restrict__ fm, int cols, int batch) {
    // the part of this workgroup's row tile (parts' tiles are consecutive in x)
    int pp = 0;
    while (pp + 1 < parts.n && static_cast<int>(blockIdx.x) >= parts.blk0[pp + 1]) ++pp;
    const uint32_t* __restrict__ w = parts.w[pp];
    const uint16_t* __restrict__ scales = parts.s[pp];
    const uint16_t* __restrict__ biases = parts.b[pp];
    void* __restrict__ y = parts.y[pp];
    const void* __restrict__ res = parts.res[pp];
    const int rows = parts.rows[pp];
    const bool ybf = parts.ybf16[pp];
    const int G = cols / 64;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int R0 = (blockIdx.x - parts.blk0[pp]) * kQ4GemmRows, M0 = blockIdx.y * kQ4GemmToks;

    __shared__ __attribute__((aligned(16))) uint16_t Xl[2][kQ4GemmToks * 64];
    extern __shared__ __attribute__((aligned(16))) uint32_t sbl[];   // [G][256] packed fp16 (256 s, 256 b)

    for (int idx = t; idx < kQ4GemmRows * G; idx += 256) {
        const int r = idx / G, g = idx % G;
        const size_t gi = static_cast<size_t>(min(R0 + r, rows - 1)) * G + g;
        sbl[g * kQ4GemmRows + r] = pack_f16x2(256.0f * elem<SB_DT>::load(scales, gi), 256.0f * elem<SB_DT>::load(biases, gi));
    }

    // x16 staging straight from global memory into LDS: wave w's load i fills
    // tokens 8 (4w + i) .. +7 of the [128][64] tile, lane l the 16-byte
    // piece l & 7 of token l >> 3, which holds the token's 8-column block
    // (l & 7) ^ ((token >> 1) & 7) of the group (the swizzle spreads the 32
    // rows of an operand read over the bank groups)
    const uint16_t* xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int tok = 8 * (4 * wave + i) + (lane >> 3);
        xsrc[i] = x16 + static_cast<size_t>(min(M0 + tok, batch - 1)) * cols + 8 * ((lane & 7) ^ ((tok >> 1) & 7));
    }
    // weight words: lane -> rows 64 wave + 32 rt + r, words 4h .. 4h + 3 of each group
    // (rows past the part's end read its last row; their outputs are not stored)
    const int r = lane & 31, h = lane >> 5;
    const int wrow = R0 + 64 * wave + r;
    const uint32_t* wsrc = w + static_cast<size_t>(min(wrow, rows - 1)) * (cols / 8) + 4 * h;
    const int wstep1 = (min(wrow + 32, rows - 1) - min(wrow, rows - 1)) * (cols / 8);   // row tile 1's word offset

    u32x4_t wa[2][2];
    auto stage_x = [&](int buf, int g) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(xsrc[i] + 64 * g),
                                             (__attribute__((address_space(3))) void*)&Xl[buf][8 * (4 * wave + i) * 64],
                                             16, 0, 0);
    };
    auto fetch_w = [&](u32x4_t (&dst)[2], int g) {
        dst[0] = *reinterpret_cast<const u32x4_t*>(wsrc + 8 * g);
        dst[1] = *reinterpret_cast<const u32x4_t*>(wsrc + wstep1 + 8 * g);
    };

    f32x16_t acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    // group g: x16 in LDS buffer g & 1, its weight words in wa[s]; on the
    // way, group g + 1's x16 is requested into the other buffer and its
    // weight words into wa[s ^ 1] (clamped, so every load is unconditional)
    uint32_t e1024 = 0x64006400u;
    asm volatile("" : "+v"(e1024));   // kept in a VGPR
    auto step = [&](int s, int g) {
        // (the two unrolled steps are kept apart: interleaved by the
        // scheduler they would not fit the registers)
        __builtin_amdgcn_sched_barrier(0);
        // every wave's pieces of group g have landed, and every wave is done
        // with group g - 1's buffer
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        stage_x((g + 1) & 1, min(g + 1, G - 1));
        const u32x4_t (&cur)[2] = wa[s];
        fetch_w(wa[s ^ 1], min(g + 1, G - 1));
        // the loads stay at the top of the step, a whole group's work ahead
        // of their use (the scheduler would sink them next to it)
        __builtin_amdgcn_sched_barrier(0);
        uint32_t sb[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) sb[rt] = sbl[g * kQ4GemmRows + 64 * wave + 32 * rt + r];
        // B operand of token tile mt, step ks: token 32 mt + r, x16 piece
        // 4h + ks (swizzled by (token / 2) % 8, so the 32 rows of a read
        // meet every bank group twice)
        const uint16_t* xb = &Xl[g & 1][r * 64];
        const int sw = (r >> 1) & 7;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4_t A[2], B[4];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) A[rt] = q4_to_f16_scaled(cur[rt][ks], sb[rt], e1024);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                B[mt] = *reinterpret_cast<const u32x4_t*>(xb + 32 * mt * 64 + 8 * ((4 * h + ks) ^ sw));
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc[rt][mt] = mfma_32x32x16_f16(A[rt], B[mt], acc[rt][mt]);
        }
    };
    stage_x(0, 0);
    fetch_w(wa[0], 0);
    int g = 0;
    for (; g + 1 < G; g += 2) {
        step(0, g);
        step(1, g + 1);
    }
    if (g < G) step(0, g);

    // lane: token 32 mt + r, rows 64 wave + 32 rt + 8 j + 4 h .. +3 (adjacent in y)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int m = M0 + 32 * mt + r;
        if (m >= batch) continue;
        const float f = fm[m];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rr = R0 + 64 * wave + 32 * rt + 8 * j + 4 * h;
                const size_t o = static_cast<size_t>(m) * rows + rr;
                f32x4_t v = f32x4_t{acc[rt][mt][4 * j], acc[rt][mt][4 * j + 1], acc[rt][mt][4 * j + 2],
                                    acc[rt][mt][4 * j + 3]};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] *= f;
                    if (res && rr + i < rows) v[i] += ybf ? elem<1>::load(res, o + i) : elem<0>::load(res, o + i);
                }
                if (rr + 3 < rows && (rows & 3) == 0) {
                    if (ybf)
                        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(y) + o) =
                            u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    else
                        *reinterpret_cast<f32x4_t*>(static_cast<float*>(y) + o) = v;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (rr + i >= rows) continue;
                        if (ybf) elem<1>::store(y, o + i, v[i]);
                        else elem<0>::store(y, o + i, v[i]);
                    }
                }
            }
    }
}

hipError_t launch_q4_dequant(hipStream_t stream, const uint32_t* w, const void* scales,
                             const void* biases, qff_dtype sb_dtype, float* out, int rows, int cols) {
    const size_t words = static_cast<size_t>(rows) * (cols / 8);
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    const uint16_t* s = static_cast<const uint16_t*>(scales);
    const uint16_t* b = static_cast<const uint16_t*>(biases);
    if (sb_dtype == QFF_BF16) q4_dequant_kernel<1><<<blocks, 256, 0, stream>>>(w, s, b, out, rows, cols);
    else q4_dequant_kernel<2><<<blocks, 256, 0, stream>>>(w, s, b, out, rows, cols);
    return hipGetLastError();
}

// Dynamic LDS past 64 KB needs the kernel's attribute raised (once per
// kernel instantiation and size).
template <auto Kernel>
static hipError_t q4_allow_lds(int bytes) {
    if (bytes <= 65536) return hipSuccess;
    static int raised = 0;   // largest size set so far for this kernel
    if (bytes <= raised) return hipSuccess;
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) raised = bytes;
    return e;
}

#define QFF_CHECK_HIP_RET(x)            \
    do {                                \
        const hipError_t e_ = (x);      \
        if (e_ != hipSuccess) return e_; \
    } while (0)

// The parts laid end to end, rpb rows per workgroup.
static Q4Parts q4_pack_parts(const qff_q4_part* parts, int nparts, int rpb, int& blocks) {
    Q4Parts P{};
    blocks = 0;
    for (int i = 0; i < nparts; ++i) {
        P.w[i] = parts[i].w;
        P.s[i] = static_cast<const uint16_t*>(parts[i].scales);
        P.b[i] = static_cast<const uint16_t*>(parts[i].biases);
        P.y[i] = parts[i].y;
        P.res[i] = parts[i].residual;
        P.rows[i] = parts[i].rows;
        P.ybf16[i] = parts[i].y_dtype == QFF_BF16;
        P.blk0[i] = blocks;
        blocks += (parts[i].rows + rpb - 1) / rpb;
    }
    P.blk0[nparts] = blocks;
    for (int i = nparts + 1; i <= QFF_Q4_MAX_PARTS; ++i) P.blk0[i] = INT_MAX;   // past the last part
    P.n = nparts;
    return P;
}

// Many tokens: x16 and the per-token factors once per token slice, then one
// tiled launch over all parts (the small parts' tiles fill the chip beside the
// large one's).
template <bool NORM>
static hipError_t q4_gemm_parts(qff_ctx* ctx, hipStream_t stream, const qff_q4_part* parts, int nparts,
                                qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, const Q4Norm& norm,
                                int cols, int batch) {
    const int G = cols / 64;
    const int lds = G * kQ4GemmRows * 4;   // packed (s, b) of the row tile
    QFF_CHECK_HIP_RET((q4_allow_lds<q4_gemm_kernel<1>>(lds)));
    QFF_CHECK_HIP_RET((q4_allow_lds<q4_gemm_kernel<2>>(lds)));
    for (int m0 = 0; m0 < batch; m0 += ctx->q4_xs_tokens) {
        const int mb = min(ctx->q4_xs_tokens, batch - m0);
        const void* xm = static_cast<const char*>(x) + static_cast<size_t>(m0) * cols * (x_dtype == QFF_BF16 ? 2 : 4);
        {
            ProfScope prof(ctx, stream, "q4_x16");
            if (x_dtype == QFF_BF16)
                q4_x16_kernel<1, NORM><<<(mb + 3) / 4, 256, 0, stream>>>(xm, ctx->q4_x16, ctx->q4_fm, cols, mb, norm);
            else
                q4_x16_kernel<0, NORM><<<(mb + 3) / 4, 256, 0, stream>>>(xm, ctx->q4_x16, ctx->q4_fm, cols, mb, norm);
        }
        // one launch over every part's row tiles, outputs offset to this slice
        qff_q4_part sl[QFF_Q4_MAX_PARTS];
        for (int i = 0; i < nparts; ++i) {
            sl[i] = parts[i];
            const size_t yoff = static_cast<size_t>(m0) * parts[i].rows * (parts[i].y_dtype == QFF_BF16 ? 2 : 4);
            sl[i].y = static_cast<char*>(parts[i].y) + yoff;
            if (parts[i].residual) sl[i].residual = static_cast<const char*>(parts[i].residual) + yoff;
        }
        int tiles = 0;
        const Q4Parts P = q4_pack_parts(sl, nparts, kQ4GemmRows, tiles);
        const dim3 grid(tiles, (mb + kQ4GemmToks - 1) / kQ4GemmToks);
        ProfScope prof(ctx, stream, "q4_gemm");
        if (sb_dtype == QFF_BF16)
            q4_gemm_kernel<1><<<grid, 256, lds, stream>>>(P, ctx->q4_x16, ctx->q4_fm, cols, mb);
        else
            q4_gemm_kernel<2><<<grid, 256, lds, stream>>>(P, ctx->q4_x16, ctx->q4_fm, cols, mb);
    }
    return hipGetLastError();
}

// Decode batches: one launch over all parts.
template <bool NORM>
static hipError_t q4_gemv_parts(qff_ctx* ctx, hipStream_t stream, const qff_q4_part* parts, int nparts,
                                qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, const Q4Norm& norm,
                                int cols, int batch) {
    int blocks = 0;
    if (batch == 1) {
        // one token: the vector-unit streaming path
        const bool k2 = cols > 2048;
        const Q4Parts P = q4_pack_parts(parts, nparts, kQ4VecRows * kQ4VecWaves, blocks);
        ProfScope prof(ctx, stream, "q4_matmul");
#define QFF_Q4S(S, X)                                                                                   \
    if (k2) q4_gemv1_kernel<S, X, 2, NORM><<<blocks, 64 * kQ4VecWaves, 0, stream>>>(P, x, cols, norm); \
    else q4_gemv1_kernel<S, X, 1, NORM><<<blocks, 64 * kQ4VecWaves, 0, stream>>>(P, x, cols, norm)
#define QFF_Q4S_X(S) \
    if (x_dtype == QFF_BF16) { QFF_Q4S(S, 1); } else { QFF_Q4S(S, 0); }
        if (sb_dtype == QFF_BF16) { QFF_Q4S_X(1); } else { QFF_Q4S_X(2); }
#undef QFF_Q4S_X
#undef QFF_Q4S
        return hipGetLastError();
    }
    if (!NORM && batch <= 16 && cols == kQ4SkCols * kQ4SkSplit) {
        // 2-16 tokens at 4096 columns: the split-slice kernel and its
        // reduction launch, when the tiles fit the workspace's partials
        const Q4Parts P = q4_pack_parts(parts, nparts, kQ4SkRows, blocks);
        if (static_cast<size_t>(blocks) * kQ4SkSplit * 16 * kQ4SkRows <= static_cast<size_t>(kQ4SkSlots) * 1024) {
            ProfScope prof(ctx, stream, "q4_matmul");
            const dim3 grid(blocks, kQ4SkSplit);
#define QFF_Q4K(S, X) q4_gemv_sk_kernel<S, X><<<grid, 256, 0, stream>>>(P, x, batch, ctx->q4_sk_part)
#define QFF_Q4K_X(S) \
    if (x_dtype == QFF_BF16) { QFF_Q4K(S, 1); } else { QFF_Q4K(S, 0); }
            if (sb_dtype == QFF_BF16) { QFF_Q4K_X(1); } else { QFF_Q4K_X(2); }
#undef QFF_Q4K_X
#undef QFF_Q4K
            q4_sk_reduce_kernel<<<blocks, 256, 0, stream>>>(P, batch, ctx->q4_sk_part);
            return hipGetLastError();
        }
    }
    if (NORM && batch > 16) {
        // the normed product keeps one 16-token tile per launch (two tiles
        // of normed x do not fit the registers): tokens 0-15, then the rest
        qff_q4_part hi[QFF_Q4_MAX_PARTS];
        for (int i = 0; i < nparts; ++i) {
            const size_t off = static_cast<size_t>(16) * parts[i].rows * (parts[i].y_dtype == QFF_BF16 ? 2 : 4);
            hi[i] = parts[i];
            hi[i].y = static_cast<char*>(parts[i].y) + off;
            if (parts[i].residual) hi[i].residual = static_cast<const char*>(parts[i].residual) + off;
        }
        QFF_CHECK_HIP_RET((q4_gemv_parts<true>(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, 16)));
        const void* xh = static_cast<const char*>(x) + static_cast<size_t>(16) * cols * (x_dtype == QFF_BF16 ? 2 : 4);
        return q4_gemv_parts<true>(ctx, stream, hi, nparts, sb_dtype, xh, x_dtype, norm, cols, batch - 16);
    }
    // four row tiles per workgroup when x is read for several tokens over
    // enough rows to keep one workgroup per CU busy; one otherwise
    int total_rows = 0;
    for (int i = 0; i < nparts; ++i) total_rows += parts[i].rows;
    const bool rt4 = cols <= 2048 && total_rows >= 8192;
    const Q4Parts P = q4_pack_parts(parts, nparts, rt4 ? 64 : 16, blocks);
    const int nbt = (batch + 15) / 16;
    const bool g4 = q4_gemv_gpw(cols) == 4;
    ProfScope prof(ctx, stream, "q4_matmul");
#define QFF_Q4V1(S, X, NB, RTT, GP)                                                                        \
    {                                                                                                      \
        const int bytes = q4_gemv_lds_bytes<RTT, NB, GP>(cols);                                            \
        QFF_CHECK_HIP_RET((q4_allow_lds<q4_gemv_kernel<S, X, NB, RTT, NORM, GP>>(bytes)));                  \
        q4_gemv_kernel<S, X, NB, RTT, NORM, GP><<<blocks, 64 * q4_gemv_waves<GP>(cols), bytes, stream>>>(   \
            P, x, cols, batch, norm);                                                                      \
    }
#define QFF_Q4V(S, X, NB)                                        \
    if (rt4) {                                                   \
        QFF_Q4V1(S, X, NB, 4, 2)                                 \
    } else {                                                     \
        if (g4) QFF_Q4V1(S, X, NB, 1, 4) else QFF_Q4V1(S, X, NB, 1, 2) \
    }
#define QFF_Q4V_B(S, X)                          \
    if constexpr (NORM) {                        \
        QFF_Q4V(S, X, 1);                        \
    } else {                                     \
        if (nbt == 1) { QFF_Q4V(S, X, 1); } else { QFF_Q4V(S, X, 2); } \
    }
#define QFF_Q4V_X(S) \
    if (x_dtype == QFF_BF16) { QFF_Q4V_B(S, 1); } else { QFF_Q4V_B(S, 0); }
    if (sb_dtype == QFF_BF16) { QFF_Q4V_X(1); } else { QFF_Q4V_X(2); }
#undef QFF_Q4V_X
#undef QFF_Q4V_B
#undef QFF_Q4V
#undef QFF_Q4V1
    return hipGetLastError();
}

hipError_t launch_q4_parts(qff_ctx* ctx, hipStream_t stream, const qff_q4_part* parts, int nparts,
                           qff_dtype sb_dtype, const void* x, qff_dtype x_dtype, const Q4Norm& norm, int cols,
                           int batch) {
    if (cols / 64 > kQ4MaxGroups || nparts < 1 || nparts > QFF_Q4_MAX_PARTS) return hipErrorInvalidValue;
    const bool nrm = norm.w != nullptr;
    if (batch >= kQ4GemmMinBatch)
        return nrm ? q4_gemm_parts<true>(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, batch)
                   : q4_gemm_parts<false>(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, batch);
    return nrm ? q4_gemv_parts<true>(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, batch)
               : q4_gemv_parts<false>(ctx, stream, parts, nparts, sb_dtype, x, x_dtype, norm, cols, batch);
}

hipError_t launch_q4_matmul(qff_ctx* ctx, hipStream_t stream, const uint32_t* w, const void* scales,
                            const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                            void* y, qff_dtype y_dtype, int rows, int cols, int batch) {
    const qff_q4_part part{w, scales, biases, rows, y, y_dtype, nullptr};
    return launch_q4_parts(ctx, stream, &part, 1, sb_dtype, x, x_dtype, Q4Norm{}, cols, batch);
}

}  // namespace qff
