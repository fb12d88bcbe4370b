// mfma.hpp -- CDNA4 matrix-core operand types, the bf16 and fp16 MFMA
// shapes the kernels use and the operand conversions around them.
//
// Register layouts (wave64, lane l):
//   16x16x32 bf16 / f16: A[16 x 32]: lane l holds row l%16, k = 8*(l/16) .. +7
//                  B[32 x 16]: lane l holds col l%16, k = 8*(l/16) .. +7
//   16x16x16 bf16 / f16: A[16 x 16]: lane l holds row l%16, k = 4*(l/16) .. +3
//                  B[16 x 16]: lane l holds col l%16, k = 4*(l/16) .. +3
//   C/D[16 x 16] fp32: lane l holds col l%16, rows 4*(l/16) .. +3
//   32x32x16 f16: A[32 x 16]: lane l holds row l%32, k = 8*(l/32) .. +7
//                 B[16 x 32]: lane l holds col l%32, k = 8*(l/32) .. +7
//   C/D[32 x 32] fp32: lane l holds col l%32, element i row 8*(i/4) + 4*(l/32) + i%4
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qff {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4_t mfma_16x16x32_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma_16x16x16_bf16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4_t mfma_16x16x32_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma_32x32x16_f16(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma_16x16x16_f16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                 0, 0, 0);
}

// Two floats -> packed fp16 pair, round to nearest even; the low half holds lo.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// Two floats as fp16 hi and lo pairs: hi = fp16(x), lo = fp16(x - hi), so
// hi + lo carries ~22 significant bits for x in fp16's normal range (the
// remainder is exact in fp32; lo loses bits only where it falls below
// 2^-14, an absolute error under 2^-25).
__device__ __forceinline__ void split_f16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t h = {static_cast<_Float16>(x0), static_cast<_Float16>(x1)};
    hi = __builtin_bit_cast(uint32_t, h);
    lo = pack_f16x2(x0 - static_cast<float>(h[0]), x1 - static_cast<float>(h[1]));
}

// Two packed bf16 -> two packed fp16. Exact for every bf16 value inside the
// fp16 normal range (8 significant bits fit in 11); values below 2^-14 lose
// low bits to fp16's subnormals and values of magnitude >= 65520 become
// +-65504 (the reference keeps its KV cache in fp16 with the same limits).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ u32x4_t bf16x8_to_f16x8(u32x4_t v) {
    return u32x4_t{bf16x2_to_f16x2(v[0]), bf16x2_to_f16x2(v[1]), bf16x2_to_f16x2(v[2]), bf16x2_to_f16x2(v[3])};
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16). Within each group of 16
// lanes, lane s reads 4 consecutive 16-bit elements D[s][0..3] at its own
// address; lane i receives R[i][k] = D[4k + i/4][i % 4], k = 0..3. With a
// row-major [position][dim] tile in LDS, source lane s of group g pointing at
// row 4g + s/4, dims d0 + 4(s%4) .. +3 yields R[i][k] = tile[4g + k][d0 + i]:
// the B operand of a 16x16x16 MFMA whose k runs over positions.
__device__ __forceinline__ u32x2_t lds_read_tr16(const uint16_t* p) {
    typedef short s16x4_lds __attribute__((ext_vector_type(4)));
    const s16x4_lds v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s16x4_lds __attribute__((address_space(3)))*)(p));
    return __builtin_bit_cast(u32x2_t, v);
}

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32);
// the low half holds lo.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// fp32 -> (hi, lo) bf16 pair with hi + lo == x to ~2^-16 relative: the
// operands of the three-product "bf16x3" MFMA scheme
//   a b ~= a_hi b_hi + a_hi b_lo + a_lo b_hi
// which keeps fp32-class accuracy (~2^-16 relative per product) on the
// bf16 matrix cores. Inputs are finite.
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    const uint32_t h = pack_bf16x2(x, 0.0f);
    const float r = x - __uint_as_float(h << 16);
    hi = static_cast<uint16_t>(h);
    lo = static_cast<uint16_t>(pack_bf16x2(r, 0.0f));
}

// Two floats at once: packed hi pair and packed lo pair.
__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16x2(x0, x1);
    lo = pack_bf16x2(x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xffff0000u));
}

}  // namespace qff

namespace qff {

// 16x16 output tile, C += A B, bf16x3 on 16x16x32 MFMAs. A is row-major
// [16 rows][K] (hi/lo arrays, row stride lda elements, K contiguous).
// "NT": B is given as its transpose, row-major [16 cols][K] (stride ldb).
// "NN": B is row-major [K][16 cols] (stride ldb) and is read with the LDS
// transpose read, two per MFMA (k = 8kb .. 8kb+3 and 8kb+4 .. 8kb+7).
// All pointers are LDS addresses of the tile's first element; strides keep
// 16-byte (NT) / 8-byte (NN) alignment.
template <int K>
__device__ __forceinline__ f32x4_t mma_nt_x3(f32x4_t acc, const uint16_t* ah, const uint16_t* al, int lda,
                                             const uint16_t* bh, const uint16_t* bl, int ldb, int lane) {
    const int n = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 32) {
        const int ao = n * lda + k0 + 8 * kb, bo = n * ldb + k0 + 8 * kb;
        const u32x4_t a_h = *reinterpret_cast<const u32x4_t*>(ah + ao);
        const u32x4_t a_l = *reinterpret_cast<const u32x4_t*>(al + ao);
        const u32x4_t b_h = *reinterpret_cast<const u32x4_t*>(bh + bo);
        const u32x4_t b_l = *reinterpret_cast<const u32x4_t*>(bl + bo);
        acc = mfma_16x16x32_bf16(a_l, b_h, acc);
        acc = mfma_16x16x32_bf16(a_h, b_l, acc);
        acc = mfma_16x16x32_bf16(a_h, b_h, acc);
    }
    return acc;
}

template <int K>
__device__ __forceinline__ f32x4_t mma_nn_x3(f32x4_t acc, const uint16_t* ah, const uint16_t* al, int lda,
                                             const uint16_t* bh, const uint16_t* bl, int ldb, int lane) {
    const int n = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 32) {
        const int ao = n * lda + k0 + 8 * kb;
        const int bo = (k0 + 8 * kb + (n >> 2)) * ldb + 4 * (n & 3);
        const u32x4_t a_h = *reinterpret_cast<const u32x4_t*>(ah + ao);
        const u32x4_t a_l = *reinterpret_cast<const u32x4_t*>(al + ao);
        const u32x2_t h0 = lds_read_tr16(bh + bo), h1 = lds_read_tr16(bh + bo + 4 * ldb);
        const u32x2_t l0 = lds_read_tr16(bl + bo), l1 = lds_read_tr16(bl + bo + 4 * ldb);
        const u32x4_t b_h = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
        const u32x4_t b_l = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
        acc = mfma_16x16x32_bf16(a_l, b_h, acc);
        acc = mfma_16x16x32_bf16(a_h, b_l, acc);
        acc = mfma_16x16x32_bf16(a_h, b_h, acc);
    }
    return acc;
}

// acc += A[16x16] B[16x16] in fp32 on v_mfma_f32_16x16x4_f32 (A row-major
// stride lda, B row-major stride ldb; LDS or global).
// Layout: A lane l holds A[l%16][k = l/16], B lane l holds B[k = l/16][l%16].
__device__ __forceinline__ f32x4_t mm16_f32(const float* A, int lda, const float* B, int ldb, f32x4_t acc,
                                            int lane) {
    const int n = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[n * lda + 4 * kk + kq], B[(4 * kk + kq) * ldb + n], acc, 0, 0, 0);
    return acc;
}

// MR x NC block of 16x16 tiles, C[r][c] += A_r B_c with bf16x3, sharing each
// operand read across the block: A row tile r starts at row ar + 16 r of a
// row-major [rows][K] array; B column tile c starts at column bc + 16 c,
// given as its transpose (NT: row-major [cols][K]) or as row-major [K][cols]
// (NN, read with the LDS transpose read).
template <int K, int MR, int NC, bool NN>
__device__ __forceinline__ void mma_block_x3(f32x4_t (&acc)[MR][NC], const uint16_t* ah, const uint16_t* al,
                                             int lda, int ar, const uint16_t* bh, const uint16_t* bl, int ldb,
                                             int bc, int lane) {
    const int n = lane & 15, kb = lane >> 4;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 32) {
        u32x4_t a_h[MR], a_l[MR], b_h[NC], b_l[NC];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const int ao = (ar + 16 * r + n) * lda + k0 + 8 * kb;
            a_h[r] = *reinterpret_cast<const u32x4_t*>(ah + ao);
            a_l[r] = *reinterpret_cast<const u32x4_t*>(al + ao);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (NN) {
                const int bo = (k0 + 8 * kb + (n >> 2)) * ldb + bc + 16 * c + 4 * (n & 3);
                const u32x2_t h0 = lds_read_tr16(bh + bo), h1 = lds_read_tr16(bh + bo + 4 * ldb);
                const u32x2_t l0 = lds_read_tr16(bl + bo), l1 = lds_read_tr16(bl + bo + 4 * ldb);
                b_h[c] = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
                b_l[c] = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
            } else {
                const int bo = (bc + 16 * c + n) * ldb + k0 + 8 * kb;
                b_h[c] = *reinterpret_cast<const u32x4_t*>(bh + bo);
                b_l[c] = *reinterpret_cast<const u32x4_t*>(bl + bo);
            }
        }
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[r][c] = mfma_16x16x32_bf16(a_l[r], b_h[c], acc[r][c]);
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[r][c] = mfma_16x16x32_bf16(a_h[r], b_l[c], acc[r][c]);
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[r][c] = mfma_16x16x32_bf16(a_h[r], b_h[c], acc[r][c]);
    }
}

// Store 4 fp32 values as hi/lo bf16 at hi[i..i+3], lo[i..i+3] (8-byte aligned).
__device__ __forceinline__ void store_split4(uint16_t* hi, uint16_t* lo, int i, float a, float b, float c, float d) {
    uint32_t h0, l0, h1, l1;
    split_bf16x2(a, b, h0, l0);
    split_bf16x2(c, d, h1, l1);
    *reinterpret_cast<u32x2_t*>(hi + i) = u32x2_t{h0, h1};
    *reinterpret_cast<u32x2_t*>(lo + i) = u32x2_t{l0, l1};
}

}  // namespace qff
