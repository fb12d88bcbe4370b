// mfma.hpp -- CDNA4 matrix-core operand types and the two bf16 MFMA shapes
// the attention kernels use.
//
// Register layouts (wave64, lane l):
//   16x16x32 bf16: A[16 x 32]: lane l holds row l%16, k = 8*(l/16) .. +7
//                  B[32 x 16]: lane l holds col l%16, k = 8*(l/16) .. +7
//   16x16x16 bf16: A[16 x 16]: lane l holds row l%16, k = 4*(l/16) .. +3
//                  B[16 x 16]: lane l holds col l%16, k = 4*(l/16) .. +3
//   C/D[16 x 16] fp32: lane l holds col l%16, rows 4*(l/16) .. +3
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

// Two floats -> packed bf16 pair (round to nearest even), low half = lo.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    uint32_t a = __float_as_uint(lo), b = __float_as_uint(hi);
    a += 0x7fffu + ((a >> 16) & 1u);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (a >> 16) | (b & 0xffff0000u);
}

}  // namespace qff
