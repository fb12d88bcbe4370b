// common.hpp -- device helpers shared by the gfx950 kernels: storage
// conversions, wave64 reductions and dtype-generic loads/stores.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qff {

// bf16 and f16 tensors travel as 16-bit patterns.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 v = static_cast<_Float16>(f);
    return __builtin_bit_cast(uint16_t, v);
}

// Element access for a runtime dtype code (0 f32, 1 bf16, 2 f16) resolved at
// compile time through the template parameter.
template <int DT> struct elem;
template <> struct elem<0> {
    static __device__ __forceinline__ float load(const void* p, size_t i) { return static_cast<const float*>(p)[i]; }
    static __device__ __forceinline__ void store(void* p, size_t i, float v) { static_cast<float*>(p)[i] = v; }
};
template <> struct elem<1> {
    static __device__ __forceinline__ float load(const void* p, size_t i) { return bf16_to_f32(static_cast<const uint16_t*>(p)[i]); }
    static __device__ __forceinline__ void store(void* p, size_t i, float v) { static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); }
};
template <> struct elem<2> {
    static __device__ __forceinline__ float load(const void* p, size_t i) { return f16_to_f32(static_cast<const uint16_t*>(p)[i]); }
    static __device__ __forceinline__ void store(void* p, size_t i, float v) { static_cast<uint16_t*>(p)[i] = f32_to_f16(v); }
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
// SiLU on the hardware exp2 and reciprocal (a few ulp) for bulk elementwise
// work whose consumers tolerate it.
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return expf(x);
    return log1pf(expf(x));
}

// Butterfly sum over aligned groups of `W` lanes (W a power of two <= 64);
// every lane of the group ends with the group total.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = W / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int m = W / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

}  // namespace qff
