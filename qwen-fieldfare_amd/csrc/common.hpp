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

// Cross-lane moves for reductions over aligned lane groups, on the DPP and
// swizzle paths rather than LDS permutes: lane ^ 1 and lane ^ 2 (quad
// permutes), the mirror of a half row (8 lanes) and of a row (16 lanes),
// lane ^ 16 within 32 (swizzle), and the two 32-lane halves (permlane32
// swap). After the quad steps every lane of a quad holds the same value, so
// the mirrors pair each quad with the other one of its half row / row just
// as lane ^ 4 and lane ^ 8 would.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));   // and 0x1f, xor 0x10
}

// Sum over aligned groups of `W` lanes (W a power of two <= 64, all lanes of
// the group active); every lane of the group ends with the same total.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if (W >= 2) v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    if (W >= 4) v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    if (W >= 8) v += dpp_mov<0x141>(v);   // row_half_mirror
    if (W >= 16) v += dpp_mov<0x140>(v);  // row_mirror
    if (W >= 32) v += swizzle_xor16(v);
    if (W >= 64) {
        const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(h[0]) + __uint_as_float(h[1]);   // lower half + upper half, in every lane
    }
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
    if (W >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
    if (W >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
    if (W >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
    if (W >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if (W >= 32) v = fmaxf(v, swizzle_xor16(v));
    if (W >= 64) {
        const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    }
    return v;
}

// Integer sum / maximum over the whole wave (every lane gets the result) and
// the inclusive prefix sum over lanes 0 .. l, on the same DPP paths. The
// scan is the row-shift ladder within each row of 16 lanes, then
// row_bcast:15 (row r's last lane added to row r + 1) and row_bcast:31
// (lane 31 added to rows 2 and 3); lanes without a source add 0.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ int dpp_int(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, BANK_MASK, true);
}
__device__ __forceinline__ int wave_sum_int(int v) {
    v += dpp_int<0xB1>(v);
    v += dpp_int<0x4E>(v);
    v += dpp_int<0x141>(v);
    v += dpp_int<0x140>(v);
    v += __builtin_amdgcn_ds_swizzle(v, 0x401f);
    const auto h = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    return static_cast<int>(h[0] + h[1]);
}
__device__ __forceinline__ int wave_max_int(int v) {
    v = max(v, dpp_int<0xB1>(v));
    v = max(v, dpp_int<0x4E>(v));
    v = max(v, dpp_int<0x141>(v));
    v = max(v, dpp_int<0x140>(v));
    v = max(v, __builtin_amdgcn_ds_swizzle(v, 0x401f));
    const auto h = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    return max(static_cast<int>(h[0]), static_cast<int>(h[1]));
}
__device__ __forceinline__ int wave_inclusive_scan_int(int v) {
    v += dpp_int<0x111>(v);               // row_shr:1
    v += dpp_int<0x112>(v);               // row_shr:2
    v += dpp_int<0x114>(v);               // row_shr:4
    v += dpp_int<0x118>(v);               // row_shr:8
    v += dpp_int<0x142, 0xa>(v);          // row_bcast:15 into rows 1, 3
    v += dpp_int<0x143, 0xc>(v);          // row_bcast:31 into rows 2, 3
    return v;
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// 32-bit LDS byte address of a shared-memory element.
__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint16_t*)(p)));
}

// global_load_lds_dwordx4 from base + voff (base uniform, voff a 32-bit lane
// offset) to the LDS address in M0, lane l's 16 bytes at M0 + 16 l (the
// s_nop is the wait state an M0 write needs before an LDS DMA). The copy
// counts in vmcnt until its bytes are in LDS.
__device__ __forceinline__ void dma16(const char* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

}  // namespace qff
