// peaks.hip -- what this part delivers, measured: the roofline denominators
// bench.py reports beside the datasheet peaks (HBM 8 TB/s, dense bf16 MFMA
// 2.5 PFLOP/s). A measurement helper of bench.py only (libqff_probe.so),
// not part of the product's C ABI.
//
//   qffp_mfma_bf16   every wave issues `iters` rounds of independent bf16
//                    MFMAs on register operands, one float per wave out:
//                    shape 0 two v_mfma_f32_32x32x16_bf16 chains (32768
//                    flops each), shape 1 sixteen v_mfma_f32_16x16x32_bf16
//                    chains (16384 flops each). Fewer 16x16x32 chains than
//                    that leave the matrix core waiting on each chain's
//                    result (8 chains: ~1.4-1.6 PFLOP/s).
//   qffp_stream_read every thread reads 16-byte pieces of `bytes` at a
//                    grid-wide stride (global_load_dwordx4) and folds them
//                    into one float it writes out.
//   qffp_stream_copy the same access pattern, each piece written to dst.
//   qffp_stream_rmw  the same access pattern, each piece scaled in place
//                    (what an in-place state update moves: read + write of
//                    the same bytes).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int kShape>
__global__ __launch_bounds__(256) void mfma_bf16_kernel(int iters, float* __restrict__ sink) {
    constexpr int kChains = kShape == 0 ? 2 : 16;
    using acc_t = typename std::conditional<kShape == 0, f32x16_t, f32x4_t>::type;
    const int lane = threadIdx.x & 63;
    const u32x4_t a = u32x4_t{0x3f803f80u + lane, 0x3f803f80u, 0x3f813f81u, 0x3f823f82u};
    const u32x4_t b = u32x4_t{0x3c003c00u, 0x3c013c01u + lane, 0x3c023c02u, 0x3c033c03u};
    acc_t acc[kChains];
#pragma unroll
    for (int i = 0; i < kChains; ++i) acc[i] = acc_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < kChains; ++i) {
            if constexpr (kShape == 0)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                                 __builtin_bit_cast(bf16x8_t, b), acc[i], 0, 0, 0);
            else
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                                 __builtin_bit_cast(bf16x8_t, b), acc[i], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kChains; ++i) s += acc[i][0] + acc[i][3];
    if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* __restrict__ src, size_t n,
                                                          float* __restrict__ sink) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    uint32_t x = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const u32x4_t v = src[i];
        x ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    sink[static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x] = __uint_as_float(x);
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                          size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void stream_rmw_kernel(float4* __restrict__ p, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        float4 v = p[i];
        v.x *= 0.999f;
        v.y *= 0.999f;
        v.z *= 0.999f;
        v.w *= 0.999f;
        p[i] = v;
    }
}

extern "C" {

// blocks workgroups of 4 waves; sink holds blocks * 4 floats. Flops:
// blocks * 4 * iters * 65536 (shape 0) or * 262144 (shape 1).
int qffp_mfma_bf16(hipStream_t stream, int shape, int blocks, int iters, float* sink) {
    if (blocks <= 0 || iters <= 0 || !sink || (shape != 0 && shape != 1)) return -1;
    if (shape == 0)
        mfma_bf16_kernel<0><<<blocks, 256, 0, stream>>>(iters, sink);
    else
        mfma_bf16_kernel<1><<<blocks, 256, 0, stream>>>(iters, sink);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// bytes a multiple of 16; sink holds blocks * 256 floats.
int qffp_stream_read(hipStream_t stream, const void* src, size_t bytes, int blocks, float* sink) {
    if (!src || !sink || blocks <= 0 || bytes % 16) return -1;
    stream_read_kernel<<<blocks, 256, 0, stream>>>(static_cast<const u32x4_t*>(src), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int qffp_stream_copy(hipStream_t stream, const void* src, void* dst, size_t bytes, int blocks) {
    if (!src || !dst || blocks <= 0 || bytes % 16) return -1;
    stream_copy_kernel<<<blocks, 256, 0, stream>>>(static_cast<const u32x4_t*>(src), static_cast<u32x4_t*>(dst),
                                                   bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int qffp_stream_rmw(hipStream_t stream, void* p, size_t bytes, int blocks) {
    if (!p || blocks <= 0 || bytes % 16) return -1;
    stream_rmw_kernel<<<blocks, 256, 0, stream>>>(static_cast<float4*>(p), bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
