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
// 128 + q by OR-ing it into the mantissa of 0x4300 (128.0), so one
// v_mfma_f32_16x16x32_bf16 yields P = sum (128 + q) x over 32 columns, and
//   sum_c W x = s * P + (b - 128 s) * sum(x)       (per group, per row)
// with sum(x) over the same bf16-rounded x the MFMA saw. A wave owns a
// 16-row x 16-column output tile and walks the groups; each group's scale
// and folded bias come from LDS, staged once per workgroup.
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

// 8 nibbles -> 4 dwords of bf16 pairs holding 128 + q (exact).
__device__ __forceinline__ u32x4_t q4_to_bf16_offset(uint32_t w) {
    u32x4_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = 0x43004300u | ((w >> (8 * i)) & 0xFu) | (((w >> (8 * i + 4)) & 0xFu) << 16);
    return r;
}

// x[m][c0 .. c0+7] as 8 bf16 (rounded when x is fp32); zeros past `batch`.
template <int X_DT>
__device__ __forceinline__ u32x4_t load_x8(const void* x, int m, int batch, int cols, int c0) {
    if (m >= batch) return u32x4_t{0u, 0u, 0u, 0u};
    const size_t off = static_cast<size_t>(m) * cols + c0;
    if (X_DT == 1) return *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + off);
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + off);
    const float4 a = p[0], b = p[1];
    return u32x4_t{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
}

template <int X_DT>
__device__ __forceinline__ float load_x_rounded(const void* x, size_t i) {
    if (X_DT == 1) return bf16_to_f32(static_cast<const uint16_t*>(x)[i]);
    return bf16_to_f32(f32_to_bf16(static_cast<const float*>(x)[i]));
}

constexpr int kQ4MaxGroups = 64;  // cols <= 4096

// grid (ceil(rows/64), ceil(batch/16)), 256 threads: wave w owns rows
// blockIdx.x*64 + 16w .. +15 and batch columns blockIdx.y*16 .. +15.
template <int SB_DT, int X_DT, int Y_DT>
__global__ __launch_bounds__(256) void q4_matmul_mfma_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const void* __restrict__ x, void* __restrict__ y, int rows, int cols, int batch) {
    const int G = cols / 64;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = lane & 15, kb = lane >> 4;
    const int r0 = blockIdx.x * 64 + wave * 16;
    const int m0 = blockIdx.y * 16;

    __shared__ float xsum[16][kQ4MaxGroups];
    __shared__ float2 sb[4][kQ4MaxGroups][16];

    for (int idx = t; idx < 16 * G; idx += 256) {
        const int m = idx / G, g = idx % G;
        float acc = 0.0f;
        if (m0 + m < batch) {
            const size_t base = static_cast<size_t>(m0 + m) * cols + g * 64;
            for (int c = 0; c < 64; ++c) acc += load_x_rounded<X_DT>(x, base + c);
        }
        xsum[m][g] = acc;
    }
    for (int idx = lane; idx < 16 * G; idx += 64) {
        const int i = idx / G, g = idx % G;
        float2 v = make_float2(0.0f, 0.0f);
        if (r0 + i < rows) {
            const size_t gi = static_cast<size_t>(r0 + i) * G + g;
            const float s = elem<SB_DT>::load(scales, gi);
            const float b = elem<SB_DT>::load(biases, gi);
            v = make_float2(s, b - 128.0f * s);
        }
        sb[wave][g][i] = v;
    }
    __syncthreads();

    const int row = min(r0 + n, rows - 1);
    const uint32_t* wrow = w + static_cast<size_t>(row) * (cols / 8);
    const int m = m0 + n;
    float yacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g = 0; g < G; ++g) {
        f32x4_t P = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int c0 = 64 * g + 32 * hf + 8 * kb;
            const u32x4_t a = q4_to_bf16_offset(wrow[c0 / 8]);
            const u32x4_t b = load_x8<X_DT>(x, m, batch, cols, c0);
            P = mfma_16x16x32_bf16(a, b, P);
        }
        const float X = xsum[n][g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 v = sb[wave][g][4 * kb + i];
            yacc[i] = fmaf(v.x, P[i], fmaf(v.y, X, yacc[i]));
        }
    }
    if (m < batch) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 4 * kb + i;
            if (r < rows) elem<Y_DT>::store(y, static_cast<size_t>(m) * rows + r, yacc[i]);
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

hipError_t launch_q4_matmul(qff_ctx* ctx, hipStream_t stream, const uint32_t* w, const void* scales,
                            const void* biases, qff_dtype sb_dtype, const void* x, qff_dtype x_dtype,
                            void* y, qff_dtype y_dtype, int rows, int cols, int batch) {
    if (cols / 64 > kQ4MaxGroups) return hipErrorInvalidValue;
    const dim3 grid((rows + 63) / 64, (batch + 15) / 16);
    ProfScope prof(ctx, stream, "q4_matmul");
    const uint16_t* s = static_cast<const uint16_t*>(scales);
    const uint16_t* b = static_cast<const uint16_t*>(biases);
#define QFF_Q4(S, X, Y) q4_matmul_mfma_kernel<S, X, Y><<<grid, 256, 0, stream>>>(w, s, b, x, y, rows, cols, batch)
#define QFF_Q4_Y(S, X) \
    if (y_dtype == QFF_BF16) QFF_Q4(S, X, 1); else QFF_Q4(S, X, 0)
#define QFF_Q4_X(S) \
    if (x_dtype == QFF_BF16) { QFF_Q4_Y(S, 1); } else { QFF_Q4_Y(S, 0); }
    if (sb_dtype == QFF_BF16) { QFF_Q4_X(1); } else { QFF_Q4_X(2); }
#undef QFF_Q4_X
#undef QFF_Q4_Y
#undef QFF_Q4
    return hipGetLastError();
}

}  // namespace qff
