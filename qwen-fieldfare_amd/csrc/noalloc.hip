// noalloc.hip -- qff_gqa_decode_static: the full-attention decode of
// qff_gqa_decode for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The split-KV partials (m, d, o per (sequence, kv head, chunk) slot) that
// qff_gqa_decode keeps in its context's workspace live here in one
// file-scope device array, `scratch`, of kSlots slots. Each GPU the library
// runs on holds its own copy of it until the process ends. Its device
// address on the current device is looked up with hipGetSymbolAddress on
// the first call there that succeeds in doing so, and cached; kernels only
// ever see that address. Nothing here calls hipMalloc, hipFree or any allocating
// routine.
//
// Every call on one GPU shares that GPU's array and it keeps the last
// call's contents: each partial is written by the call before the same call
// reads it, so nothing needs clearing, but two calls that overlap on one GPU
// (different streams, different threads) race on the slots.
#include <string.h>

#include <mutex>

#include "common.hpp"
#include "internal.hpp"

namespace qff {

constexpr int kStaticSlots = 4096;                  // (sequence, kv head, chunk) partial slots
constexpr int kStaticMaxBatch = 64;                 // 2 kv heads x 32 chunks each at the largest batch
constexpr size_t kSlotFloats = 8 + 8 + 8 * 256;     // m[8], d[8], o[8][256]
constexpr int kMaxDevices = 64;

// 4096 x 2064 fp32 = 33.8 MB per device.
static __device__ __align__(256) float scratch[kStaticSlots * kSlotFloats];

namespace {
std::mutex g_mu;
float* g_ptr[kMaxDevices];      // scratch's device address, per device (null until looked up)
int g_num_cu[kMaxDevices];
}  // namespace

// scratch's address and CU count on the current device. Only a successful
// set-up is cached: a failed one (a transient runtime error, a call refused
// while the stream is being captured) returns its status and is tried again
// on the next call.
static int static_scratch(float** ptr, int* num_cu) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return QFF_ERR_HIP;
    if (dev < 0 || dev >= kMaxDevices) return QFF_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        hipDeviceProp_t prop;
        void* p = nullptr;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return QFF_ERR_HIP;
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return QFF_ERR_UNSUPPORTED;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            (void)hipGetLastError();   // leave no sticky error for the caller's next call
            return QFF_ERR_HIP;
        }
        g_num_cu[dev] = prop.multiProcessorCount;
        g_ptr[dev] = static_cast<float*>(p);
    }
    *ptr = g_ptr[dev];
    *num_cu = g_num_cu[dev];
    return QFF_OK;
}

}  // namespace qff

using namespace qff;

extern "C" int qff_gqa_decode_static(qff_stream_t stream, const qff_gqa_params* p, const void* q_gate,
                                     const void* k_new, const void* v_new, qff_dtype in_dtype, void* k_cache,
                                     void* v_cache, const int32_t* positions, void* out, qff_dtype out_dtype,
                                     int batch, int max_ctx) {
    if (!q_gate || !k_new || !v_new || !k_cache || !v_cache || !positions || !out) return QFF_ERR_INVALID_ARG;
    if (const int st = gqa_params_status(p)) return st;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return QFF_ERR_INVALID_ARG;
    if (batch <= 0 || max_ctx <= 0) return QFF_ERR_INVALID_ARG;
    if (batch > kStaticMaxBatch) return QFF_ERR_WORKSPACE;
    float* base = nullptr;
    int num_cu = 0;
    const int st = static_scratch(&base, &num_cu);
    if (st != QFF_OK) return st;
    const size_t slots = kStaticSlots;
    int cap = kStaticSlots / (2 * batch);
    if (cap > kGqaMaxChunks) cap = kGqaMaxChunks;
    const GqaPartials ws{base, base + slots * 8, base + slots * 16, cap, num_cu};
    if (launch_gqa_decode_into(nullptr, ws, stream, p, q_gate, k_new, v_new, in_dtype, k_cache, v_cache, positions,
                               out, out_dtype, batch, max_ctx) != hipSuccess)
        return QFF_ERR_HIP;
    return QFF_OK;
}
