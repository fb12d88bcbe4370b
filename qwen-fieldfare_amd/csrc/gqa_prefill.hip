// gqa_prefill.hip -- causal full-attention prefill (placeholder until the
// flash kernel lands): reports the shape as unsupported.
#include "internal.hpp"

namespace qff {

hipError_t launch_gqa_prefill(qff_ctx*, hipStream_t, const qff_gqa_params*, const void*, const void*,
                              const void*, qff_dtype, void*, void*, int, void*, qff_dtype, int, int) {
    return hipErrorNotSupported;
}

}  // namespace qff
