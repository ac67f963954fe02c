// Whole-prompt / long-chunk causal attention on the matrix cores (flash form, no scratch).
#include "common.h"
#include "internal.h"
namespace it {
hipError_t launch_attn_flash(const float*, int, const uint16_t*, const uint16_t*, int, int, int, int, int, float, float*,
                             int, hipStream_t) {
    return hipErrorNotSupported;
}
}  // namespace it
