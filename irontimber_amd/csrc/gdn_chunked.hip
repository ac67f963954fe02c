// Chunk-64 WY/UT gated-delta scan on the matrix cores.
#include "common.h"
#include "internal.h"
namespace it {
size_t gdn_chunked_scratch_bytes(int, int, int) { return 0; }
hipError_t launch_gdn_chunked(const float*, int, const float*, const float*, int, const float*, const float*, float*,
                              float*, int, int, int, int, void*, hipStream_t) {
    return hipErrorNotSupported;
}
}  // namespace it
