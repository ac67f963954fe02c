// KV append for the f16 cache: f32 K/V rows -> f16 rows at pos0.. (round to nearest even, or
// toward zero like the reference's packHalf2x16 on its HAWAII GPU).
//
// Reference behaviour: kernels/src/lib.rs:743-750 (KV pack), src/vk/r012_parity.rs:14-18 (RTZ).
#include "common.h"
#include "internal.h"

namespace it {

// ------------------------------------------------------------------------------------------------
// KV append: f32 rows -> f16 cache rows pos0..pos0+nt-1. One thread per 4 values.
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                        int sts, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                        int pos0, int nt, int kvd, int rtz) {
    const int per_tok = kvd / 4;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)nt * per_tok * 2) return;
    const int which = i >= (long)nt * per_tok;           // 0 = K, 1 = V
    const long j = which ? i - (long)nt * per_tok : i;
    const int t = (int)(j / per_tok), c = (int)(j % per_tok) * 4;
    const f4 x = ld_f4((which ? v : k) + (size_t)t * sts + c);
    uint16_t* dst = (which ? vc : kc) + (size_t)(pos0 + t) * kvd + c;
    uint32_t w0, w1;
    if (rtz) {
        w0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[0], x[1]));
        w1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[2], x[3]));
    } else {
        h2 a = {(_Float16)x[0], (_Float16)x[1]}, b = {(_Float16)x[2], (_Float16)x[3]};
        w0 = __builtin_bit_cast(uint32_t, a); w1 = __builtin_bit_cast(uint32_t, b);
    }
    uint32_t* d = (uint32_t*)dst;
    d[0] = w0; d[1] = w1;
}

// ------------------------------------------------------------------------------------------------
hipError_t launch_kv_append(const float* k, const float* v, int sts, uint16_t* kc, uint16_t* vc, int pos0, int nt,
                            int kvd, int rtz, hipStream_t st) {
    const long n = (long)nt * (kvd / 4) * 2;
    if (n == 0) return hipSuccess;
    kv_append_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(k, v, sts, kc, vc, pos0, nt, kvd, rtz);
    return hipGetLastError();
}

}  // namespace it
