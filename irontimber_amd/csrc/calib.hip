// Matrix-core ceiling of this device, measured: every wave of a full grid runs chains of
// independent 32x32x16 f16 MFMAs (the instruction the attention and GDN products use) with no
// memory traffic, so flops / time is the f16 rate the hardware sustains at its clock under load.
// The prefill rooflines are quoted against the published peak and against this figure.
#include "common.h"
#include "internal.h"

namespace it {

constexpr int CALIB_CHAINS = 4;   // independent accumulators per wave: enough to fill the pipeline

__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* __restrict__ out) {
    const int tid = threadIdx.x;
    h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(((tid + i) & 7) * 0.125f);
        b[i] = (_Float16)(((tid * 3 + i) & 7) * 0.0625f);
    }
    f16v acc[CALIB_CHAINS];
#pragma unroll
    for (int j = 0; j < CALIB_CHAINS; ++j) acc[j] = f16v{};
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int j = 0; j < CALIB_CHAINS; ++j) acc[j] = mfma32x32x16(a, b, acc[j]);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CALIB_CHAINS; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[j][i];
    out[(size_t)blockIdx.x * 256 + tid] = s;   // keeps the chains live
}

hipError_t launch_mfma_peak(int wgs, int iters, float* out, hipStream_t st) {
    mfma_peak_kernel<<<wgs, 256, 0, st>>>(iters, out);
    return hipGetLastError();
}

}  // namespace it
