// Attention pre-pass in one launch: per-head RMSNorm of q and k with their weights, neox-style
// (I)MRoPE on the first n_rot dims of each q/k head, and the f16 append of K and V to the cache.
// The q half of each [q | gate] head block is rewritten in place (f32); the gate half is not touched.
// Optionally q also goes out as the flash prefill kernel's f16 operand, q16[t][h][d] =
// f16(q * q16s) with q16s = scale * log2(e), rounded as that kernel would round it.
//
// Reference behaviour: cpu.rs:249-258 (norm, rope, f16 round, append), cpu.rs:14-18 (rmsnorm),
// cpu.rs:145-162 and shaders/rope.comp:1-19 (rope and its sector rule), kernels/src/lib.rs:207-229
// mode 0 (weighted RMSNorm), lib.rs:743-750 (KV pack); dispatch sequence vk/mod.rs:822-838.
#include "common.h"
#include "internal.h"

namespace it {

constexpr int PREP_WAVES = 4;

// Rotation angle of frequency i at position p: theta = p * tsc^i, with tsc the caller's f32
// theta_scale. The power (binary exponentiation, at most 14 f64 products) and the reduction to
// [-pi, pi] run in f64, so the f32 sin/cos see an argument accurate to f32 rounding even at
// positions near 2^22 (the reference's f32 recurrences lose ~2e-4 rad by position 8191).
__device__ __forceinline__ void rope_angle(int p, int i, float tsc, float& c, float& s) {
    double pw = 1.0, b = (double)tsc;
    for (int e = i; e; e >>= 1, b *= b)
        if (e & 1) pw *= b;
    const double th = (double)p * pw;
    const double two_pi = 6.283185307179586476925286766559;
    const float r = (float)(th - two_pi * __builtin_rint(th * (1.0 / two_pi)));
    sincosf(r, &s, &c);
}

// The sector rule of cpu.rs:152-155 / rope.comp:11-13: a frequency whose sector lies beyond the
// text sections takes the "e" position, 0 for text tokens.
__device__ __forceinline__ bool rope_use_e(int i, int s0, int s1, int s2, int s3) {
    const int sect = s0 + s1 + s2 + s3;
    if (sect <= 0) return false;
    const int sec = i % sect;
    return !((sec % 3 == 1 && sec < 3 * s1) || (sec % 3 == 2 && sec < 3 * s2) || (sec % 3 == 0 && sec < 3 * s0));
}

template <int E>
struct RowT;
template <> struct RowT<2> { typedef f2 T; };
template <> struct RowT<4> { typedef f4 T; };

__device__ __forceinline__ uint32_t pack_f16(float a, float b, int rtz) {
    if (rtz) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    h2 x = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, x);
}

// One wave per head row, ceil((nh + 2 nkv) / 4) workgroups per token. Token t is roped at position
// pos0 + t and its K/V rows go to cache row row0 + t (row0 = pos0 for the model's f16 cache; the
// MTP head's f32 cache keeps position p in slot p - 1, src/mtp.rs:120). KVT = uint16_t stores f16,
// KVT = float stores the f32 values as they are. Rows of token t: [0, nh) q heads, [nh, nh+nkv) k heads, then nkv v heads.
// Lane l holds elements E*l .. E*l+E-1 of the row (hd = 64*E).
template <int E, class KVT>
__global__ __launch_bounds__(64 * PREP_WAVES) void attn_prep_kernel(
    float* __restrict__ q, int qts, const float* __restrict__ k, const float* __restrict__ v, int kts,
    const float* __restrict__ qw, const float* __restrict__ kw, float eps, KVT* __restrict__ kc,
    KVT* __restrict__ vc, int kvd, int pos0, int row0, int nh, int nkv, int n_rot, float tsc, int s0, int s1, int s2,
    int s3, int rtz, _Float16* __restrict__ q16, int q16ts, float q16s) {
    typedef typename RowT<E>::T V;
    constexpr int HDK = 64 * E;
    __shared__ float cs_c[HDK / 2], cs_s[HDK / 2];
    const int groups = (nh + 2 * nkv + PREP_WAVES - 1) / PREP_WAVES;
    const int t = blockIdx.x / groups, g = blockIdx.x - t * groups, w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int half = n_rot >> 1, p = pos0 + t;
    // The row load goes out first; the angle table below is computed while it is in flight.
    const int r = g * PREP_WAVES + w;
    const bool live = r < nh + 2 * nkv;
    const int kind = r < nh ? 0 : (r < nh + nkv ? 1 : 2);   // 0 q, 1 k, 2 v
    const int kh = kind == 0 ? r : (kind == 1 ? r - nh : r - nh - nkv);
    const float* src = kind == 0 ? q + (size_t)t * qts + (size_t)kh * 2 * HDK
                                 : (kind == 1 ? k : v) + (size_t)t * kts + (size_t)kh * HDK;
    V x = {};
    if (live) x = *(const V*)(src + E * l);
    for (int i = threadIdx.x; i < half; i += 64 * PREP_WAVES) {
        float c = 1.0f, s = 0.0f;
        if (!rope_use_e(i, s0, s1, s2, s3)) rope_angle(p, i, tsc, c, s);
        cs_c[i] = c;
        cs_s[i] = s;
    }
    __syncthreads();
    if (!live) return;   // whole wave: nothing below synchronises across waves
    if (kind != 2) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < E; ++j) ss += x[j] * x[j];
        ss = wave_sum(ss);
        const float sc = 1.0f / sqrtf(ss / (float)HDK + eps);
        const float* wt = kind == 0 ? qw : kw;
        V wv;
        if (wt) wv = *(const V*)(wt + E * l);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = wt ? (x[j] * sc) * wv[j] : x[j] * sc;
        // Rotation of the pair (e, e + half) for e < half: both partners sit in lanes half/E apart
        // with the same element slot (half % E == 0, checked by the host).
        const int e0 = E * l, dl = half / E;
        const bool lo = e0 < half, rot = e0 < n_rot;
        const int src_lane = lo ? l + dl : l - dl;
        V y = x;
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float other = __shfl(x[j], rot ? src_lane : l);
            if (rot) {
                const int i = (lo ? e0 : e0 - half) + j;
                const float c = cs_c[i], s = cs_s[i];
                y[j] = lo ? x[j] * c - other * s : other * s + x[j] * c;
            }
        }
        x = y;
    }
    if (kind == 0) {
        *(V*)(q + (size_t)t * qts + (size_t)kh * 2 * HDK + E * l) = x;
        if (q16) {
            _Float16* d = q16 + (size_t)t * q16ts + (size_t)kh * HDK + E * l;
            if constexpr (E == 4) *(h4*)d = h4{(_Float16)(x[0] * q16s), (_Float16)(x[1] * q16s), (_Float16)(x[2] * q16s),
                                              (_Float16)(x[3] * q16s)};
            else *(h2*)d = h2{(_Float16)(x[0] * q16s), (_Float16)(x[1] * q16s)};
        }
        return;
    }
    KVT* dst = (kind == 1 ? kc : vc) + (size_t)(row0 + t) * kvd + (size_t)kh * HDK + E * l;
    if constexpr (sizeof(KVT) == 4) {
        *(V*)dst = x;
    } else if constexpr (E == 4) {
        uint32_t* d = (uint32_t*)dst;
        d[0] = pack_f16(x[0], x[1], rtz);
        d[1] = pack_f16(x[2], x[3], rtz);
    } else {
        *(uint32_t*)dst = pack_f16(x[0], x[1], rtz);
    }
}

template <class KVT>
static hipError_t launch_prep(float* q, int qts, const float* k, const float* v, int kts, const float* qw,
                              const float* kw, float eps, KVT* kc, KVT* vc, int pos0, int row0, int hd, int nh,
                              int nkv, int nt, int n_rot, float tsc, const int* sec, int rtz, hipStream_t st,
                              _Float16* q16 = nullptr, int q16ts = 0, float q16s = 0.f) {
    const long groups = (nh + 2 * nkv + PREP_WAVES - 1) / PREP_WAVES;   // workgroups per token
    const dim3 grid((unsigned)(groups * nt)), block(64 * PREP_WAVES);
    const int kvd = nkv * hd;
    if (hd == 256)
        attn_prep_kernel<4, KVT><<<grid, block, 0, st>>>(q, qts, k, v, kts, qw, kw, eps, kc, vc, kvd, pos0, row0, nh,
                                                        nkv, n_rot, tsc, sec[0], sec[1], sec[2], sec[3], rtz, q16,
                                                        q16ts, q16s);
    else
        attn_prep_kernel<2, KVT><<<grid, block, 0, st>>>(q, qts, k, v, kts, qw, kw, eps, kc, vc, kvd, pos0, row0, nh,
                                                        nkv, n_rot, tsc, sec[0], sec[1], sec[2], sec[3], rtz, q16,
                                                        q16ts, q16s);
    return hipGetLastError();
}

hipError_t launch_attn_prep(float* q, int qts, const float* k, const float* v, int kts, const float* qw,
                            const float* kw, float eps, uint16_t* kc, uint16_t* vc, int pos0, int hd, int nh, int nkv,
                            int nt, int n_rot, float tsc, const int* sec, int rtz, hipStream_t st, uint16_t* q16,
                            int q16ts, float q16s) {
    return launch_prep<uint16_t>(q, qts, k, v, kts, qw, kw, eps, kc, vc, pos0, pos0, hd, nh, nkv, nt, n_rot, tsc, sec,
                                 rtz, st, (_Float16*)q16, q16ts, q16s);
}

hipError_t launch_attn_prep_f32kv(float* q, int qts, const float* k, const float* v, int kts, const float* qw,
                                  const float* kw, float eps, float* kc, float* vc, int pos0, int row0, int hd, int nh,
                                  int nkv, int nt, int n_rot, float tsc, const int* sec, hipStream_t st) {
    return launch_prep<float>(q, qts, k, v, kts, qw, kw, eps, kc, vc, pos0, row0, hd, nh, nkv, nt, n_rot, tsc, sec, 0,
                              st);
}

}  // namespace it
