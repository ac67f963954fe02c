// Softmax attention over an f16 KV cache for gfx950: KV append, split-K partials on the matrix
// cores, log-sum-exp combine with the sigmoid output gate.
//
// Reference behaviour: src/cpu.rs:260-272 (math), kernels/src/lib.rs:722-798 (split-K partial
// record {m, l, pad, pad, o[256]} and its merge), kernels/src/lib.rs:743-750 (KV pack).
#include "common.h"
#include "internal.h"

namespace it {

constexpr int HD = 256;     // head_dim (the only one the reference's f16 path supports)
constexpr int PART = 260;   // partial record words: m, l, pad, pad, o[256]
constexpr int VTS = 72;     // LDS row stride (halves) of the transposed V tile: 64 keys + 8 pad

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
// Split-K partials for a block of query rows sharing one KV head.
//
// Rows r = t*G + g (token t, head g of the KV group, G = nh/nkv) all read the same K/V, so one
// workgroup loads each key once for up to 8*NB rows (the reference reloads K/V per q head,
// kernels/src/lib.rs:753-798). Grid: (split s, KV head kh, row group rg); 4 waves.
// Per 64-key tile:
//   scores  : wave w takes keys 16w..16w+15; K rows are the MFMA B operand straight from HBM
//             (16-byte loads); the query is split f16 hi+lo into MFMA rows 0-7 / 8-15 so that
//             hi.K + lo.K reproduces an f32 dot product against the exact f16 keys.
//   softmax : online (running max m and sum l per row), 8 threads per row.
//   P.V     : P split hi+lo the same way; V transposed through LDS so keys are the contraction
//             dimension; wave w owns output dims 64w..64w+63.
// Writes the reference's partial record at part + ((t*nh + h)*smax + s)*260.
template <int NB>
__global__ __launch_bounds__(256) void attn_partial_kernel(
    const float* __restrict__ q, int qts, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    int kvd, int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ part, int chunk, int smax) {
    constexpr int ROWS = 8 * NB;
    __shared__ __align__(16) float Ps[ROWS][64 + 4];
    __shared__ float alpha_s[ROWS];
    __shared__ __align__(16) uint16_t Vt[HD * VTS];

    const int s = blockIdx.x, kh = blockIdx.y, rg = blockIdx.z;
    const int G = nh / nkv, R = nt * G, r0 = rg * ROWS;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int tmax = (min(R, r0 + ROWS) - 1) / G;
    const int p0 = s * chunk;
    const int pend = min(p0 + chunk, pos0 + tmax + 1);
    if (p0 >= pend) return;  // no row of this group sees these keys; the combine never reads them

    const int sr = tid >> 3, c8 = tid & 7;     // softmax role: row sr, columns 8*c8..8*c8+7
    float m_run = -INFINITY, l_run = 0.0f;
    f4 acc[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[b][n] = f4{0.f, 0.f, 0.f, 0.f};

    const size_t head_off = (size_t)kh * HD;
    const int kp = tid & 31, dcb = tid >> 5;   // V transpose role: keys 2kp, 2kp+1; dim chunks dcb+8c

    for (int kb = p0; kb < pend; kb += 64) {
        // ---- issue the tile's HBM loads first (K operand, V rows)
        const int pk = kb + 16 * w + (l & 15);
        const uint16_t* krow = kc + (size_t)min(pk, pend - 1) * kvd + head_off + 8 * (l >> 4);
        h8 kop[8];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) kop[ks] = ld_h8(krow + 32 * ks);
        u4 vv[2][4];
        {
            const uint16_t* v0 = vc + (size_t)min(kb + 2 * kp, pend - 1) * kvd + head_off;
            const uint16_t* v1 = vc + (size_t)min(kb + 2 * kp + 1, pend - 1) * kvd + head_off;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                vv[0][c] = *(const u4*)(v0 + (dcb + 8 * c) * 8);
                vv[1][c] = *(const u4*)(v1 + (dcb + 8 * c) * 8);
            }
        }
        // ---- scores for every row block
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int row16 = l & 15;
            const int rr = r0 + b * 8 + (row16 & 7);
            f4 sacc = {0.f, 0.f, 0.f, 0.f};
            if (r0 + b * 8 < R) {   // wave-uniform: skip empty row blocks
                const bool lo_half = row16 >= 8;
                const float* qrow = nullptr;
                if (rr < R) qrow = q + (size_t)(rr / G) * qts + (size_t)(kh * G + rr % G) * 2 * HD + 8 * (l >> 4);
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    h8 hi = {}, lo = {};
                    if (qrow) split_hi_lo(ld_f4(qrow + 32 * ks), ld_f4(qrow + 32 * ks + 4), hi, lo);
                    sacc = mfma16x16x32(lo_half ? lo : hi, kop[ks], sacc);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float tot = sacc[i] + __shfl_xor(sacc[i], 32);
                if (l < 32) {
                    const int rloc = 4 * (l >> 4) + i;
                    const int rq = r0 + b * 8 + rloc;
                    const bool valid = rq < R && pk < pos0 + rq / G + 1;
                    Ps[b * 8 + rloc][16 * w + (l & 15)] = valid ? tot * scale : -INFINITY;
                }
            }
        }
        // ---- V tile -> LDS, transposed to [dim][key]
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t a = (vv[0][c][j >> 1] >> (16 * (j & 1))) & 0xffffu;
                const uint32_t bb = (vv[1][c][j >> 1] >> (16 * (j & 1))) & 0xffffu;
                *(uint32_t*)&Vt[((dcb + 8 * c) * 8 + j) * VTS + 2 * kp] = a | (bb << 16);
            }
        }
        __syncthreads();
        // ---- online softmax update
        if (sr < ROWS) {
            f4 x0 = *(const f4*)&Ps[sr][8 * c8], x1 = *(const f4*)&Ps[sr][8 * c8 + 4];
            float mx = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3])),
                             fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3])));
            mx = fmaxf(mx, __shfl_xor(mx, 1));
            mx = fmaxf(mx, __shfl_xor(mx, 2));
            mx = fmaxf(mx, __shfl_xor(mx, 4));
            const float mnew = fmaxf(m_run, mx);
            const float a = (mnew == -INFINITY) ? 1.0f : expf(m_run - mnew);
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x0[j] = (x0[j] == -INFINITY) ? 0.f : expf(x0[j] - mnew);
                x1[j] = (x1[j] == -INFINITY) ? 0.f : expf(x1[j] - mnew);
                sum += x0[j] + x1[j];
            }
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            sum += __shfl_xor(sum, 4);
            l_run = l_run * a + sum;
            m_run = mnew;
            *(f4*)&Ps[sr][8 * c8] = x0;
            *(f4*)&Ps[sr][8 * c8 + 4] = x1;
            if (c8 == 0) alpha_s[sr] = a;
        } else {
            // keep the shuffles above convergent: rows past ROWS do nothing
        }
        __syncthreads();
        // ---- O = diag(alpha) O + P V
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (r0 + b * 8 >= R) continue;   // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = alpha_s[b * 8 + ((4 * (l >> 4) + i) & 7)];
#pragma unroll
                for (int n = 0; n < 4; ++n) acc[b][n][i] *= a;
            }
            const int row16 = l & 15;
            const float* prow = &Ps[b * 8 + (row16 & 7)][0];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                h8 hi, lo;
                split_hi_lo(*(const f4*)(prow + 32 * ks + 8 * (l >> 4)), *(const f4*)(prow + 32 * ks + 8 * (l >> 4) + 4), hi, lo);
                const h8 pa = row16 >= 8 ? lo : hi;
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    const int dim = 64 * w + 16 * n + (l & 15);
                    acc[b][n] = mfma16x16x32(pa, ld_h8(&Vt[dim * VTS + 32 * ks + 8 * (l >> 4)]), acc[b][n]);
                }
            }
        }
        __syncthreads();
    }
    // ---- write the partial records
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int n = 0; n < 4; ++n) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float o = acc[b][n][i] + __shfl_xor(acc[b][n][i], 32);
                const int rq = r0 + b * 8 + 4 * (l >> 4) + i;
                if (l < 32 && rq < R) {
                    const int t = rq / G, h = kh * G + rq % G;
                    part[((size_t)(t * nh + h) * smax + s) * PART + 4 + 64 * w + 16 * n + (l & 15)] = o;
                }
            }
        }
    }
    if (sr < ROWS && c8 == 0 && r0 + sr < R) {
        const int rq = r0 + sr, t = rq / G, h = kh * G + rq % G;
        float* rec = part + ((size_t)(t * nh + h) * smax + s) * PART;
        rec[0] = m_run; rec[1] = l_run;
    }
}

// ------------------------------------------------------------------------------------------------
// Merge the partials of (head h, token t): M = max m_s, den = sum l_s e^(m_s-M),
// out = sum o_s e^(m_s-M) / den * sigmoid(gate). Same merge as kernels/src/lib.rs:722-740.
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ q, int qts, int pos0, int nh,
                                                         const float* __restrict__ part, int chunk, int smax,
                                                         float* __restrict__ out, int ots) {
    const int h = blockIdx.x, t = blockIdx.y, l = threadIdx.x;
    const int n = pos0 + t + 1, ns = (n + chunk - 1) / chunk;
    const float* base = part + (size_t)(t * nh + h) * smax * PART;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, base[(size_t)s * PART]);
    float den = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < ns; ++s) {
        const float* rec = base + (size_t)s * PART;
        const float wgt = expf(rec[0] - M);
        den += rec[1] * wgt;
        o += ld_f4(rec + 4 + 4 * l) * wgt;
    }
    const f4 g = ld_f4(q + (size_t)t * qts + (size_t)h * 2 * HD + HD + 4 * l);
    f4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = o[j] / den * sigmoidf_(g[j]);
    *(f4*)(out + (size_t)t * ots + (size_t)h * HD + 4 * l) = r;
}

// ------------------------------------------------------------------------------------------------
hipError_t launch_kv_append(const float* k, const float* v, int sts, uint16_t* kc, uint16_t* vc, int pos0, int nt,
                            int kvd, int rtz, hipStream_t st) {
    const long n = (long)nt * (kvd / 4) * 2;
    if (n == 0) return hipSuccess;
    kv_append_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(k, v, sts, kc, vc, pos0, nt, kvd, rtz);
    return hipGetLastError();
}

int attn_partial_rows_per_group(int nt, int G) {
    const int R = nt * G;
    return R <= 8 ? 8 : R <= 16 ? 16 : R <= 24 ? 24 : 32;
}

hipError_t launch_attn_splitk(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                              int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                              hipStream_t st) {
    const int G = nh / nkv, R = nt * G;
    const int smax = (pos0 + nt + chunk - 1) / chunk;
    const int rows = attn_partial_rows_per_group(nt, G);
    const dim3 grid(smax, nkv, (R + rows - 1) / rows);
    switch (rows / 8) {
        case 1: attn_partial_kernel<1><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
        case 2: attn_partial_kernel<2><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
        case 3: attn_partial_kernel<3><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
        default: attn_partial_kernel<4><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_combine_kernel<<<dim3(nh, nt), 64, 0, st>>>(q, qts, pos0, nh, part, chunk, smax, out, ots);
    return hipGetLastError();
}

}  // namespace it
