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
//   load    : K and V rows with fully coalesced 16-byte loads (a wave instruction covers two whole
//             512-byte head rows), staged row-major in LDS; the query rows are staged once as
//             f16 hi + lo (hi + lo == q to ~2^-22), all loads in flight together.
//   scores  : wave w takes keys 16w..16w+15 (MFMA 16x16x32, B = K rows from LDS); MFMA rows 0-7
//             carry q_hi, rows 8-15 q_lo, so hi.K + lo.K is an f32-accurate dot product.
//   softmax : online (running max m and sum l per row), 8 threads per row.
//   P.V     : P split hi+lo the same way; V's B operand comes from the row-major tile through the
//             LDS transpose read; wave w owns output dims 64w..64w+63.
// Writes the reference's partial record at part + ((t*nh + h)*smax + s)*260.
constexpr int KST = HD + 8;    // LDS row stride (halves) of the K tile: 528 B, 4-bank shift per row
constexpr int VST = HD + 16;   // LDS row stride (halves) of the V tile: 544 B, 8-bank shift per row

// WAVES waves per workgroup; a tile is KT = 16*WAVES keys (each wave scores 16 keys). The decode
// shape (8 rows) uses 8 waves / 128-key tiles so one workgroup covers a whole split with all of
// its loads in flight at once; wider row blocks use 4 waves / 64-key tiles to fit LDS.
template <int NB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void attn_partial_kernel(
    const float* __restrict__ q, int qts, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    int kvd, int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ part, int chunk, int smax) {
    constexpr int ROWS = 8 * NB, KT = 16 * WAVES, NTH = 64 * WAVES;
    constexpr int CPR = KT / 8;              // softmax threads per row (8 columns each)
    constexpr int NTW = 16 / WAVES;          // 16-dim output tiles per wave
    __shared__ __align__(16) _Float16 Ks[KT * KST];
    __shared__ __align__(16) _Float16 Vs[KT * VST];
    __shared__ __align__(16) _Float16 Qs[2][ROWS][KST];   // [hi|lo][row][dim]
    __shared__ __align__(16) float Ps[ROWS][KT + 4];
    __shared__ float alpha_s[ROWS];

    const int s = blockIdx.x, kh = blockIdx.y, rg = blockIdx.z;
    const int G = nh / nkv, R = nt * G, r0 = rg * ROWS;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int tmax = (min(R, r0 + ROWS) - 1) / G;
    const int p0 = s * chunk;
    const int pend = min(p0 + chunk, pos0 + tmax + 1);
    if (p0 >= pend) return;  // no row of this group sees these keys; the combine never reads them

    const int sr = tid / CPR, c8 = tid % CPR;   // softmax role: row sr, columns 8*c8..8*c8+7
    float m_run = -INFINITY, l_run = 0.0f;
    f4 acc[NB][NTW];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int n = 0; n < NTW; ++n) acc[b][n] = f4{0.f, 0.f, 0.f, 0.f};

    const size_t head_off = (size_t)kh * HD;
    const int lrow = tid >> 5, lch = tid & 31;   // load role: rows lrow + (NTH/32)*i, 16-byte chunk lch
    // Loads are issued in the order they are consumed -- query rows, then the tile's K rows, then
    // its V rows -- so the scores and the softmax run while V is still arriving, and the next
    // tile's K/V are loaded while the current P.V runs. Rows past pend are clamped to a valid row
    // (masked scores, P = 0).
    u4 kr[8], vr[8];
    auto load_k = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            kr[i] = *(const u4*)(kc + (size_t)min(kb + lrow + (NTH / 32) * i, pend - 1) * kvd + head_off + 8 * lch);
    };
    auto load_v = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            vr[i] = *(const u4*)(vc + (size_t)min(kb + lrow + (NTH / 32) * i, pend - 1) * kvd + head_off + 8 * lch);
    };
    constexpr int QIT = (ROWS * HD / 8 + NTH - 1) / NTH;
    f4 qx[QIT][2];
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
        const int idx = tid + NTH * it;          // 8-float piece: row idx/32, dims 8*(idx%32)
        const int row = idx >> 5, rr = r0 + row;
        qx[it][0] = qx[it][1] = f4{0.f, 0.f, 0.f, 0.f};
        if (idx < ROWS * HD / 8 && rr < R) {
            const float* src = q + (size_t)(rr / G) * qts + (size_t)(kh * G + rr % G) * 2 * HD + 8 * (idx & 31);
            qx[it][0] = ld_f4(src); qx[it][1] = ld_f4(src + 4);
        }
    }
    load_k(p0);
    load_v(p0);
    // stage the query rows once, as f16 hi + lo
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
        const int idx = tid + NTH * it;
        if (idx < ROWS * HD / 8) {
            const int row = idx >> 5, d0 = 8 * (idx & 31);
            h8 hi, lo;
            split_hi_lo(qx[it][0], qx[it][1], hi, lo);
            *(h8*)&Qs[0][row][d0] = hi;
            *(h8*)&Qs[1][row][d0] = lo;
        }
    }

    for (int kb = p0; kb < pend; kb += KT) {
#pragma unroll
        for (int i = 0; i < 8; ++i) *(u4*)&Ks[(lrow + (NTH / 32) * i) * KST + 8 * lch] = kr[i];
        __syncthreads();
        // ---- scores for every row block
        const int pk = kb + 16 * w + (l & 15);
        const _Float16* krow = &Ks[(16 * w + (l & 15)) * KST + 8 * (l >> 4)];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int row16 = l & 15;
            f4 sacc = {0.f, 0.f, 0.f, 0.f};
            if (r0 + b * 8 < R) {   // wave-uniform: skip empty row blocks
                const _Float16* qrow = &Qs[row16 >> 3][b * 8 + (row16 & 7)][8 * (l >> 4)];
                h8 qa[8], kbv[8];
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) { qa[ks] = ld_h8(qrow + 32 * ks); kbv[ks] = ld_h8(krow + 32 * ks); }
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) sacc = mfma16x16x32(qa[ks], kbv[ks], sacc);
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
        __syncthreads();
        // ---- online softmax update (ROWS*CPR is a multiple of 64: whole waves take part)
        if (sr < ROWS) {
            f4 x0 = *(const f4*)&Ps[sr][8 * c8], x1 = *(const f4*)&Ps[sr][8 * c8 + 4];
            float mx = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3])),
                             fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3])));
#pragma unroll
            for (int m = 1; m < CPR; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
            const float mnew = fmaxf(m_run, mx);
            const float a = (mnew == -INFINITY) ? 1.0f : expf(m_run - mnew);
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x0[j] = (x0[j] == -INFINITY) ? 0.f : expf(x0[j] - mnew);
                x1[j] = (x1[j] == -INFINITY) ? 0.f : expf(x1[j] - mnew);
                sum += x0[j] + x1[j];
            }
#pragma unroll
            for (int m = 1; m < CPR; m <<= 1) sum += __shfl_xor(sum, m);
            l_run = l_run * a + sum;
            m_run = mnew;
            *(f4*)&Ps[sr][8 * c8] = x0;
            *(f4*)&Ps[sr][8 * c8 + 4] = x1;
            if (c8 == 0) alpha_s[sr] = a;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) *(u4*)&Vs[(lrow + (NTH / 32) * i) * VST + 8 * lch] = vr[i];
        if (kb + KT < pend) { load_k(kb + KT); load_v(kb + KT); }
        __syncthreads();
        // ---- O = diag(alpha) O + P V; wave w owns dims (256/WAVES)*w ..
        const int g = l >> 4, si = l & 15;
        const int dw = (HD / WAVES) * w;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (r0 + b * 8 >= R) continue;   // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = alpha_s[b * 8 + ((4 * g + i) & 7)];
#pragma unroll
                for (int n = 0; n < NTW; ++n) acc[b][n][i] *= a;
            }
            const float* prow = &Ps[b * 8 + (si & 7)][0];
#pragma unroll
            for (int ks = 0; ks < KT / 32; ++ks) {
                h8 hi, lo;
                split_hi_lo(*(const f4*)(prow + 32 * ks + 8 * g), *(const f4*)(prow + 32 * ks + 8 * g + 4), hi, lo);
                const h8 pa = si >= 8 ? lo : hi;
                const _Float16* vsrc = &Vs[(32 * ks + 8 * g + (si >> 2)) * VST + dw + 4 * (si & 3)];
#pragma unroll
                for (int n = 0; n < NTW; ++n) {
                    const h8 vb = cat_h4(lds_tr4(vsrc + 16 * n), lds_tr4(vsrc + 4 * VST + 16 * n));
                    acc[b][n] = mfma16x16x32(pa, vb, acc[b][n]);
                }
            }
        }
        __syncthreads();
    }
    // ---- write the partial records {m, l, 0, 0, o[256]}: stage o in LDS (reusing the K tile),
    // then 16-byte coalesced stores of whole 1040-byte records
    float* Os = (float*)Ks;   // [ROWS][256]
    const int dw = (HD / WAVES) * w;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int n = 0; n < NTW; ++n) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float o = acc[b][n][i] + __shfl_xor(acc[b][n][i], 32);
                if (l < 32) Os[(b * 8 + 4 * (l >> 4) + i) * HD + dw + 16 * n + (l & 15)] = o;
            }
        }
    }
    if (sr < ROWS && c8 == 0) { Ps[sr][0] = m_run; Ps[sr][1] = l_run; }
    __syncthreads();
    for (int idx = tid; idx < ROWS * 65; idx += NTH) {
        const int row = idx / 65, c = idx % 65, rq = r0 + row;
        if (rq >= R) continue;
        const int t = rq / G, h = kh * G + rq % G;
        const f4 v = c == 0 ? f4{Ps[row][0], Ps[row][1], 0.f, 0.f} : *(const f4*)&Os[row * HD + 4 * (c - 1)];
        *(f4*)(part + ((size_t)(t * nh + h) * smax + s) * PART + 4 * c) = v;
    }
}

// ------------------------------------------------------------------------------------------------
// Merge the partials of (head h, token t): M = max m_s, den = sum l_s e^(m_s-M),
// out = sum o_s e^(m_s-M) / den * sigmoid(gate). Same merge as kernels/src/lib.rs:722-740, spread
// over the splits: workgroup (h, t, quarter of the 256 dims); thread = (split lane sg = tid/16,
// 4 dims); the 16 split lanes reduce through LDS.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ q, int qts, int pos0, int nh,
                                                          const float* __restrict__ part, int chunk, int smax,
                                                          float* __restrict__ out, int ots) {
    __shared__ float red_m[4];
    __shared__ f4 red_o[16][16];
    __shared__ float red_d[16];
    const int h = blockIdx.x, t = blockIdx.y, dq = blockIdx.z, tid = threadIdx.x, l = tid & 63, w = tid >> 6;
    const int n = pos0 + t + 1, ns = (n + chunk - 1) / chunk;
    const float* base = part + (size_t)(t * nh + h) * smax * PART;
    float M = -INFINITY;
    for (int s = tid; s < ns; s += 256) M = fmaxf(M, base[(size_t)s * PART]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) M = fmaxf(M, __shfl_xor(M, m));
    if (l == 0) red_m[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    const int sg = tid >> 4, dl = tid & 15, d0 = 64 * dq + 4 * dl;
    float den = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
    for (int s = sg; s < ns; s += 16) {
        const float* rec = base + (size_t)s * PART;
        const float wgt = expf(rec[0] - M);
        den += rec[1] * wgt;
        o += ld_f4(rec + 4 + d0) * wgt;
    }
    red_o[sg][dl] = o;
    if (dl == 0) red_d[sg] = den;
    __syncthreads();
    if (tid < 16) {
        f4 acc = red_o[0][tid];
        float dd = red_d[0];
        for (int j = 1; j < 16; ++j) { acc += red_o[j][tid]; dd += red_d[j]; }
        const int dd0 = 64 * dq + 4 * tid;
        const f4 g = ld_f4(q + (size_t)t * qts + (size_t)h * 2 * HD + HD + dd0);
        f4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = acc[j] / dd * sigmoidf_(g[j]);
        *(f4*)(out + (size_t)t * ots + (size_t)h * HD + dd0) = r;
    }
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

hipError_t launch_attn_partials(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                                int nh, int nkv, int nt, float scale, float* part, int chunk, hipStream_t st) {
    const int G = nh / nkv, R = nt * G;
    const int smax = (pos0 + nt + chunk - 1) / chunk;
    const int rows = attn_partial_rows_per_group(nt, G);
    const dim3 grid(smax, nkv, (R + rows - 1) / rows);
    switch (rows / 8) {
        case 1:
            if (chunk % 128 == 0)
                attn_partial_kernel<1, 8><<<grid, 512, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax);
            else
                attn_partial_kernel<1, 4><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax);
            break;
        case 2: attn_partial_kernel<2, 4><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
        case 3: attn_partial_kernel<3, 4><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
        default: attn_partial_kernel<4, 4><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax); break;
    }
    return hipGetLastError();
}

hipError_t launch_attn_combine(const float* q, int qts, const float* part, int pos0, int nh, int nt, int chunk,
                               float* out, int ots, hipStream_t st) {
    const int smax = (pos0 + nt + chunk - 1) / chunk;
    attn_combine_kernel<<<dim3(nh, nt, 4), 256, 0, st>>>(q, qts, pos0, nh, part, chunk, smax, out, ots);
    return hipGetLastError();
}

hipError_t launch_attn_splitk(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                              int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                              hipStream_t st) {
    hipError_t e = launch_attn_partials(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, st);
    if (e != hipSuccess) return e;
    return launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, st);
}

}  // namespace it
