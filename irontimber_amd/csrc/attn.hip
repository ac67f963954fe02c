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
// Scores are kept in log2 units (q.k * scale * log2 e) so the exponentials are single v_exp_f32;
// the MFMA rows of the q hi and q lo halves land in separate LDS score rows and are summed when
// read (no cross-lane shuffle); the softmax gives each wave whole rows and reduces with DPP.
constexpr float LOG2E_F = 1.4426950408889634f;
constexpr float LN2_F = 0.6931471805599453f;

template <int NB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void attn_partial_kernel(
    const float* __restrict__ q, int qts, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    int kvd, int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ part, int chunk, int smax) {
    constexpr int ROWS = 8 * NB, KT = 16 * WAVES, NTH = 64 * WAVES;
    constexpr int NTW = 16 / WAVES;          // 16-dim output tiles per wave
    constexpr int VPL = KT / 64;             // softmax values per lane
    constexpr int RPW = ROWS / WAVES;        // softmax rows per wave (1 for decode)
    static_assert(ROWS % WAVES == 0, "rows spread evenly over waves");
    __shared__ __align__(16) _Float16 Ks[KT * KST];
    __shared__ __align__(16) _Float16 Vs[KT * VST];
    __shared__ __align__(16) _Float16 Qs[2][ROWS][KST];   // [hi|lo][row][dim]
    __shared__ __align__(16) float Ps[2][ROWS][KT + 4];   // scores of the q-hi / q-lo MFMA rows
    __shared__ float alpha_s[ROWS];
    __shared__ int lim_s[ROWS];                            // row sees keys < lim (0 for padding rows)
    __shared__ int qoff_s[ROWS];                           // row's q offset (floats), -1 for padding

    const int s = blockIdx.x, kh = blockIdx.y, rg = blockIdx.z;
    const int G = nh / nkv, R = nt * G, r0 = rg * ROWS;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int tmax = (min(R, r0 + ROWS) - 1) / G;
    const int p0 = s * chunk;
    const int pend = min(p0 + chunk, pos0 + tmax + 1);
    if (p0 >= pend) return;  // no row of this group sees these keys; the combine never reads them
    const float sc2 = scale * LOG2E_F;

    if (tid < ROWS) {
        const int rr = r0 + tid;
        const bool ok = rr < R;
        const int t = ok ? rr / G : 0;
        lim_s[tid] = ok ? pos0 + t + 1 : 0;
        qoff_s[tid] = ok ? t * qts + (kh * G + rr % G) * 2 * HD : -1;
    }
    float m_run[RPW], l_run[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) { m_run[j] = -INFINITY; l_run[j] = 0.f; }
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
    __syncthreads();                                 // lim_s / qoff_s
    constexpr int QIT = (ROWS * HD / 8 + NTH - 1) / NTH;
    f4 qx[QIT][2];
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
        const int idx = tid + NTH * it;          // 8-float piece: row idx/32, dims 8*(idx%32)
        qx[it][0] = qx[it][1] = f4{0.f, 0.f, 0.f, 0.f};
        if (idx < ROWS * HD / 8) {
            const int qo = qoff_s[idx >> 5];
            if (qo >= 0) {
                const float* src = q + qo + 8 * (idx & 31);
                qx[it][0] = ld_f4(src); qx[it][1] = ld_f4(src + 4);
            }
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
        // ---- scores for every row block: MFMA rows 0-7 = q_hi, 8-15 = q_lo of the block's 8 rows
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
            // lane l holds MFMA rows 4*(l>>4)+i: rows 0-7 (l < 32) are q_hi, rows 8-15 are q_lo
            const int half = l >> 5;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rloc = (4 * (l >> 4) + i) & 7;
                Ps[half][b * 8 + rloc][16 * w + (l & 15)] = sacc[i];
            }
        }
        __syncthreads();
        // ---- online softmax: wave w owns rows w, w + WAVES, ...; lane covers VPL key columns
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int row = w + WAVES * j;
            const int lim = lim_s[row];
            float x[VPL];
            float mx = -INFINITY;
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
                const int col = l + 64 * v;
                const bool ok = kb + col < lim;
                x[v] = ok ? (Ps[0][row][col] + Ps[1][row][col]) * sc2 : -INFINITY;
                mx = fmaxf(mx, x[v]);
            }
            mx = wave_max(mx);
            const float mnew = fmaxf(m_run[j], mx);
            const float a = (mnew == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[j] - mnew);
            const float msub = (mnew == -INFINITY) ? 0.0f : mnew;
            float sum = 0.f;
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
                x[v] = __builtin_amdgcn_exp2f(x[v] - msub);
                sum += x[v];
                Ps[0][row][l + 64 * v] = x[v];
            }
            sum = wave_sum(sum);
            l_run[j] = l_run[j] * a + sum;
            m_run[j] = mnew;
            if (l == 0) alpha_s[row] = a;
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
            const float* prow = &Ps[0][b * 8 + (si & 7)][0];
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
    // ---- write the partial records {m, l, 0, 0, o[256]} (m in natural-log units): the P-hi and
    // P-lo MFMA rows of O are summed across the two lane halves, staged in LDS (reusing the K
    // tile), then stored as whole 1040-byte records with 16-byte stores
    float* Os = (float*)Ks;   // [ROWS][256]
    static_assert(ROWS * HD * 4 <= KT * KST * 2, "O fits in the K tile");
    const int dw = (HD / WAVES) * w;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int n = 0; n < NTW; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float o = acc[b][n][i] + __shfl_xor(acc[b][n][i], 32);
                if (l < 32) Os[(b * 8 + 4 * (l >> 4) + i) * HD + dw + 16 * n + (l & 15)] = o;
            }
#pragma unroll
    for (int j = 0; j < RPW; ++j)
        if (l == 0) { Ps[1][w + WAVES * j][0] = m_run[j] * LN2_F; Ps[1][w + WAVES * j][1] = l_run[j]; }
    __syncthreads();
    for (int idx = tid; idx < ROWS * 65; idx += NTH) {
        const int row = idx / 65, c = idx % 65, rq = r0 + row;
        if (rq >= R) continue;
        const int t = rq / G, h = kh * G + rq % G;
        const f4 v = c == 0 ? f4{Ps[1][row][0], Ps[1][row][1], 0.f, 0.f} : *(const f4*)&Os[row * HD + 4 * (c - 1)];
        *(f4*)(part + ((size_t)(t * nh + h) * smax + s) * PART + 4 * c) = v;
    }
}

// ------------------------------------------------------------------------------------------------
// Merge the partials of (head h, token t): M = max m_s, den = sum l_s e^(m_s-M),
// out = sum o_s e^(m_s-M) / den * sigmoid(gate). Same merge as kernels/src/lib.rs:722-740, spread
// over the splits: workgroup (h, t, quarter of the 256 dims); thread = (split lane sg = tid/16,
// 4 dims). Each thread loads the m, l and o of its splits in one batch (one memory round trip),
// the maxima and sums reduce through LDS.
constexpr int COMB_SPL = 8;   // splits per split lane held in registers (larger ns loops)
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ q, int qts, int pos0, int nh,
                                                          const float* __restrict__ part, int chunk, int smax,
                                                          float* __restrict__ out, int ots) {
    __shared__ float red_m[16];
    __shared__ f4 red_o[16][16];
    __shared__ float red_d[16];
    const int h = blockIdx.x, t = blockIdx.y, dq = blockIdx.z, tid = threadIdx.x;
    const int n = pos0 + t + 1, ns = (n + chunk - 1) / chunk;
    const float* base = part + (size_t)(t * nh + h) * smax * PART;
    const int sg = tid >> 4, dl = tid & 15, d0 = 64 * dq + 4 * dl;
    float M = -INFINITY, den = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += 16 * COMB_SPL) {
        float mv[COMB_SPL], lv[COMB_SPL];
        f4 ov[COMB_SPL];
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) {
            const int s = s0 + sg + 16 * j;
            mv[j] = -INFINITY; lv[j] = 0.f; ov[j] = f4{0.f, 0.f, 0.f, 0.f};
            if (s < ns) {
                const float* rec = base + (size_t)s * PART;
                mv[j] = rec[0]; lv[j] = rec[1]; ov[j] = ld_f4(rec + 4 + d0);
            }
        }
        float mloc = M;
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) mloc = fmaxf(mloc, mv[j]);
        // group maximum over the 16 split lanes (lanes with the same dl share nothing else)
        if (dl == 0) red_m[sg] = mloc;
        __syncthreads();
        float Mn = red_m[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) Mn = fmaxf(Mn, red_m[j]);
        __syncthreads();
        const float r = (M == -INFINITY) ? 0.f : expf(M - Mn);
        den *= r; o *= r;
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) {
            const float wgt = mv[j] == -INFINITY ? 0.f : expf(mv[j] - Mn);
            den += lv[j] * wgt;
            o += ov[j] * wgt;
        }
        M = Mn;
    }
    red_o[sg][dl] = o;
    if (dl == 0) red_d[sg] = den;
    __syncthreads();
    if (tid < 16) {
        f4 acc = red_o[0][tid];
        float dd = red_d[0];
        for (int j = 1; j < 16; ++j) { acc += red_o[j][tid]; dd += red_d[j]; }
        const f4 gt = ld_f4(q + (size_t)t * qts + (size_t)h * 2 * HD + HD + 64 * dq + 4 * tid);
        f4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = acc[j] / dd * sigmoidf_(gt[j]);
        *(f4*)(out + (size_t)t * ots + (size_t)h * HD + 64 * dq + 4 * tid) = r;
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
