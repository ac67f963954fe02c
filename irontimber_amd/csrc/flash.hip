// Causal GQA attention for prefill on the matrix cores (flash form: one pass over the keys, online
// softmax, no scratch). Same math as src/cpu.rs:260-272 for every query row; the reference's GPU
// counterparts are the multi-query split-K tiles of kernels/src/prefill_attention*.rs and
// kernels/src/prefill_gqa.rs.
//
// Workgroup = 128 query rows sharing one KV head (rows r = t*G + g: token t, head g of the group,
// G = nh/nkv), 4 waves of 32 rows. Per 64-key tile, in the transposed form so that every lane owns
// one query row:
//   S^T  = K Q^T          MFMA 32x32x16: A = K rows from LDS, B = q (f16, pre-scaled by
//                         scale*log2 e) held in registers for the whole kernel.
//                         Lane l holds query (l & 31), keys 8*(i/4) + 4*(l>>5) + (i&3).
//   softmax              running max / sum per query in the log2 domain: 32 scores in the lane, one
//                         exchange with lane l^32 for the other 32.
//   O^T += V^T P^T        A = V^T through the LDS transpose read of the row-major V tile, B = P^T
//                         straight from the S^T accumulator (f16); O^T lives in 8 accumulator
//                         tiles (256 dims x 32 queries per wave).
// K/V tiles are staged in LDS with fully coalesced 16-byte loads; the next tile is loaded into
// registers while the current one is computed. Row tiles are scheduled heaviest (most keys) first.
#include "common.h"
#include "internal.h"

namespace it {

namespace {
constexpr int HD = 256;
constexpr int BM = 128, BN = 64;
constexpr int KST = HD + 8;    // K tile row stride (halves)
constexpr int VST = HD + 16;   // V tile row stride (halves)
constexpr float LOG2E = 1.4426950408889634f;
}

__global__ __launch_bounds__(256) void attn_flash_kernel(
    const float* __restrict__ q, int qts, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int kvd,
    int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ out, int ots) {
    __shared__ __align__(16) _Float16 Ks[BN * KST];
    __shared__ __align__(16) _Float16 Vs[BN * VST];

    const int G = nh / nkv, R = nt * G;
    const int nrt = (R + BM - 1) / BM;
    const int rt = nrt - 1 - (int)blockIdx.x;          // heaviest row tile first
    const int kh = blockIdx.y;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, hh = l >> 5, c = l & 31;
    const int r = rt * BM + 32 * w + c;                 // this lane's query row
    const bool rvalid = r < R;
    const int t = rvalid ? r / G : 0;
    const int head = kh * G + (rvalid ? r % G : 0);
    const int tmin = (rt * BM) / G, tmax = (min(R, rt * BM + BM) - 1) / G;
    const int kend = pos0 + tmax + 1;                   // keys any row of the tile sees
    const int kfull = pos0 + tmin + 1;                  // keys every row of the tile sees
    const int qlim = pos0 + t;                          // this row sees keys <= qlim

    // q as the B operand: column = query c, k = dims 16*ks + 8*hh + 0..7, scaled into log2 units
    h8 qb[16];
    {
        const float sc = scale * LOG2E;
        const float* src = q + (size_t)t * qts + (size_t)head * 2 * HD + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            if (rvalid) qb[ks] = to_h8(ld_f4(src + 16 * ks) * sc, ld_f4(src + 16 * ks + 4) * sc);
            else qb[ks] = h8{};
        }
    }
    f16v o[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] = f16v{};
    float m_run = -INFINITY, l_run = 0.f;

    const size_t head_off = (size_t)kh * HD;
    const int lrow = tid >> 5, lch = tid & 31;          // load role: rows lrow + 8i, chunk lch
    u4 kr[8], vr[8];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const size_t row = (size_t)min(kb + lrow + 8 * i, kend - 1) * kvd + head_off + 8 * lch;
            kr[i] = *(const u4*)(kc + row);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const size_t row = (size_t)min(kb + lrow + 8 * i, kend - 1) * kvd + head_off + 8 * lch;
            vr[i] = *(const u4*)(vc + row);
        }
    };
    load_tile(0);

    // V^T operand addressing for the transpose read: lane l provides &V[key0 + (l&15)/4][col0 + 4*(l&3)]
    const int vrow = (l & 15) >> 2, vcol = 16 * ((l >> 4) & 1) + 4 * (l & 3);

    for (int kb = 0; kb < kend; kb += BN) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            *(u4*)&Ks[(lrow + 8 * i) * KST + 8 * lch] = kr[i];
            *(u4*)&Vs[(lrow + 8 * i) * VST + 8 * lch] = vr[i];
        }
        if (kb + BN < kend) load_tile(kb + BN);
        __syncthreads();

        // ---- S^T = K Q^T for two 32-key blocks
        f16v s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            s[b] = f16v{};
            const _Float16* ka = &Ks[(32 * b + c) * KST + 8 * hh];
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) s[b] = mfma32x32x16(ld_h8(ka + 16 * ks), qb[ks], s[b]);
        }
        // ---- causal mask (only tiles that reach past the first row's diagonal)
        if (kb + BN > kfull) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kb + 32 * b + 8 * (i >> 2) + 4 * hh + (i & 3);
                    if (!rvalid || key > qlim) s[b][i] = -INFINITY;
                }
        }
        // ---- online softmax (log2 domain)
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[b][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(m_run, mx);
        const float alpha = (mnew == -INFINITY) ? 1.0f : exp2f(m_run - mnew);
        const float msub = (mnew == -INFINITY) ? 0.0f : mnew;
        float lsum = 0.f;
        h8 pb[4];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = exp2f(s[b][8 * kk + j] - msub);
                    lsum += p;
                    pb[2 * b + kk][j] = (_Float16)p;
                }
        lsum += __shfl_xor(lsum, 32);
        l_run = l_run * alpha + lsum;
        m_run = mnew;
#pragma unroll
        for (int db = 0; db < 8; ++db) o[db] *= alpha;
        // ---- O^T += V^T P^T: k-step ks covers keys 16ks + {4hh + 0..3, 8 + 4hh + 0..3}
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const _Float16* vsrc = &Vs[(16 * ks + 4 * hh + vrow) * VST + vcol];
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const h8 va = cat_h4(lds_tr4(vsrc + 32 * db), lds_tr4(vsrc + 8 * VST + 32 * db));
                o[db] = mfma32x32x16(va, pb[ks], o[db]);
            }
        }
        __syncthreads();
    }
    // ---- out = O / l * sigmoid(gate): lane holds query c, dims 32db + 8*(i/4) + 4hh + (i&3)
    if (!rvalid) return;
    const float inv = 1.0f / l_run;
    const float* gate = q + (size_t)t * qts + (size_t)head * 2 * HD + HD;
    float* dst = out + (size_t)t * ots + (size_t)head * HD;
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const int d0 = 32 * db + 8 * i4 + 4 * hh;
            const f4 gt = ld_f4(gate + d0);
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = o[db][4 * i4 + j] * inv * sigmoidf_(gt[j]);
            *(f4*)(dst + d0) = v;
        }
}

hipError_t launch_attn_flash(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                             int nh, int nkv, int nt, float scale, float* out, int ots, hipStream_t st) {
    const int R = nt * (nh / nkv);
    const dim3 grid((R + BM - 1) / BM, nkv);
    attn_flash_kernel<<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots);
    return hipGetLastError();
}

}  // namespace it
