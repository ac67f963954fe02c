// Split-K attention over an f32 KV cache (the MTP head's own cache), f32 matrix cores.
//
// The MTP head keeps its K/V in f32 (src/mtp.rs:96-129 on the CPU; src/vk/mod.rs:942 dispatches the
// non-f16 attention, i.e. attn_s + attn_comb, kernels/src/lib.rs:682-740). The arithmetic is the
// same softmax attention as the f16 path; the partial records have the same 260-float layout, so
// the f16 path's combine kernel merges them.
//
// gfx950 f32 matrix rate (v_mfma_f32_16x16x4_f32, ~256 flop/clk/CU) is twice the non-packed VALU
// rate and the products are exact f32, so both products run on the matrix cores:
//   S^T = K . Q^T      A = K (16 keys x 4 dims), B = Q^T (4 dims x 16 query rows)
//   O^T += V^T . P^T   A = V^T (16 dims x 4 keys), B = P^T (4 keys x 16 query rows)
// K and V reach the operands through LDS (see the kernel). In both products lane l's D column is
// query row l & 15, so each lane owns one query row: the running
// max, sum and rescale of the online softmax are lane-local, with the 16 keys of a wave's block
// reduced across the four 16-lane groups by permlane swaps.
#include "common.h"
#include "internal.h"

namespace it {

namespace {

constexpr int F32KV_HD = 256;
constexpr int F32KV_KEYS = 64;   // keys per tile: 16 per wave

__device__ __forceinline__ f4 mfma16x16x4f32(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}


}  // namespace

// Workgroup = (key split s, KV head kh, group of tpw tokens); 4 waves; RB blocks of 16 query rows
// (rows r = lt*G + g for the group's token lt and the KV head's q-head g, G = nh/nkv,
// tpw*G <= 16*RB). Per 64-key tile:
//   scores  wave w: keys 16w .. 16w+15 against every row (its own 16 K rows, staged by itself);
//   softmax the rows' tile maximum across the four waves through LDS (barrier 1); each wave
//           writes its P (16 keys x rows) and its partial row sums to LDS (barrier 2, after which
//           every wave's V rows have landed too);
//   P.V     wave w: output dims 64w .. 64w+63 over all 64 keys (A = V^T from every wave's V rows,
//           B = P^T from LDS).
// Every wave then holds the same running max and sum and its own quarter of the dims, so the
// record part[((t*nh + h)*smax + s)*260] = {m, l, 0, 0, o[256]} (m in natural-log units) goes out
// straight from the accumulators, with no merge of the waves. RB = 2 (multi-token calls) makes
// each K/V tile serve 32 rows: the 64-token catch-up reads the cache 16 times instead of 32.
//
// Each wave stages its own 16 K rows and 16 V rows in LDS with global_load_lds (one coalesced
// 1 KB row per instruction, nothing held in VGPRs while in flight); rows are padded to 260 floats
// so the 16 lanes of a quarter-wave reading 16 rows at one column hit distinct banks.
constexpr int F32KV_ROW = F32KV_HD + 4;                 // padded LDS row (floats)
#define IT_F32KV_WAIT_VMCNT0() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")
#define IT_F32KV_WAIT_VMCNT16() asm volatile("s_waitcnt vmcnt(16)" ::: "memory")

//
// DIRECT (one pass, no scratch): the grid has one split covering every key, so instead of a record
// each row's final output o / l * sigmoid(gate) is written straight to out[t*ots + h*256 + d]. This
// is the fallback for a caller whose scratch cannot hold even one record per (token, head), the
// role of the reference's whole-context `attn` kernel (kernels/src/lib.rs:83-116, chosen at
// src/vk/mod.rs:740).
// CR: the same values in the piece layout of common.h (decode and short verify calls whose merge is
// the wave merge).
template <int RB, bool DIRECT, bool CR = false>
__global__ __launch_bounds__(256) void attn_f32kv_kernel(const float* __restrict__ q, int qts,
                                                         const float* __restrict__ kc, const float* __restrict__ vc,
                                                         int kvd, int pos0, int nh, int nkv, int nt, int tpw,
                                                         float qscale, float* __restrict__ part, int chunk, int smax,
                                                         float* __restrict__ out, int ots) {
    typedef __attribute__((address_space(3))) void lds_void;
    constexpr int NR = 16 * RB;                                   // query rows per workgroup
    __shared__ __attribute__((aligned(16))) float Ks[F32KV_KEYS * F32KV_ROW];
    __shared__ __attribute__((aligned(16))) float Vs[F32KV_KEYS * F32KV_ROW];
    __shared__ float Ps[F32KV_KEYS][NR];                          // P of the tile, [key][row]
    __shared__ float mxs[4][NR], pss[4][NR];                      // per wave: row max, row sum
    const int s = blockIdx.x, kh = blockIdx.y, t0 = blockIdx.z * tpw;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
    const int G = nh / nkv;
    const int ntg = min(tpw, nt - t0);
    const int rows = ntg * G;
    const int kb0 = s * chunk;
    const int kend = min(kb0 + chunk, pos0 + t0 + ntg);   // keys the group's last token sees
    if (kb0 >= kend) return;   // whole workgroup: no token of the group sees this split
    const int total = pos0 + nt;
    float* Kw = Ks + 16 * w * F32KV_ROW;
    float* Vw = Vs + 16 * w * F32KV_ROW;

    // This wave's 16 K and V rows of tile kt (keys kt + 16w + r), lane l bringing dims 4l .. 4l+3.
    // K rows first, V rows after: the scores and the softmax only wait for the K rows (16 loads
    // older than the 16 V loads), so they run while V lands.
    auto stage_k = [&](int kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const size_t row = (size_t)min(kt + 16 * w + r, total - 1) * kvd + (size_t)kh * F32KV_HD + 4 * l;
            __builtin_amdgcn_global_load_lds(kc + row, (lds_void*)(Kw + r * F32KV_ROW), 16, 0, 0);
        }
    };
    auto stage_v = [&](int kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const size_t row = (size_t)min(kt + 16 * w + r, total - 1) * kvd + (size_t)kh * F32KV_HD + 4 * l;
            __builtin_amdgcn_global_load_lds(vc + row, (lds_void*)(Vw + r * F32KV_ROW), 16, 0, 0);
        }
    };
    stage_k(kb0);   // the first tile's K rows are in flight while q loads below

    // Score product j = 4*jj + c contracts dims {16*jj + 4*lg + c : lg = 0..3}: lane l holds dims
    // 16*jj + 4*lg .. +3 of its key row (A) and of its query row (B), for each row block.
    int nvis[RB];
    f4 qv[RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * rb + lr;
        const bool rv = r < rows;
        const int tq = t0 + (rv ? r / G : 0), hq = kh * G + (rv ? r % G : 0);
        nvis[rb] = pos0 + tq + 1;   // keys visible to this row
        const float* qp = q + (size_t)tq * qts + (size_t)hq * 2 * F32KV_HD + 4 * lg;
        const float qs = rv ? qscale : 0.f;   // padding rows: a valid row's load, scaled to zero
#pragma unroll
        for (int j = 0; j < 16; ++j) qv[rb][j] = ld_f4(qp + 16 * j) * qs;
    }
    stage_v(kb0);

    float m_run[RB], l_run[RB];   // log2 units; a finite floor keeps fully masked rows NaN-free
    f4 acc[RB][4];                // O^T block e of row block rb: dims 64w + 4*(4lg + i) + e of row lr
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        m_run[rb] = -1e30f;
        l_run[rb] = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[rb][e] = f4{0.f, 0.f, 0.f, 0.f};
    }

    for (int kt = kb0; kt < kend; kt += F32KV_KEYS) {
        const bool more = kt + F32KV_KEYS < kend;
        if (kt != kb0) {
            __syncthreads();   // every wave is done with the previous tile's V and P
            stage_v(kt);       // (its K rows were staged during the previous tile)
        }
        IT_F32KV_WAIT_VMCNT16();   // K rows (and q): the 16 V loads may still fly
        // S^T block: element i = key kt + 16w + 4lg + i, query row lr of block rb.
        f4 sc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            f4 sa[2] = {};
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const f4 kf = *(const f4*)(Kw + lr * F32KV_ROW + 16 * jj + 4 * lg);
#pragma unroll
                for (int c = 0; c < 4; ++c) sa[c & 1] = mfma16x16x4f32(kf[c], qv[rb][jj][c], sa[c & 1]);
            }
            sc[rb] = sa[0] + sa[1];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kt + 16 * w + 4 * lg + i;
                sc[rb][i] = key < nvis[rb] ? sc[rb][i] : -INFINITY;
                mx = fmaxf(mx, sc[rb][i]);
            }
            mx = max_xor32(max_xor16(mx));
            if (lg == 0) mxs[w][16 * rb + lr] = mx;
        }
        // the next tile's K rows go out now: a wave's scores read only its own 16 K rows, so once
        // they are done its rows can be refilled (no barrier), and the rows land during this
        // tile's softmax and P.V instead of after the next tile's barrier
        if (more) stage_k(kt + F32KV_KEYS);
        __syncthreads();   // the four waves' row maxima
        float alpha[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = 16 * rb + lr;
            const float mt = fmaxf(fmaxf(mxs[0][r], mxs[1][r]), fmaxf(mxs[2][r], mxs[3][r]));
            const float m_new = fmaxf(m_run[rb], mt);
            alpha[rb] = exp2f(m_run[rb] - m_new);
            m_run[rb] = m_new;
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = exp2f(sc[rb][i] - m_new);
                ps += p;
                Ps[16 * w + 4 * lg + i][r] = p;
            }
            ps = sum_xor32(sum_xor16(ps));
            if (lg == 0) pss[w][r] = ps;
        }
        // this wave's V rows (issued before the next tile's 16 K loads, which may still fly)
        if (more) IT_F32KV_WAIT_VMCNT16();
        else IT_F32KV_WAIT_VMCNT0();
        __syncthreads();          // every wave's P, row sums and V rows
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = 16 * rb + lr;
            l_run[rb] = l_run[rb] * alpha[rb] + ((pss[0][r] + pss[1][r]) + (pss[2][r] + pss[3][r]));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[rb][e] *= alpha[rb];
        }
        // O^T += V^T P^T, key quad kq: MFMA A element = V[4kq + lg][64w + 4lr + e] (one f4 read
        // gives the four blocks e), B element = P[4kq + lg][row lr of block rb].
#pragma unroll
        for (int kq = 0; kq < 16; ++kq) {
            const f4 vv = *(const f4*)(Vs + (4 * kq + lg) * F32KV_ROW + 64 * w + 4 * lr);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const float pb = Ps[4 * kq + lg][16 * rb + lr];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[rb][e] = mfma16x16x4f32(vv[e], pb, acc[rb][e]);
            }
        }
    }

    // Records straight from the accumulators: lane (lr, lg) holds dims 64w + 16lg + 4i + e
    // (e = 0..3 contiguous) of row 16rb + lr; wave 0 adds the headers.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * rb + lr;
        if (r >= rows) continue;
        const int tr = t0 + r / G, hr = kh * G + r % G;
        if constexpr (DIRECT) {
            // every visible row has seen at least key 0, so l_run > 0
            const float inv = 1.0f / l_run[rb];
            const float* gate = q + (size_t)tr * qts + (size_t)hr * 2 * F32KV_HD + F32KV_HD;
            float* orow = out + (size_t)tr * ots + (size_t)hr * F32KV_HD;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 64 * w + 16 * lg + 4 * i;
                const f4 g = ld_f4(gate + d);
                f4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = acc[rb][e][i] * inv * sigmoidf_(g[e]);
                *(f4*)(orow + d) = o;
            }
            continue;
        }
        if constexpr (CR) {   // the piece layout: this lane's 16 dims are piece (row, 4w + lg)
            const int th = tr * nh + hr;
            float* pc = prec_o(part, th, 4 * w + lg, s, smax);
#pragma unroll
            for (int i = 0; i < 4; ++i) *(f4*)(pc + 4 * i) = f4{acc[rb][0][i], acc[rb][1][i], acc[rb][2][i], acc[rb][3][i]};
            if (w == 0 && lg == 0) *(f2*)prec_h(part, nt * nh, th, s, smax) = f2{m_run[rb] * 0.69314718055994530942f, l_run[rb]};
            continue;
        }
        float* rec = part + idx::rec(tr * nh + hr, s, smax) * idx::PART;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *(f4*)(rec + 4 + 64 * w + 16 * lg + 4 * i) = f4{acc[rb][0][i], acc[rb][1][i], acc[rb][2][i], acc[rb][3][i]};
        if (w == 0 && lg == 0) *(f4*)rec = f4{m_run[rb] * 0.69314718055994530942f, l_run[rb], 0.f, 0.f};
    }
}

hipError_t launch_attn_f32kv(const float* q, int qts, const float* kc, const float* vc, int kvd, int pos0, int nh,
                             int nkv, int nt, float scale, float* out, int ots, float* part, int chunk, hipStream_t st) {
    const int G = nh / nkv;
    const bool direct = chunk == 0;   // one pass over every key, output written directly, no records
    if (direct) chunk = pos0 + nt;
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    const float qs = scale * 1.44269504088896340736f;
    // two 16-row blocks per workgroup once a call has more rows than one block holds
    const int rb = nt * G > 16 ? 2 : 1;
    const int tpw = 16 * rb / G;
    // the piece layout for the wave merge (one 16-row block: decode and short verify calls)
    const bool pieces = !direct && rb == 1 && piece_records(pos0, nt, nh, chunk);
    const dim3 grid((unsigned)smax, (unsigned)nkv, (unsigned)((nt + tpw - 1) / tpw));
    if (rb == 2 && direct)
        attn_f32kv_kernel<2, true><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw, qs, part, chunk,
                                                        smax, out, ots);
    else if (rb == 2)
        attn_f32kv_kernel<2, false><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw, qs, part, chunk,
                                                         smax, out, ots);
    else if (direct)
        attn_f32kv_kernel<1, true><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw, qs, part, chunk,
                                                        smax, out, ots);
    else if (pieces)
        attn_f32kv_kernel<1, false, true><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw, qs, part,
                                                               chunk, smax, out, ots);
    else
        attn_f32kv_kernel<1, false><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw, qs, part, chunk,
                                                         smax, out, ots);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || direct) return e;
    return launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, st, pieces);
}

}  // namespace it
