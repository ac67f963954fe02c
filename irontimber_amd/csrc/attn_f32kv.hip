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

// Workgroup = (key split s, KV head kh, group of tpw tokens); 4 waves. Query rows: r = lt*G + g for
// the group's token lt and the KV head's q-head g (G = nh/nkv, tpw*G <= 16). Wave w takes keys
// 16w..16w+15 of every 64-key tile of the split and runs its own online softmax; the four waves
// are merged through LDS at the end and one record per (token, q-head) row is written:
// part[((t*nh + h)*smax + s)*260] = {m, l, 0, 0, o[256]}, m in natural-log units.
//
// Each wave stages its own 16 K rows and 16 V rows in LDS with global_load_lds (one coalesced
// 1 KB row per instruction, nothing held in VGPRs while in flight); rows are padded to 260 floats
// so the 16 lanes of a quarter-wave reading 16 rows at one column hit distinct banks. No other
// wave reads them, so a wave-local wait replaces a barrier.
constexpr int F32KV_ROW = F32KV_HD + 4;                 // padded LDS row (floats)
constexpr int F32KV_WAVE = 2 * 16 * F32KV_ROW;          // K then V rows of one wave
#define IT_F32KV_WAIT_VMCNT0() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")
#define IT_F32KV_WAIT_VMCNT16() asm volatile("s_waitcnt vmcnt(16)" ::: "memory")

__global__ __launch_bounds__(256) void attn_f32kv_kernel(const float* __restrict__ q, int qts,
                                                         const float* __restrict__ kc, const float* __restrict__ vc,
                                                         int kvd, int pos0, int nh, int nkv, int nt, int tpw,
                                                         float qscale, float* __restrict__ part, int chunk, int smax) {
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ float ml[4][2][16];
    __shared__ __attribute__((aligned(16))) float smem[4 * F32KV_WAVE];   // tile staging, then the merge
    const int s = blockIdx.x, kh = blockIdx.y, t0 = blockIdx.z * tpw;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
    const int G = nh / nkv;
    const int ntg = min(tpw, nt - t0);
    const int rows = ntg * G;
    const int kb0 = s * chunk;
    const int kend = min(kb0 + chunk, pos0 + t0 + ntg);   // keys the group's last token sees
    if (kb0 >= kend) return;   // whole workgroup: no token of the group sees this split
    const int total = pos0 + nt;
    float* Kw = smem + w * F32KV_WAVE;
    float* Vw = Kw + 16 * F32KV_ROW;

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
    // 16*jj + 4*lg .. +3 of its key row (A) and of its query row (B).
    const bool rv = lr < rows;
    const int tq = t0 + (rv ? lr / G : 0), hq = kh * G + (rv ? lr % G : 0);
    const int nvis = pos0 + tq + 1;   // keys visible to this row
    const float* qp = q + (size_t)tq * qts + (size_t)hq * 2 * F32KV_HD + 4 * lg;
    const float qs = rv ? qscale : 0.f;   // padding rows: a valid row's load, scaled to zero
    f4 qv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) qv[j] = ld_f4(qp + 16 * j) * qs;
    stage_v(kb0);

    float m_run = -1e30f, l_run = 0.f;   // log2 units; finite floor keeps fully masked blocks NaN-free
    f4 acc[16];                          // O^T blocks (dq, e): dims 16*lg + 4*ii + 64*dq + e of row lr
#pragma unroll
    for (int b = 0; b < 16; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};

    for (int kt = kb0; kt < kend; kt += F32KV_KEYS) {
        if (kt != kb0) {
            stage_k(kt);
            stage_v(kt);
        }
        IT_F32KV_WAIT_VMCNT16();   // K rows (and q): the 16 V loads may still fly
        // S^T block: element i = key kt + 16w + 4lg + i, query row lr (4 independent chains).
        f4 sa[4] = {};
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const f4 kf = *(const f4*)(Kw + lr * F32KV_ROW + 16 * jj + 4 * lg);
#pragma unroll
            for (int c = 0; c < 4; ++c) sa[c] = mfma16x16x4f32(kf[c], qv[jj][c], sa[c]);
        }
        f4 sc = (sa[0] + sa[1]) + (sa[2] + sa[3]);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = kt + 16 * w + 4 * lg + i;
            sc[i] = key < nvis ? sc[i] : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = max_xor32(max_xor16(mx));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = exp2f(m_run - m_new);
        f4 p;
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = exp2f(sc[i] - m_new);
            ps += p[i];
        }
        l_run = l_run * alpha + sum_xor32(sum_xor16(ps));
        m_run = m_new;
        IT_F32KV_WAIT_VMCNT0();   // V rows
        // O^T += V^T P^T: MFMA i takes key 4lg + i of the block (its A element from V, its B element
        // this lane's p[i]); output block b = (dq, e) holds dims 16lg + 4ii + 64dq + e.
#pragma unroll
        for (int dq = 0; dq < 4; ++dq) {
            f4 vv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = *(const f4*)(Vw + (4 * lg + i) * F32KV_ROW + 4 * lr + 64 * dq);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f4 o = acc[4 * dq + e] * alpha;
#pragma unroll
                for (int i = 0; i < 4; ++i) o = mfma16x16x4f32(vv[i][e], p[i], o);
                acc[4 * dq + e] = o;
            }
        }
        // The next tile's DMA overwrites this wave's rows: every lane's LDS reads must be done.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // Merge the four waves (each saw a different quarter of every tile) and write the records.
    if (lg == 0) {
        ml[w][0][lr] = m_run;
        ml[w][1][lr] = l_run;
    }
    __syncthreads();   // also: every wave is done with its staging rows, which Os reuses
    f4* Os = (f4*)smem;   // [4][16][65] f4: +1 per row staggers the rows across banks
    const float M = fmaxf(fmaxf(ml[0][0][lr], ml[1][0][lr]), fmaxf(ml[2][0][lr], ml[3][0][lr]));
    const float f = exp2f(m_run - M);
#pragma unroll
    for (int dq = 0; dq < 4; ++dq)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            // block (dq, e) element ii: dim 16lg + 4ii + 64dq + e, e = 0..3 -> one f4
            const f4 o = f4{acc[dq * 4 + 0][ii], acc[dq * 4 + 1][ii], acc[dq * 4 + 2][ii], acc[dq * 4 + 3][ii]} * f;
            Os[(w * 16 + lr) * 65 + (16 * lg + 4 * ii + 64 * dq) / 4] = o;
        }
    __syncthreads();
    // Thread -> (row r = tid >> 4, dims 16*(tid & 15) .. +15).
    const int r = threadIdx.x >> 4, c4 = (threadIdx.x & 15) * 4;
    if (r >= rows) return;
    const float Mr = fmaxf(fmaxf(ml[0][0][r], ml[1][0][r]), fmaxf(ml[2][0][r], ml[3][0][r]));
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) L += ml[ww][1][r] * exp2f(ml[ww][0][r] - Mr);
    const int tr = t0 + r / G, hr = kh * G + r % G;
    float* rec = part + ((size_t)(tr * nh + hr) * smax + s) * 260;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const f4 o = Os[(0 * 16 + r) * 65 + c4 + c] + Os[(1 * 16 + r) * 65 + c4 + c] + Os[(2 * 16 + r) * 65 + c4 + c] +
                     Os[(3 * 16 + r) * 65 + c4 + c];
        *(f4*)(rec + 4 + 4 * (c4 + c)) = o;
    }
    if ((threadIdx.x & 15) == 0) *(f4*)rec = f4{Mr * 0.69314718055994530942f, L, 0.f, 0.f};
}

hipError_t launch_attn_f32kv(const float* q, int qts, const float* kc, const float* vc, int kvd, int pos0, int nh,
                             int nkv, int nt, float scale, float* out, int ots, float* part, int chunk, hipStream_t st) {
    const int G = nh / nkv;
    const int tpw = 16 / G;
    const int smax = (pos0 + nt + chunk - 1) / chunk;
    const dim3 grid((unsigned)smax, (unsigned)nkv, (unsigned)((nt + tpw - 1) / tpw));
    attn_f32kv_kernel<<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, tpw,
                                            scale * 1.44269504088896340736f, part, chunk, smax);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, st);
}

}  // namespace it
