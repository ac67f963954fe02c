// Gated DeltaNet for gfx950: depthwise causal conv + SiLU, per-head L2 norm, and the gated-delta
// recurrence for decode / short token runs with the state held in registers.
//
// Reference behaviour: src/cpu.rs:201-232 (math), kernels/src/lib.rs:119-140 (conv),
// 207-229 (rmsnorm mode 2), 252-331 (gdn, gdn_p).
#include "common.h"
#include "internal.h"

namespace it {

// ------------------------------------------------------------------------------------------------
// Conv: thread per (channel, run of TT tokens). The K-1 inputs before the run come from x or, for
// tokens before 0, from the carried state (oldest first). With one run (grid.y == 1) the same
// thread also writes the new state; otherwise gdn_conv_state_kernel does it after this kernel.
// ck (optional): with one run, the state after token ck_after is written there from the window
// (the MTP verify checkpoint); with several runs the host launches gdn_conv_state_kernel for it
// before this kernel instead.
// TMAX: the longest run the kernel is built for (1, 2, 4 or 16; the host passes TT <= TMAX), so a
// decode or verify launch loads no inputs for tokens it does not have.
template <int K, int TMAX>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const float* __restrict__ x, int xts, const float* __restrict__ w,
                                                       float* __restrict__ state, float* __restrict__ out, int ots,
                                                       int cd, int nt, int TT, float* __restrict__ ck, int ck_after) {
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= cd) return;
    const int t0 = blockIdx.y * TT, n = min(nt, t0 + TT) - t0;
    // the run's inputs are all loaded before any is used: one memory round trip per run
    float xs[TMAX], wt[K], win[K - 1];
#pragma unroll
    for (int j = 0; j < TMAX; ++j) xs[j] = x[(size_t)(t0 + min(j, n - 1)) * xts + ch];
#pragma unroll
    for (int i = 0; i < K; ++i) wt[i] = w[(size_t)ch * K + i];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
        const int tt = t0 - (K - 1) + i;
        win[i] = tt >= 0 ? x[(size_t)tt * xts + ch] : state[(size_t)(tt + K - 1) * cd + ch];
    }
#pragma unroll
    for (int j = 0; j < TMAX; ++j) {
        if (j >= n) continue;
        const int t = t0 + j;
        const float xv = xs[j];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < K - 1; ++i) s += win[i] * wt[i];
        s += xv * wt[K - 1];
        out[(size_t)t * ots + ch] = siluf_(s);
#pragma unroll
        for (int i = 0; i + 1 < K - 1; ++i) win[i] = win[i + 1];
        win[K - 2] = xv;
        if (ck && t == ck_after && gridDim.y == 1) {
#pragma unroll
            for (int i = 0; i < K - 1; ++i) ck[(size_t)i * cd + ch] = win[i];
        }
    }
    if (gridDim.y == 1) {
#pragma unroll
        for (int i = 0; i < K - 1; ++i) state[(size_t)i * cd + ch] = win[i];
    }
}

// The conv state after the first nt tokens, from the state before them and x, written to dst
// (dst == state: the state update after a multi-run conv; dst != state: a checkpoint).
template <int K>
__global__ __launch_bounds__(256) void gdn_conv_state_kernel(const float* __restrict__ x, int xts, const float* state,
                                                             float* dst, int cd, int nt) {
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= cd) return;
    float nv[K - 1];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
        const int tt = nt - (K - 1) + i;
        nv[i] = tt >= 0 ? x[(size_t)tt * xts + ch] : state[(size_t)(tt + K - 1) * cd + ch];
    }
#pragma unroll
    for (int i = 0; i < K - 1; ++i) dst[(size_t)i * cd + ch] = nv[i];
}

// ------------------------------------------------------------------------------------------------
// Conv + SiLU with the per-head L2 norm fused (one pass over the activations instead of two).
// Wave = (128-channel head block hb, run of TT tokens); lane l holds channels 128hb + l and
// 128hb + 64 + l, so a token's head vector is the whole wave and its sum of squares one DPP
// reduction. Head blocks hb < nnorm (the q and k heads) are normalised, x / max(||x||, eps); the
// rest (v) pass through. State and checkpoint handling as in gdn_conv_kernel.
template <int K, typename OutT, int TMAX>   // TMAX as in gdn_conv_kernel
__global__ __launch_bounds__(256) void gdn_conv_l2_kernel(const float* __restrict__ x, int xts,
                                                          const float* __restrict__ w, float* __restrict__ state,
                                                          OutT* __restrict__ out, int ots, int cd, int nt, int TT,
                                                          int nnorm, float eps, float* __restrict__ ck, int ck_after) {
    const int hb = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (hb >= cd / 128) return;   // whole waves
    const bool norm = hb < nnorm;
    const int t0 = blockIdx.y * TT, n = min(nt, t0 + TT) - t0;
    int ch[2] = {128 * hb + l, 128 * hb + 64 + l};
    // Every input of the run is loaded before any is used (one memory round trip per run instead
    // of one per token): the run's tokens (clamped to the last one), the K-1 inputs before it and
    // the weights.
    float xs[2][TMAX], wt[2][K], win[2][K - 1];
#pragma unroll
    for (int j = 0; j < TMAX; ++j) {
        const size_t row = (size_t)(t0 + min(j, n - 1)) * xts;
#pragma unroll
        for (int c = 0; c < 2; ++c) xs[c][j] = x[row + ch[c]];
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int i = 0; i < K; ++i) wt[c][i] = w[(size_t)ch[c] * K + i];
#pragma unroll
        for (int i = 0; i < K - 1; ++i) {
            const int tt = t0 - (K - 1) + i;
            win[c][i] = tt >= 0 ? x[(size_t)tt * xts + ch[c]] : state[(size_t)(tt + K - 1) * cd + ch[c]];
        }
    }
#pragma unroll
    for (int j = 0; j < TMAX; ++j) {
        if (j >= n) continue;   // wave-uniform; keeps the loop fully unrollable
        float y[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < K - 1; ++i) s += win[c][i] * wt[c][i];
            s += xs[c][j] * wt[c][K - 1];
            y[c] = silu_hw(s);
        }
        if (norm) {
            const float sc = 1.0f / fmaxf(sqrtf(wave_sum(y[0] * y[0] + y[1] * y[1])), eps);
            y[0] *= sc;
            y[1] *= sc;
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            out[(size_t)(t0 + j) * ots + ch[c]] = (OutT)y[c];
#pragma unroll
            for (int i = 0; i + 1 < K - 1; ++i) win[c][i] = win[c][i + 1];
            win[c][K - 2] = xs[c][j];
        }
        if (ck && t0 + j == ck_after && gridDim.y == 1) {
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int i = 0; i < K - 1; ++i) ck[(size_t)i * cd + ch[c]] = win[c][i];
        }
    }
    if (gridDim.y == 1) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int i = 0; i < K - 1; ++i) state[(size_t)i * cd + ch[c]] = win[c][i];
    }
}

// The same pass with 16-byte accesses (strides and bases 16-byte aligned, cd % 256 == 0): lane l
// holds channels 256*wb + 4l .. 4l+3 of wave block wb, so lanes 0-31 and 32-63 each hold one
// 128-channel head and a head's sum of squares is a reduction over its 32 lanes (DPP within the
// 16-lane rows, then a row swap). A quarter of the memory instructions of the scalar form.
template <int K, typename OutT>
__global__ __launch_bounds__(256) void gdn_conv_l2_v4_kernel(const float* __restrict__ x, int xts,
                                                             const float* __restrict__ w, float* __restrict__ state,
                                                             OutT* __restrict__ out, int ots, int cd, int nt, int TT,
                                                             int nnorm, float eps, float* __restrict__ ck,
                                                             int ck_after) {
    constexpr int TMAX = 16;   // tokens per run (the host passes TT <= TMAX)
    const int wb = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (wb >= cd / 256) return;   // whole waves
    const int ch = 256 * wb + 4 * l;
    const bool norm = (ch >> 7) < nnorm;   // uniform over each 32-lane half
    const int t0 = blockIdx.y * TT, n = min(nt, t0 + TT) - t0;
    f4 xs[TMAX], wt[K], win[K - 1];
#pragma unroll
    for (int j = 0; j < TMAX; ++j) xs[j] = ld_f4(x + (size_t)(t0 + min(j, n - 1)) * xts + ch);
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // taps of channel ch + e are w[(ch + e) * K .. + K)
#pragma unroll
        for (int i = 0; i < K; ++i) wt[i][e] = w[(size_t)(ch + e) * K + i];
    }
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
        const int tt = t0 - (K - 1) + i;
        win[i] = tt >= 0 ? ld_f4(x + (size_t)tt * xts + ch) : ld_f4(state + (size_t)(tt + K - 1) * cd + ch);
    }
#pragma unroll
    for (int j = 0; j < TMAX; ++j) {
        if (j >= n) continue;   // wave-uniform; keeps the loop fully unrollable
        f4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < K - 1; ++i) acc += win[i][e] * wt[i][e];
            acc += xs[j][e] * wt[K - 1][e];
            y[e] = silu_hw(acc);
        }
        float ss = y[0] * y[0] + y[1] * y[1] + y[2] * y[2] + y[3] * y[3];
        ss += dppc<0xB1>(ss);    // quad_perm [1,0,3,2]
        ss += dppc<0x4E>(ss);    // quad_perm [2,3,0,1]
        ss += dppc<0x141>(ss);   // row_half_mirror
        ss += dppc<0x140>(ss);   // row_mirror
        ss = sum_xor16(ss);      // rows 0+1 and 2+3: the two heads' sums
        if (norm) y *= 1.0f / fmaxf(sqrtf(ss), eps);
        st4(out + (size_t)(t0 + j) * ots + ch, y);
#pragma unroll
        for (int i = 0; i + 1 < K - 1; ++i) win[i] = win[i + 1];
        win[K - 2] = xs[j];
        if (ck && t0 + j == ck_after && gridDim.y == 1) {
#pragma unroll
            for (int i = 0; i < K - 1; ++i) *(f4*)(ck + (size_t)i * cd + ch) = win[i];
        }
    }
    if (gridDim.y == 1) {
#pragma unroll
        for (int i = 0; i < K - 1; ++i) *(f4*)(state + (size_t)i * cd + ch) = win[i];
    }
}

// ------------------------------------------------------------------------------------------------
// L2 norm of rows of D floats, one wave per row, in place: x / max(||x||, eps).
template <int D>
__global__ __launch_bounds__(256) void l2norm_kernel(float* __restrict__ x, int ts, int nheads, int nt, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (row >= nheads * nt) return;
    const int t = row / nheads, r = row % nheads;
    float* p = x + (size_t)t * ts + (size_t)r * D;
    constexpr int PER = D / 64;
    float v[PER];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) { v[i] = p[l + 64 * i]; ss += v[i] * v[i]; }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) ss += __shfl_xor(ss, m);
    const float sc = 1.0f / fmaxf(sqrtf(ss), eps);
#pragma unroll
    for (int i = 0; i < PER; ++i) p[l + 64 * i] = v[i] * sc;
}

// ------------------------------------------------------------------------------------------------
// Gated-delta recurrence, S = 128, token-sequential with the state slice in registers.
// Workgroup = (16-column block cb, V head h); thread = (column quad cg = tid & 3, row pair
// rp = tid >> 2): it holds S[2rp..2rp+1][16cb+4cg .. +3]. Column sums over the 128 rows reduce
// across lanes (xor 4..32) and then across the 4 waves through LDS.
// ck (optional): the state after token ck_after is also written there, straight from the
// registers (the MTP verify checkpoint; no second pass over the state).
// Sum over the 16 lanes of a wave that share l & 3 (lane bits 2-5), every lane receiving its
// group's sum: two DPP row rotates (by 4 and 8) sum within each 16-lane row, then the rows are
// added by swapping lane halves (v_permlane16_swap, then v_permlane32_swap). No LDS traffic.
__device__ __forceinline__ float rowsum_stride4(float v) {
    v += dppc<0x124>(v);   // row_ror:4
    v += dppc<0x128>(v);   // row_ror:8
    return v;
}
__device__ __forceinline__ float sum_lanes_stride4(float v) { return sum_xor32(sum_xor16(rowsum_stride4(v))); }
// The wave's column sums of p and r (4 columns each) with 6 swaps instead of 16: row sums, then
// (p_j, r_j) folded over row pairs and (j, j + 1) over the wave halves. Lane l of row rho = l >> 4
// ends with, for its column group l & 3, the sums of (rho & 1 ? r : p) elements rho >> 1 (u0) and
// 2 + (rho >> 1) (u1).
__device__ __forceinline__ void colsums_pr(f4 p, f4 r, float& u0, float& u1) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = fold16(rowsum_stride4(p[j]), rowsum_stride4(r[j]));
    u0 = fold32(t[0], t[1]);
    u1 = fold32(t[2], t[3]);
}

// Workgroup id -> (16-column block cb, V head h) of the 8 x nv step grid, launched 1-D.
// Workgroups go to the 8 XCDs round-robin by id, each XCD with its own L2; the two column blocks
// that share every 128-byte state line get ids 8 apart (the same XCD), so each line is fetched
// from HBM once instead of once per block. Needs nv even; odd nv keeps the plain order.
__device__ __forceinline__ void step_wg(int id, int nv, int& cb, int& h) {
    if (nv & 1) { cb = id & 7; h = id >> 3; return; }
    const int xcd = id & 7, slot = id >> 3;
    const int u = ((slot >> 1) << 3) | xcd;   // (head, column-block pair)
    h = u >> 2;
    cb = 2 * (u & 3) + (slot & 1);
}

__global__ __launch_bounds__(256) void gdn_step_kernel(const float* __restrict__ co, int cts, const float* __restrict__ br,
                                                       const float* __restrict__ ar, int bts, const float* __restrict__ dt,
                                                       const float* __restrict__ A, float* __restrict__ state,
                                                       float* __restrict__ out, int ots, int nt, int nv, int nk,
                                                       float* __restrict__ ck, int ck_after) {
    constexpr int S = 128;
    // per token parity: {S^T k, S^T q} column sums of each wave, and its k.q
    __shared__ f4 red[2][4][2][4];
    __shared__ float rkq[2][4];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    int cb, h;
    step_wg(blockIdx.x, nv, cb, h);
    const int cg = tid & 3, rp = tid >> 2;
    const int kh = h % nk, qk = nk * S;
    const int j0 = cb * 16 + 4 * cg, i0 = 2 * rp;
    float* sb = state + (size_t)h * S * S;
    f4 s0 = ld_f4(sb + (size_t)i0 * S + j0), s1 = ld_f4(sb + (size_t)(i0 + 1) * S + j0);
    const float scale = 1.0f / sqrtf((float)S);
    const float dth = dt[h], ah = A[h];
    // token inputs one token ahead: token t + 1's loads are issued before token t's barriers, so a
    // run of tokens waits for memory once instead of once per token
    struct Tok { float q0, q1, k0, k1; f4 v; float b, a; };
    auto load_tok = [&](int t) {
        const float* c = co + (size_t)t * cts;
        Tok r;
        r.q0 = c[kh * S + i0];
        r.q1 = c[kh * S + i0 + 1];
        r.k0 = c[qk + kh * S + i0];
        r.k1 = c[qk + kh * S + i0 + 1];
        r.v = ld_f4(c + 2 * qk + h * S + j0);
        r.b = br[(size_t)t * bts + h];
        r.a = ar[(size_t)t * bts + h];
        return r;
    };
    // one token: decay, the fused exchange, the update; the output row (threads tid < 4) in o4
    auto step = [&](int t, const Tok& cur, f4& o4) {
        const float q0 = cur.q0, q1 = cur.q1, k0 = cur.k0, k1 = cur.k1;
        const f4 v = cur.v;
        const float beta = sigmoid_hw(cur.b);
        const float eg = exp_hw(softplus_hw(cur.a + dth) * ah);
        s0 *= eg; s1 *= eg;
        // With S' = S + k delta^T (S already decayed), S'^T q = S^T q + (k.q) delta: S^T k, S^T q
        // and k.q reduce together, one exchange and one barrier a token. The parity-indexed
        // buffers are rewritten two tokens later, after every wave has passed the next barrier.
        float u0, u1;
        colsums_pr(s0 * k0 + s1 * k1, s0 * q0 + s1 * q1, u0, u1);
        const float kq = sum_lanes_stride4(k0 * q0 + k1 * q1);
        const int b = t & 1;
        if ((l & 15) < 4) {
            const int rho = l >> 4;
            float* d = (float*)&red[b][w][rho & 1][cg];
            d[rho >> 1] = u0;
            d[2 + (rho >> 1)] = u1;
        }
        if (l == 0) rkq[b][w] = kq;
        __syncthreads();
        const f4 sk = (red[b][0][0][cg] + red[b][1][0][cg]) + (red[b][2][0][cg] + red[b][3][0][cg]);
        const f4 delta = (v - sk) * beta;
        s0 += k0 * delta; s1 += k1 * delta;
        if (tid < 4) {
            const f4 sq = (red[b][0][1][cg] + red[b][1][1][cg]) + (red[b][2][1][cg] + red[b][3][1][cg]);
            const float kqs = (rkq[b][0] + rkq[b][1]) + (rkq[b][2] + rkq[b][3]);
            o4 = (sq + kqs * delta) * scale;
        }
        if (ck && t == ck_after) {
            float* cb_ = ck + (size_t)h * S * S;
            *(f4*)(cb_ + (size_t)i0 * S + j0) = s0;
            *(f4*)(cb_ + (size_t)(i0 + 1) * S + j0) = s1;
        }
    };
    // Every token but the last in a loop, storing its output there; the last one (nt >= 1) as
    // straight-line code with the state stored before its output row. The load counter also
    // counts stores, and at a loop's merge points the compiler cannot tell which of them a wave
    // issued, so it waits for all: with the decode step inside the loop, the state stores waited
    // for the output store's round trip.
    Tok nx = load_tok(0);
    f4 o4 = {0.f, 0.f, 0.f, 0.f};
    int t = 0;
    for (; t + 1 < nt; ++t) {
        const Tok cur = nx;
        nx = load_tok(t + 1);
        step(t, cur, o4);
        if (tid < 4) *(f4*)(out + (size_t)t * ots + (size_t)h * S + j0) = o4;
    }
    step(t, nx, o4);
    *(f4*)(sb + (size_t)i0 * S + j0) = s0;
    *(f4*)(sb + (size_t)(i0 + 1) * S + j0) = s1;
    if (tid < 4) *(f4*)(out + (size_t)t * ots + (size_t)h * S + j0) = o4;
}

// ------------------------------------------------------------------------------------------------
// Decode layer in one launch: conv + SiLU + q/k L2 norm + recurrence for up to 4 tokens.
// Same workgroup and thread layout as gdn_step_kernel; each thread also runs the conv of the
// channels it consumes (q and k at rows i0, i0+1 of its QK head, v at columns j0..j0+3 of its V
// head) from the old conv state, so no workgroup waits for another. The q/k head norms sum over
// the workgroup (each row pair is held by the 4 threads of a column group: lanes with equal l & 3
// cover 16 distinct rows per wave, then the 4 waves through LDS). The new conv state goes to a
// separate buffer (reading and rewriting one buffer would race between workgroups): q/k channels
// by the first column block of the QK head's first V head, v channels by row pair 0 of each
// workgroup. With one wave per SIMD every instruction is on the critical path, so the activations
// use the hardware exp2 / log2 / reciprocal (a few ulp), and the q/k norms, being per-head scalars,
// are applied after the S k and S^T q sums: their sums of squares share the one exchange of the
// token (one barrier a token). Results agree with conv + L2 + gdn_step_kernel to rounding.
// TM: the tokens of the call (1 to 4; the launch builds the kernel for exactly nt = TM): every
// token's inputs are loaded up front, and the token loop has no exit other than its end, so the
// compiler's load-counter waits need not assume a path that skipped tokens (such a path made the
// state stores wait for the output and checkpoint stores of the earlier tokens).
template <int K, int TM>
__global__ __launch_bounds__(256) void gdn_decode_fused_kernel(
    const float* __restrict__ x, int xts, const float* __restrict__ cw, const float* __restrict__ cst_in,
    float* __restrict__ cst_out, const float* __restrict__ br, const float* __restrict__ ar, int bts,
    const float* __restrict__ dt, const float* __restrict__ A, float* __restrict__ state, float* __restrict__ out,
    int ots, int nt, int nv, int nk, float eps, float* __restrict__ ck_state, float* __restrict__ ck_conv,
    int ck_after) {
    constexpr int S = 128;
    // per token parity, per wave: {S^T k, S^T q} column sums and {sum q^2, sum k^2, k.q} of its
    // 16 row pairs (raw conv outputs, before the head norms)
    __shared__ f4 red[2][4][2][4];
    __shared__ f4 nrm[2][4];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    int cb, h;
    step_wg(blockIdx.x, nv, cb, h);
    const int cg = tid & 3, rp = tid >> 2;
    const int kh = h % nk, qk = nk * S, cd = (2 * nk + nv) * S;
    const int j0 = cb * 16 + 4 * cg, i0 = 2 * rp;
    const int cq = kh * S + i0, ck = qk + kh * S + i0;   // q and k channel bases of row i0
    float* sb = state + (size_t)h * S * S;
    // every load up front: tokens, weights, the conv window, the gates, then the state. The
    // vector-memory counter retires in order, so the conv inputs issued first can be used (the
    // conv, SiLU and norm sums run) while the state slice is still landing.
    // Each lane convolves one q/k channel (by its place cg in the row pair's lane quad: q row i0,
    // q row i0 + 1, k row i0, k row i0 + 1) and one of the workgroup's 16 v channels (lane & 15);
    // the quad's four values reach its lanes by DPP broadcasts and each lane's four v channels by
    // lane shuffles. Loading and convolving all 8 of its channels in every thread (the four lanes of
    // a row pair alike, and all 64 row pairs the same 16 v channels) moved ~64 KB a workgroup
    // through the CU's load path against its 8 KB state slice.
    const int cqk = (cg < 2 ? cq : ck) + (cg & 1);
    const int cvl = 2 * qk + h * S + cb * 16 + (l & 15);
    float xa[TM], xb[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        xa[t] = x[(size_t)t * xts + cqk];
        xb[t] = x[(size_t)t * xts + cvl];
    }
    float wa[K], wb[K];
    if constexpr (K == 4) {   // a channel's taps are one aligned f4
        const f4 a4 = ld_f4(cw + (size_t)cqk * 4), b4 = ld_f4(cw + (size_t)cvl * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { wa[i] = a4[i]; wb[i] = b4[i]; }
    } else {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            wa[i] = cw[(size_t)cqk * K + i];
            wb[i] = cw[(size_t)cvl * K + i];
        }
    }
    float wna[K - 1], wnb[K - 1];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
        wna[i] = cst_in[(size_t)i * cd + cqk];
        wnb[i] = cst_in[(size_t)i * cd + cvl];
    }
    // the gate inputs too: loaded inside the loop they would wait behind the norm barrier
    float brt[TM], art[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        brt[t] = br[(size_t)t * bts + h];
        art[t] = ar[(size_t)t * bts + h];
    }
    const float dth = dt[h], ah = A[h];
    f4 s0 = ld_f4(sb + (size_t)i0 * S + j0), s1 = ld_f4(sb + (size_t)(i0 + 1) * S + j0);
    const float scale = 1.0f / sqrtf((float)S);
    f4 olast = {0.f, 0.f, 0.f, 0.f};   // the last token's output row (threads tid < 4)
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        // ---- conv + SiLU of this lane's two channels, then the exchanges
        float ca = 0.f, cv_ = 0.f;
#pragma unroll
        for (int i = 0; i < K - 1; ++i) { ca += wna[i] * wa[i]; cv_ += wnb[i] * wb[i]; }
        ca += xa[t] * wa[K - 1];
        cv_ += xb[t] * wb[K - 1];
        ca = silu_hw(ca);
        cv_ = silu_hw(cv_);
#pragma unroll
        for (int i = 0; i + 1 < K - 1; ++i) { wna[i] = wna[i + 1]; wnb[i] = wnb[i + 1]; }
        wna[K - 2] = xa[t];
        wnb[K - 2] = xb[t];
        float q[2], k[2];
        q[0] = dppc<0x00>(ca);   // quad_perm [0,0,0,0]: q row i0
        q[1] = dppc<0x55>(ca);   // quad_perm [1,1,1,1]: q row i0 + 1
        k[0] = dppc<0xAA>(ca);   // quad_perm [2,2,2,2]: k row i0
        k[1] = dppc<0xFF>(ca);   // quad_perm [3,3,3,3]: k row i0 + 1
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __shfl(cv_, 4 * cg + e);   // column j0 + e = cb*16 + 4cg + e
        // ---- recurrence (gdn_step_kernel) with the q/k L2 norms folded in. The head norms are
        // scalars fq, fk, so with raw q, k: S^T k-hat = fk S^T k, and with S' = S + k-hat delta^T
        // (S already decayed), S'^T q-hat = fq S^T q + fq fk (k.q) delta. The two column sums, the
        // sums of squares and k.q all ride in one LDS exchange: one barrier a token. The parity-
        // indexed buffers are rewritten two tokens later, after every wave has passed the next barrier.
        const float beta = sigmoid_hw(brt[t]);
        const float eg = exp_hw(softplus_hw(art[t] + dth) * ah);
        s0 *= eg; s1 *= eg;
        float u0, u1;
        colsums_pr(s0 * k[0] + s1 * k[1], s0 * q[0] + s1 * q[1], u0, u1);
        // the three scalars: sum q^2 ends in row 0, sum k^2 in row 1, k.q in rows 2 and 3
        const float sn = fold32(fold16(rowsum_stride4(q[0] * q[0] + q[1] * q[1]),
                                       rowsum_stride4(k[0] * k[0] + k[1] * k[1])),
                                sum_xor16(rowsum_stride4(k[0] * q[0] + k[1] * q[1])));
        const int b = t & 1;
        if ((l & 15) < 4) {
            const int rho = l >> 4;
            float* d = (float*)&red[b][w][rho & 1][cg];
            d[rho >> 1] = u0;
            d[2 + (rho >> 1)] = u1;
        }
        if (l == 0 || l == 16 || l == 32) ((float*)&nrm[b][w])[l >> 4] = sn;
        __syncthreads();
        const f4 n = (nrm[b][0] + nrm[b][1]) + (nrm[b][2] + nrm[b][3]);
        const float fq = 1.0f / fmaxf(sqrtf(n[0]), eps), fk = 1.0f / fmaxf(sqrtf(n[1]), eps);
        const float k0 = k[0] * fk, k1 = k[1] * fk;
        const f4 skv = ((red[b][0][0][cg] + red[b][1][0][cg]) + (red[b][2][0][cg] + red[b][3][0][cg])) * fk;
        const f4 delta = (v - skv) * beta;
        s0 += k0 * delta; s1 += k1 * delta;
        if (tid < 4) {
            const f4 sq4 = (red[b][0][1][cg] + red[b][1][1][cg]) + (red[b][2][1][cg] + red[b][3][1][cg]);
            olast = (sq4 * fq + (fq * fk * n[2]) * delta) * scale;
            // the last token's row goes out after the state (see below)
            if (t + 1 < TM) *(f4*)(out + (size_t)t * ots + (size_t)h * S + j0) = olast;
        }
        if (t == ck_after) {   // MTP verify checkpoint: both states after this token, from registers
            if (ck_state) {
                float* cb_ = ck_state + (size_t)h * S * S;
                *(f4*)(cb_ + (size_t)i0 * S + j0) = s0;
                *(f4*)(cb_ + (size_t)(i0 + 1) * S + j0) = s1;
            }
            if (ck_conv) {
                if (cb == 0 && h == kh) {   // every q/k channel of the head, one per thread
#pragma unroll
                    for (int i = 0; i < K - 1; ++i) ck_conv[(size_t)i * cd + cqk] = wna[i];
                }
                if (tid < 16) {             // the workgroup's 16 v channels
#pragma unroll
                    for (int i = 0; i < K - 1; ++i) ck_conv[(size_t)i * cd + cvl] = wnb[i];
                }
            }
        }
    }
    // the state first: the load counter also counts stores, and a wait the compiler places for a
    // store it cannot count (one under a branch) must not hold up the state
    *(f4*)(sb + (size_t)i0 * S + j0) = s0;
    *(f4*)(sb + (size_t)(i0 + 1) * S + j0) = s1;
    if (tid < 4) *(f4*)(out + (size_t)(TM - 1) * ots + (size_t)h * S + j0) = olast;
    if (cb == 0 && h == kh) {   // every q/k channel of the head, one per thread
#pragma unroll
        for (int i = 0; i < K - 1; ++i) cst_out[(size_t)i * cd + cqk] = wna[i];
    }
    if (tid < 16) {             // the workgroup's 16 v channels
#pragma unroll
        for (int i = 0; i < K - 1; ++i) cst_out[(size_t)i * cd + cvl] = wnb[i];
    }
}

hipError_t launch_gdn_decode_fused(const float* x, int xts, const float* cw, int K, const float* cst_in, float* cst_out,
                                   const float* br, const float* ar, int bts, const float* dt, const float* a,
                                   float* state, float* out, int ots, int nt, int nv, int nk, float eps,
                                   float* ck_state, float* ck_conv, int ck_after, hipStream_t st) {
    const dim3 grid(8 * nv);
#define IT_FUSED(KK, TT)                                                                                     \
    gdn_decode_fused_kernel<KK, TT><<<grid, 256, 0, st>>>(x, xts, cw, cst_in, cst_out, br, ar, bts, dt, a, state, \
                                                          out, ots, nt, nv, nk, eps, ck_state, ck_conv, ck_after)
#define IT_FUSED_T(KK)                    \
    if (nt <= 1) IT_FUSED(KK, 1);         \
    else if (nt == 2) IT_FUSED(KK, 2);    \
    else if (nt == 3) IT_FUSED(KK, 3);    \
    else IT_FUSED(KK, 4);
    switch (K) {
        case 2: IT_FUSED_T(2) break;
        case 3: IT_FUSED_T(3) break;
        default: IT_FUSED_T(4) break;
    }
#undef IT_FUSED_T
#undef IT_FUSED
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Gated RMSNorm epilogue of the GDN output, per (token, V head) row of 128:
//   out = o / sqrt(mean(o^2) + eps) * w * silu(z)
// One wave per row, lane l holds elements l and l + 64. out may alias o.
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(const float* o, int ots, const float* __restrict__ z,
                                                             int zts, const float* __restrict__ w, float eps,
                                                             float* out, int outs, int nv, int nt) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (row >= nv * nt) return;   // whole waves
    const int t = row / nv, h = row - t * nv;
    const float* op = o + (size_t)t * ots + (size_t)h * 128;
    const float* zp = z + (size_t)t * zts + (size_t)h * 128;
    const float a = op[l], b = op[l + 64];
    const float za = zp[l], zb = zp[l + 64], wa = w[l], wb = w[l + 64];
    const float sc = 1.0f / sqrtf(wave_sum(a * a + b * b) * (1.0f / 128.0f) + eps);
    float* dp = out + (size_t)t * outs + (size_t)h * 128;
    dp[l] = (a * sc) * wa * siluf_(za);
    dp[l + 64] = (b * sc) * wb * siluf_(zb);
}

// ------------------------------------------------------------------------------------------------
// Gated-delta recurrence with one workgroup per V head (all 128 columns), so the head's output row
// is complete inside the workgroup and the gated RMSNorm epilogue can be applied before the store.
// Thread = (column quad cq = tid & 31, row group rg = tid >> 5): it holds S[16rg .. 16rg+15][4cq ..
// 4cq+3] (64 floats). Column sums: 16 rows in the thread, rows 16rg and 16(rg^1) by a lane^32
// swap, then the 4 waves through LDS. z == nullptr: plain output (o = S^T q / sqrt(S)).
__global__ __launch_bounds__(256) void gdn_step_head_kernel(
    const float* __restrict__ co, int cts, const float* __restrict__ br, const float* __restrict__ ar, int bts,
    const float* __restrict__ dt, const float* __restrict__ A, float* __restrict__ state, float* __restrict__ out,
    int ots, int nt, int nk, const float* __restrict__ z, int zts, const float* __restrict__ nw, float eps,
    float* __restrict__ ck, int ck_after) {
    constexpr int S = 128, R = 16;
    // per token parity, per wave: {S^T k, S^T q} column sums and k.q
    __shared__ f4 red[2][4][2][32];
    __shared__ float rkq[2][4];
    const int h = blockIdx.x, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int cq = tid & 31, rg = tid >> 5;
    const int kh = h % nk, qk = nk * S, j0 = 4 * cq, i0 = R * rg;
    float* sb = state + (size_t)h * S * S;
    f4 s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = ld_f4(sb + (size_t)(i0 + r) * S + j0);
    const float scale = 1.0f / sqrtf((float)S);
    const float dth = dt[h], ah = A[h];
    // Unconditional loads from a valid address when there is no epilogue: a load under a branch
    // makes the compiler wait for every load before it (here the whole state slice).
    const float* zb = z ? z : co;
    const int zstride = z ? zts : 0;
    const f4 wv = ld_f4((z ? nw : co) + j0);
    // token inputs one token ahead (issued before the previous token's barriers)
    struct Tok { f4 q[R / 4], k[R / 4], v, z; float b, a; };
    auto load_tok = [&](int t) {
        const float* c = co + (size_t)t * cts;
        Tok r;
#pragma unroll
        for (int i = 0; i < R / 4; ++i) {
            r.q[i] = ld_f4(c + kh * S + i0 + 4 * i);
            r.k[i] = ld_f4(c + qk + kh * S + i0 + 4 * i);
        }
        r.v = ld_f4(c + 2 * qk + h * S + j0);
        r.z = ld_f4(zb + (size_t)t * zstride + (z ? (size_t)h * S : 0) + j0);
        r.b = br[(size_t)t * bts + h];
        r.a = ar[(size_t)t * bts + h];
        return r;
    };
    Tok nx = load_tok(0);
    for (int t = 0; t < nt; ++t) {
        const Tok cur = nx;
        if (t + 1 < nt) nx = load_tok(t + 1);
        const f4 (&q)[R / 4] = cur.q;
        const f4 (&k)[R / 4] = cur.k;
        const f4 v = cur.v, zv = cur.z;
        const float beta = sigmoid_hw(cur.b);
        const float eg = exp_hw(softplus_hw(cur.a + dth) * ah);
        // With S' = S + k delta^T (S already decayed), S'^T q = S^T q + (k.q) delta: S^T k, S^T q
        // and k.q reduce together, one exchange and one barrier a token.
        f4 p = {}, sq = {};
        float kq = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            s[r] *= eg;
            p += s[r] * k[r / 4][r & 3];
            sq += s[r] * q[r / 4][r & 3];
            kq += k[r / 4][r & 3] * q[r / 4][r & 3];
        }
        // one swap per column: lanes 0-31 end with the wave's S^T k sums, lanes 32-63 with S^T q
        f4 u;
#pragma unroll
        for (int j = 0; j < 4; ++j) u[j] = fold32(p[j], sq[j]);
        kq = sum_xor32(kq);
        const int b = t & 1;
        red[b][w][l >> 5][cq] = u;
        if (l == 0) rkq[b][w] = kq;
        __syncthreads();
        const f4 sk = (red[b][0][0][cq] + red[b][1][0][cq]) + (red[b][2][0][cq] + red[b][3][0][cq]);
        const f4 delta = (v - sk) * beta;
#pragma unroll
        for (int r = 0; r < R; ++r) s[r] += k[r / 4][r & 3] * delta;
        if (w == 0) {
            const f4 so = (red[b][0][1][cq] + red[b][1][1][cq]) + (red[b][2][1][cq] + red[b][3][1][cq]);
            const float kqs = (rkq[b][0] + rkq[b][1]) + (rkq[b][2] + rkq[b][3]);
            const f4 ot = (so + kqs * delta) * scale;
            f4 res = ot;
            if (z) {
                // lanes 32..63 repeat lanes 0..31: the wave sum counts every column twice
                const float ss = wave_sum(ot[0] * ot[0] + ot[1] * ot[1] + ot[2] * ot[2] + ot[3] * ot[3]) * 0.5f;
                const float sc = 1.0f / sqrtf(ss * (1.0f / S) + eps);
#pragma unroll
                for (int j = 0; j < 4; ++j) res[j] = (ot[j] * sc) * wv[j] * silu_hw(zv[j]);
            }
            if (l < 32) *(f4*)(out + (size_t)t * ots + (size_t)h * S + j0) = res;
        }
        if (ck && t == ck_after) {
            float* cb_ = ck + (size_t)h * S * S;
#pragma unroll
            for (int r = 0; r < R; ++r) *(f4*)(cb_ + (size_t)(i0 + r) * S + j0) = s[r];
        }
        // red[b] / rkq[b] are rewritten two tokens later, after the next token's barrier, which
        // every wave reaches only after finishing this token's reads.
    }
#pragma unroll
    for (int r = 0; r < R; ++r) *(f4*)(sb + (size_t)(i0 + r) * S + j0) = s[r];
}

// ------------------------------------------------------------------------------------------------
hipError_t launch_gdn_conv(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt,
                           int K, float* ck, int ck_after, hipStream_t st) {
    const int TT = nt <= 16 ? nt : 16;
    const dim3 grid((cd + 255) / 256, (nt + TT - 1) / TT);
    // the kernel built for the shortest run length that holds TT tokens
#define IT_CONV_RUN(KK, TM) gdn_conv_kernel<KK, TM><<<grid, 256, 0, st>>>(x, xts, w, state, out, ots, cd, nt, TT, ck, ck_after)
#define IT_CONV(KK)                                                                                           \
    if (ck && grid.y > 1)                                                                                     \
        gdn_conv_state_kernel<KK><<<grid.x, 256, 0, st>>>(x, xts, state, ck, cd, ck_after + 1);              \
    if (TT <= 1) IT_CONV_RUN(KK, 1);                                                                          \
    else if (TT <= 2) IT_CONV_RUN(KK, 2);                                                                     \
    else if (TT <= 4) IT_CONV_RUN(KK, 4);                                                                     \
    else IT_CONV_RUN(KK, 16);                                                                                 \
    if (grid.y > 1) gdn_conv_state_kernel<KK><<<grid.x, 256, 0, st>>>(x, xts, state, state, cd, nt);
    switch (K) {
        case 2: IT_CONV(2) break;
        case 3: IT_CONV(3) break;
        default: IT_CONV(4) break;
    }
#undef IT_CONV
#undef IT_CONV_RUN
    return hipGetLastError();
}

template <typename OutT>
hipError_t launch_gdn_conv_l2(const float* x, int xts, const float* w, float* state, OutT* out, int ots, int cd,
                              int nt, int K, int nnorm, float eps, float* ck, int ck_after, hipStream_t st) {
    const int TT = nt <= 16 ? nt : 16;
    const dim3 grid((cd / 128 + 3) / 4, (nt + TT - 1) / TT);
    // 16-byte form for prompts (several 16-token runs) when every access is 16-byte aligned and a
    // wave's 256 channels are whole; a decode or verify token keeps twice the waves of the scalar form
    const bool v4 = nt > 16 && cd % 256 == 0 && xts % 4 == 0 && ots % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                    ((uintptr_t)out & 15) == 0 && ((uintptr_t)state & 15) == 0 && (!ck || ((uintptr_t)ck & 15) == 0);
    const dim3 grid4((cd / 256 + 3) / 4, (nt + TT - 1) / TT);
#define IT_L2_RUN(KK, TM)                                                                                           \
    gdn_conv_l2_kernel<KK, OutT, TM><<<grid, 256, 0, st>>>(x, xts, w, state, out, ots, cd, nt, TT, nnorm, eps, ck,     \
                                                           ck_after)
#define IT_CONVL2(KK)                                                                                               \
    if (ck && grid.y > 1)                                                                                           \
        gdn_conv_state_kernel<KK><<<(cd + 255) / 256, 256, 0, st>>>(x, xts, state, ck, cd, ck_after + 1);          \
    if (v4)                                                                                                         \
        gdn_conv_l2_v4_kernel<KK, OutT><<<grid4, 256, 0, st>>>(x, xts, w, state, out, ots, cd, nt, TT, nnorm, eps,  \
                                                               ck, ck_after);                                       \
    else if (TT <= 1) IT_L2_RUN(KK, 1);                                                                             \
    else if (TT <= 2) IT_L2_RUN(KK, 2);                                                                             \
    else if (TT <= 4) IT_L2_RUN(KK, 4);                                                                             \
    else IT_L2_RUN(KK, 16);                                                                                         \
    if (grid.y > 1) gdn_conv_state_kernel<KK><<<(cd + 255) / 256, 256, 0, st>>>(x, xts, state, state, cd, nt);
    switch (K) {
        case 2: IT_CONVL2(2) break;
        case 3: IT_CONVL2(3) break;
        default: IT_CONVL2(4) break;
    }
#undef IT_CONVL2
#undef IT_L2_RUN
    return hipGetLastError();
}
template hipError_t launch_gdn_conv_l2<float>(const float*, int, const float*, float*, float*, int, int, int, int,
                                                int, float, float*, int, hipStream_t);
template hipError_t launch_gdn_conv_l2<_Float16>(const float*, int, const float*, float*, _Float16*, int, int, int,
                                                   int, int, float, float*, int, hipStream_t);

hipError_t launch_l2norm(float* x, int ts, int nheads, int d, int nt, float eps, hipStream_t st) {
    const int rows = nheads * nt;
    const dim3 grid((rows + 3) / 4);
    if (d == 128) l2norm_kernel<128><<<grid, 256, 0, st>>>(x, ts, nheads, nt, eps);
    else l2norm_kernel<256><<<grid, 256, 0, st>>>(x, ts, nheads, nt, eps);
    return hipGetLastError();
}

hipError_t launch_gdn_step(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                           const float* a, float* state, float* out, int ots, int nt, int nv, int nk, float* ck,
                           int ck_after, hipStream_t st) {
    if (nt <= 0) return hipSuccess;   // the kernel runs its last token unconditionally
    gdn_step_kernel<<<dim3(8 * nv), 256, 0, st>>>(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, ck, ck_after);
    return hipGetLastError();
}

hipError_t launch_gdn_step_head(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                                const float* a, float* state, float* out, int ots, int nt, int nv, int nk,
                                const float* z, int zts, const float* nw, float eps, float* ck, int ck_after,
                                hipStream_t st) {
    gdn_step_head_kernel<<<dim3(nv), 256, 0, st>>>(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nk, z, zts, nw,
                                                   eps, ck, ck_after);
    return hipGetLastError();
}

hipError_t launch_gdn_gated_norm(const float* o, int ots, const float* z, int zts, const float* w, float eps,
                                 float* out, int outs, int nv, int nt, hipStream_t st) {
    const long rows = (long)nv * nt;
    gdn_gated_norm_kernel<<<dim3((unsigned)((rows + 3) / 4)), 256, 0, st>>>(o, ots, z, zts, w, eps, out, outs, nv, nt);
    return hipGetLastError();
}

// Rollback of both checkpointed states in one launch (two device copies would be two dispatches):
// element e < na of the combined range copies a, the rest b. vec: all four pointers 16-byte
// aligned and the counts multiples of 4, so whole f4s move; otherwise floats.
__global__ __launch_bounds__(256) void gdn_rollback_kernel(const float* __restrict__ as, float* __restrict__ ad,
                                                           size_t na, const float* __restrict__ bs,
                                                           float* __restrict__ bd, size_t nb, int vec) {
    const size_t stride = (size_t)gridDim.x * 256;
    if (vec) {
        const size_t na4 = na / 4, n4 = na4 + nb / 4;
        for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n4; e += stride) {
            if (e < na4) ((f4*)ad)[e] = ((const f4*)as)[e];
            else ((f4*)bd)[e - na4] = ((const f4*)bs)[e - na4];
        }
        return;
    }
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < na + nb; e += stride) {
        if (e < na) ad[e] = as[e];
        else bd[e - na] = bs[e - na];
    }
}

hipError_t launch_gdn_rollback(const float* ck_conv, float* conv, size_t nc, const float* ck_ssm, float* ssm,
                               size_t ns, hipStream_t st) {
    auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    const int vec = (!nc || (al(ck_conv) && al(conv) && nc % 4 == 0)) && (!ns || (al(ck_ssm) && al(ssm) && ns % 4 == 0));
    const size_t units = vec ? (nc + ns) / 4 : nc + ns;
    const size_t wgs = std::min<size_t>((units + 511) / 512, 2048);   // ~2 units per thread
    if (!wgs) return hipSuccess;
    gdn_rollback_kernel<<<(unsigned)wgs, 256, 0, st>>>(ck_conv, conv, nc, ck_ssm, ssm, ns, vec);
    return hipGetLastError();
}

}  // namespace it
