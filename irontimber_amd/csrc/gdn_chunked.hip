// Chunk-64 WY/UT form of the gated delta rule on the matrix cores (a new algorithm: the reference
// runs the recurrence token by token, kernels/src/lib.rs:285-331, cpu.rs:216-232). Per V head h
// and chunk of L <= 64 tokens with in-chunk cumulative log-decay G (G_t = g_0 + ... + g_t) and
// D[t,s] = exp(G_t - G_s), starting from the state S0 (key x value):
//   A'  = strict_lower(diag(beta) (D * K K^T))        M = (I + A')^-1 diag(beta)
//   Y   = V - diag(e^G) K S0                            (V' = M Y is the chunk's corrected values)
//   O   = (diag(e^G) Q S0 + P Y) / sqrt(128)            P  = lower_incl(D * Q K^T) M
//   S1  = e^{G_last} S0 + Kh^T Y                        Kh = M^T diag(e^{G_last - G}) K
// which is the token-sequential recurrence S <- e^g S + beta k (v - e^g S^T k)^T regrouped; only
// decay differences G_t - G_s <= 0 (t >= s) are exponentiated, so nothing overflows.
//
// Kernel 1 (gdn_chunk_prep, one workgroup per (chunk, V head), all chunks in parallel) produces the
// two matrices that carry M: Kh (stored transposed, f16) and P (f16), plus the chunk's decay table
// (G, e^G, e^{G_last - G}, e^{G_last}). K K^T / Q K^T are f16 MFMA products of hi+lo splits (three
// products, ~f32 accurate); Kh and P^T solve (I + A')^T [Z1 | Z2] = [diag(e^{G_last-G}) K | (D *
// Q K^T)^T] by blocked backward substitution (16x16 diagonal inverses, MFMA hi+lo products), then
// scale rows by beta. From an f32 conv output it also writes the chunk's q and k rows as f16.
// Kernel 2 (gdn_chunk_scan, one workgroup per (16-column block of the state, V head)) walks the
// chunks in order with its 128x16 slice of S in MFMA accumulators; S0 and Y enter the products as
// f16 hi+lo pairs through LDS, so the state path keeps f32 accuracy. It reads q, k and its V
// columns from the conv output in place (q and k from the record for an f32 conv output), so a
// record holds 25 KiB per chunk and V head (57 KiB with the f16 q and k rows).
#include "common.h"
#include "internal.h"

namespace it {

namespace {
constexpr int C = 64;      // chunk length
constexpr int SD = 128;    // state size (d_k = d_v)
// per-(V head, chunk) record in scratch, byte offsets
constexpr size_t OFF_KH = 0;                       // f16 [SD][C]   Kh^T (dim-major)
constexpr size_t OFF_P = OFF_KH + SD * C * 2;       // f16 [C][C]    P
constexpr size_t OFF_T = OFF_P + C * C * 2;         // f32 [4][C]    G, e^G, e^{G_last - G}, e^{G_last} (x64)
constexpr size_t OFF_Q = OFF_T + 4 * C * 4;         // f16 [C][SD]   q rows (f32 conv output only)
constexpr size_t OFF_K = OFF_Q + C * SD * 2;        // f16 [C][SD]   k rows (f32 conv output only)
constexpr size_t REC_DIRECT = OFF_Q;                // the scan reads an f16 conv output's q and k in place
constexpr size_t REC_ROWS = OFF_K + C * SD * 2;
static_assert(REC_DIRECT % 256 == 0 && REC_ROWS % 256 == 0, "records stay 256-byte aligned");
template <bool DIRECT> constexpr size_t rec_bytes() { return DIRECT ? REC_DIRECT : REC_ROWS; }
}
#define IT_SCAN_WAIT_VMCNT(N) __builtin_amdgcn_s_waitcnt((((N) & 15) | (((N) >> 4) << 14)) | 0x0F70)

size_t gdn_chunked_scratch_bytes(int nt, int nv, int S, bool f16_conv) {
    (void)S;
    const size_t nch = (size_t)(nt + C - 1) / C;
    return nch * (size_t)nv * (f16_conv ? REC_DIRECT : REC_ROWS);
}

__device__ __forceinline__ f4 mfma16x16x16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// hi + lo f16 split of 4 floats (hi + lo == x to ~2^-22)
__device__ __forceinline__ void split_hi_lo4(f4 x, h4& hi, h4& lo) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const _Float16 h = (_Float16)x[j];
        hi[j] = h;
        lo[j] = (_Float16)(x[j] - (float)h);
    }
}

// ------------------------------------------------------------------------------------------------
// 8 waves, 66 KB of LDS (two workgroups per CU, so one's loads overlap the other's products; 48 KB
// and three from an f16 conv output, whose K rows need no lo plane): the K rows as f16 hi/lo
// pairs, A'^T, the masked Q K^T block and the transposed diagonal-block inverses. Q never enters
// LDS: the Q K^T operands are read from global (the chunk's q rows stay in L2). The triangular
// solve runs in registers.
constexpr int PREP_THREADS = 512;
constexpr int KP = SD + 8;     // f16 row pitch of the K tile (272 B: 16 rows at one column hit distinct bank groups)
constexpr int NSOL = (SD + C) / 16;   // 16-column blocks of the solve: 8 of Kh, 4 of P^T

// Workgroup id -> (chunk c, V head h) of the prep grid, launched 1-D. The nv / nk V heads that
// share a QK head read the same q and k rows; they get ids 8 apart (one XCD, under the
// round-robin XCD dispatch) and are resident together, so those rows come from HBM once into that
// XCD's L2 instead of once per V head.
__device__ __forceinline__ void prep_wg(int id, int nch, int nv, int nk, int& c, int& h) {
    const int r = nv / nk;
    if (r > 1 && (nch * nk) % 8 == 0) {
        const int xcd = id & 7, slot = id >> 3;
        const int u = (slot / r) * 8 + xcd;   // (chunk, QK head)
        c = u % nch;
        h = u / nch + (slot % r) * nk;
    } else {
        c = id % nch;
        h = id / nch;
    }
}

template <typename CoT>
__global__ __launch_bounds__(PREP_THREADS) __attribute__((amdgpu_waves_per_eu(sizeof(CoT) == 2 ? 6 : 4)))
void gdn_chunk_prep(const CoT* __restrict__ co, int cts, const float* __restrict__ br, const float* __restrict__ ar,
                    int bts, const float* __restrict__ dt, const float* __restrict__ A, int nt, int nv, int nk,
                    char* __restrict__ scr) {
    // an f16 conv output is exact in f16, so its hi/lo splits have lo == 0 and the K K^T / Q K^T
    // products need only the hi x hi term (bit-identical to the three-term form); the lo plane of
    // the K tile is then not kept, and the 48 KB of LDS leave room for three workgroups per CU
    constexpr bool F16 = sizeof(CoT) == 2;
    __shared__ __align__(16) _Float16 Kx[F16 ? 1 : 2][C][KP];   // K rows hi (/ lo)
    __shared__ __align__(16) float ApT[C][C + 4];            // ApT[s][t] = A'[t][s] (tiles at and below the diagonal)
    __shared__ __align__(16) _Float16 Aq[C][C + 8];          // lower_incl(D * Q K^T) [t][s], f16 as P is stored
    __shared__ float sG[C], sB[C];
    __shared__ __align__(16) float TdT[4][16][20];           // TdT[i][c][r] = (I + A'_ii)^-1 [r][c]

    const int nch = (nt + C - 1) / C;
    int c, h;
    prep_wg(blockIdx.x, nch, nv, nk, c, h);
    const int t0 = c * C, L = min(C, nt - t0);
    const int kh = h % nk, qk = nk * SD;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, li = l & 15;
    char* rec = scr + ((size_t)h * nch + c) * rec_bytes<F16>();

    // the gate inputs go out first (wave 7 computes beta and the cumulative log-decay below)
    float braw = 0.f, araw = 0.f;
    if (w == 7) {
        const int tl = t0 + min(l, L - 1);
        braw = br[(size_t)tl * bts + h];
        araw = ar[(size_t)tl * bts + h];
    }
    // ---- K rows (zero past the prompt) as hi/lo, beta and the cumulative log-decay; unconditional
    // loads (clamped row, then masked) so no branch separates them from their use
#pragma unroll
    for (int it = 0; it < C * SD / 8 / PREP_THREADS; ++it) {
        const int idx = tid + it * PREP_THREADS;
        const int t = idx >> 4, d8 = 8 * (idx & 15);
        const CoT* row = co + (size_t)(t0 + min(t, L - 1)) * cts + qk + kh * SD + d8;
        const float m = t < L ? 1.f : 0.f;
        f4 k0, k1;
        ld8(row, k0, k1);
        k0 *= m;
        k1 *= m;
        h8 hi, lo;
        split_hi_lo(k0, k1, hi, lo);
        *(h8*)&Kx[0][t][d8] = hi;
        if constexpr (!F16) *(h8*)&Kx[F16 ? 0 : 1][t][d8] = lo;
    }
    // q rows as f16 into the record (f32 conv output only: the scan reads an f16 one in place);
    // rows past the prompt are zero
    if constexpr (!F16) {
#pragma unroll
        for (int it = 0; it < C * SD / 8 / PREP_THREADS; ++it) {
            const int idx = tid + it * PREP_THREADS;
            const int t = idx >> 4, d8 = 8 * (idx & 15);
            const float m = t < L ? 1.f : 0.f;
            f4 q0, q1;
            ld8(co + (size_t)(t0 + min(t, L - 1)) * cts + kh * SD + d8, q0, q1);
            ((u4*)(rec + OFF_Q))[idx] = __builtin_bit_cast(u4, to_h8(q0 * m, q1 * m));
        }
    }
    // q rows of the Q K^T waves (below), issued after the K rows so the K staging never waits for
    // them, and their round trip overlaps the staging and the gates
    const int nb = w == 2 ? 2 : 1;                  // row blocks of waves 0-2
    const int mb0 = w == 0 ? 3 : w == 1 ? 2 : 1;    // first row block; wave 2 then does block 0
    // (an f16 conv output's q rows stay f16 in registers: 32 VGPRs for two blocks instead of 64)
    f4 qv[F16 ? 1 : 2][F16 ? 1 : 8];
    h8 qh[2][4];
    if (w < 3) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nb) break;   // uniform
            const int ta = 16 * (mb0 - b) + li;
            const CoT* qr = co + (size_t)(t0 + min(ta, L - 1)) * cts + kh * SD;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if constexpr (F16) {
                    const h8 v = ld_h8(qr + 32 * ks + 8 * g);
                    qh[b][ks] = ta < L ? v : h8{};
                } else {
                    const float qm = ta < L ? 1.f : 0.f;
                    ld8(qr + 32 * ks + 8 * g, qv[b][2 * ks], qv[b][2 * ks + 1]);
                    qv[b][2 * ks] *= qm;
                    qv[b][2 * ks + 1] *= qm;
                }
            }
        }
    }
    if (w == 7) {
        float gg = 0.f, b = 0.f;
        if (l < L) {
            b = sigmoidf_(braw);
            gg = softplusf_(araw + dt[h]) * A[h];
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(gg, off);
            if (l >= off) gg += y;
        }
        sG[l] = gg;
        sB[l] = b;
    }
    __syncthreads();

    // k rows as f16 (the hi parts, zero past the prompt) for an f32 conv output, and the chunk's
    // decay table: G, e^G, e^{G_last - G} and e^{G_last} (64 copies, one per lane of a load)
    if constexpr (!F16) {
#pragma unroll
        for (int it = 0; it < C * SD / 8 / PREP_THREADS; ++it) {
            const int idx = tid + it * PREP_THREADS;
            ((u4*)(rec + OFF_K))[idx] = *(const u4*)&Kx[0][idx >> 4][8 * (idx & 15)];
        }
    }
    if (tid < C) {
        const float gt = sG[tid], glast = sG[C - 1];
        float* T = (float*)(rec + OFF_T);
        T[tid] = gt;
        T[C + tid] = exp_hw(gt);
        T[2 * C + tid] = exp_hw(fminf(glast - gt, 0.f));
        T[3 * C + tid] = exp_hw(glast);
    }
    // ---- lower 16x16 tiles of K K^T and Q K^T, hi+lo products. The Q K^T tiles are grouped by
    // their 16-row block, whose q rows (read from global, split in registers) serve every tile of
    // the block: wave 0 takes row block 3 (4 tiles), wave 1 row block 2 (3), wave 2 row blocks 1
    // and 0 (3, both blocks' rows loaded together), so each pays one memory round trip. Waves 3-7
    // take the 10 K K^T tiles, two each. A K K^T tile goes to A'^T as four consecutive floats a
    // lane (its rows t = 16mt + 4g + 0..3 at column s).
    if (w < 3) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nb) break;   // uniform
            const int mt = mb0 - b;
            h8 ah[4], al[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if constexpr (F16) ah[ks] = qh[b][ks];
                else split_hi_lo(qv[b][2 * ks], qv[b][2 * ks + 1], ah[ks], al[ks]);
            }
            for (int nt_ = 0; nt_ <= mt; ++nt_) {
                f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int d = 32 * ks + 8 * g;
                    const h8 bh = ld_h8(&Kx[0][16 * nt_ + li][d]);
                    acc = mfma16x16x32(ah[ks], bh, acc);
                    if constexpr (!F16) {
                        const h8 bl = ld_h8(&Kx[F16 ? 0 : 1][16 * nt_ + li][d]);
                        acc = mfma16x16x32(ah[ks], bl, acc);
                        acc = mfma16x16x32(al[ks], bh, acc);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * mt + 4 * g + i, s = 16 * nt_ + li;
                    Aq[t][s] = (_Float16)(s <= t ? exp_hw(fminf(sG[t] - sG[s], 0.f)) * acc[i] : 0.f);
                }
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int tt = (w - 3) + 5 * k;   // K K^T tile 0..9
            const int mt = tt >= 6 ? 3 : tt >= 3 ? 2 : tt >= 1 ? 1 : 0;
            const int nt_ = tt - mt * (mt + 1) / 2;
            const int ta = 16 * mt + li;
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int d = 32 * ks + 8 * g;
                const h8 ah = ld_h8(&Kx[0][ta][d]), bh = ld_h8(&Kx[0][16 * nt_ + li][d]);
                acc = mfma16x16x32(ah, bh, acc);
                if constexpr (!F16) {
                    const h8 al = ld_h8(&Kx[F16 ? 0 : 1][ta][d]), bl = ld_h8(&Kx[F16 ? 0 : 1][16 * nt_ + li][d]);
                    acc = mfma16x16x32(ah, bl, acc);
                    acc = mfma16x16x32(al, bh, acc);
                }
            }
            // acc[i] = (K K^T)[16mt + 4g + i][16nt + li]
            const int s = 16 * nt_ + li;
            f4 a;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * mt + 4 * g + i;
                a[i] = s < t ? sB[t] * exp_hw(fminf(sG[t] - sG[s], 0.f)) * acc[i] : 0.f;
            }
            *(f4*)&ApT[s][16 * mt + 4 * g] = a;
        }
    }
    // upper tiles of the Q K^T block are zero
    for (int idx = tid; idx < C * C / 8; idx += PREP_THREADS) {
        const int t = idx >> 3, s8 = 8 * (idx & 7);
        if ((s8 >> 4) > (t >> 4)) *(u4*)&Aq[t][s8] = u4{0u, 0u, 0u, 0u};
    }
    __syncthreads();   // A'^T and the Q K^T block complete
    // ---- (I + A')^T Z = R with R = [diag(e^{G_last - G}) K | (D * Q K^T)^T] (128 + 64 columns),
    // blocked by 16 rows from the last block up:
    //   T_i = (I + A'_ii)^-1 (16x16, one wave, forward substitution per column), kept transposed
    //   Z_i = T_i^T (R_i - sum_{k>i} A'_ki^T Z_k)          (MFMA, hi+lo products)
    // then Kh^T[d][t] = beta_t Z[t][d] and P[t'][s] = beta_s Z[s][128 + t']. Column block b of the
    // 12 goes to wave b % 8 (waves 0-3 take two).
    if (w == 0) {
        const int kb = l >> 4, ci = l & 15;
        float y[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float acc = r == ci ? 1.0f : 0.0f;
#pragma unroll
            for (int q = 0; q < r; ++q) acc -= ApT[16 * kb + q][16 * kb + r] * y[q];
            y[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; r += 4) *(f4*)&TdT[kb][ci][r] = f4{y[r], y[r + 1], y[r + 2], y[r + 3]};
    }
    const float glast = sG[C - 1];
    __syncthreads();   // the inverses
    // Each wave solves its own 16 columns in registers, no LDS and no barrier: the accumulator of a
    // 16x16x16 MFMA (lane = column li, rows 4g..4g+3) is exactly its B-operand layout (k = 4g..4g+3),
    // so Z_k feeds the blocks above and R_i feeds T_i^T R_i straight from registers. The A operands
    // are rows of A'^T and of T^T: lane (li, g) reads 4 consecutive floats of row li.
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const int b = w + 8 * hf;
        if (b >= NSOL) break;   // uniform
        // right-hand side of this lane's cells: rows 16i + 4g + e, column li of block b
        f4 rhs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (b < SD / 16) {
                const int d = 16 * b + li;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = 16 * i + 4 * g + e;
                    const float kv = F16 ? (float)Kx[0][t][d] : (float)Kx[0][t][d] + (float)Kx[F16 ? 0 : 1][t][d];
                    rhs[i][e] = exp_hw(fminf(glast - sG[t], 0.f)) * kv;
                }
            } else {
                const h4 a = *(const h4*)&Aq[16 * (b - SD / 16) + li][16 * i + 4 * g];
#pragma unroll
                for (int e = 0; e < 4; ++e) rhs[i][e] = (float)a[e];
            }
        }
        f4 Z[4];
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            f4 acc = rhs[i];
#pragma unroll
            for (int k = i + 1; k < 4; ++k) {
                // (A'_ki)^T [li][4g + j] = A'[16k + 4g + j][16i + li] = ApT[16i + li][16k + 4g + j]
                const f4 a = -*(const f4*)&ApT[16 * i + li][16 * k + 4 * g];
                h4 ah, al, zh, zl;
                split_hi_lo4(a, ah, al);
                split_hi_lo4(Z[k], zh, zl);
                acc = mfma16x16x16(ah, zh, acc);
                acc = mfma16x16x16(ah, zl, acc);
                acc = mfma16x16x16(al, zh, acc);
            }
            h4 th, tl, rh, rl;
            split_hi_lo4(*(const f4*)&TdT[i][li][4 * g], th, tl);   // T_i^T [li][4g + j]
            split_hi_lo4(acc, rh, rl);
            f4 z = {0.f, 0.f, 0.f, 0.f};
            z = mfma16x16x16(th, rh, z);
            z = mfma16x16x16(th, rl, z);
            z = mfma16x16x16(tl, rh, z);
            Z[i] = z;
            // rows s = 16i + 4g + 0..3 of column li, scaled by beta_s: four consecutive halves of
            // row d of Kh^T, or of row t' of P
            const int s0 = 16 * i + 4 * g;
            const h4 v = {(_Float16)(sB[s0] * z[0]), (_Float16)(sB[s0 + 1] * z[1]), (_Float16)(sB[s0 + 2] * z[2]),
                          (_Float16)(sB[s0 + 3] * z[3])};
            if (b < SD / 16) *(h4*)(rec + OFF_KH + ((size_t)(16 * b + li) * C + s0) * 2) = v;
            else *(h4*)(rec + OFF_P + ((size_t)(16 * (b - SD / 16) + li) * C + s0) * 2) = v;
        }
    }
}

// ------------------------------------------------------------------------------------------------
constexpr int CW = 16;         // state columns per scan workgroup
constexpr int NCB = SD / CW;   // column blocks of the state per head
constexpr int NI = CW / 16;    // 16-column MFMA tiles per workgroup

// Workgroup barrier for LDS data written by the waves themselves (ds_write): waits for this wave's
// LDS operations only, not for the next chunk's operand loads, which are in flight by design.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void;

// One chunk's operands for one column block, staged in LDS by the direct global->LDS path. Rows
// are XOR-swizzled by 16-byte chunk so the operand reads of 16 consecutive rows hit distinct
// banks: 256-byte rows (k, q) by row & 15, 128-byte rows (Kh^T, P) by (row >> 1) & 7 (two rows
// share a 256-byte bank window). V holds this block's CW columns of the conv output's V rows (f16
// or f32, as the conv output); T the decay table.
template <typename CoT>
struct ScanStage {
    _Float16 K[C * SD];      // [token][dim]
    _Float16 Q[C * SD];      // [token][dim]
    _Float16 KHT[SD * C];    // [dim][token]
    _Float16 P[C * C];       // [token][token]
    CoT V[C * CW];           // [token][column]
    float T[4 * C];
};
__device__ __forceinline__ int swz256(int r) { return r & 15; }
__device__ __forceinline__ int swz128(int r) { return (r >> 1) & 7; }

// Loads of one chunk into stage B, as the share `part` (0-3) of the loader waves, in two batches:
// the k and q rows (scan_stage_kq: from `qb`, row r at qb + min(r, L-1) * pitch, its k row koff
// halves further; 4 + 4 instructions a wave), and the rest (scan_stage_rest: Kh^T, P and (part 0)
// the decay table from the record `rec`, V rows from `vb`, row r at vb + min(r, L-1) * cts; Kh^T
// 4, P 2, V 2 or 4 in all, +1). Instructions of 64 lanes x 16 bytes; lane l lands at byte 16*l of
// its instruction's 1 KB.
template <typename CoT>
__device__ __forceinline__ void scan_stage_kq(const _Float16* __restrict__ qb, int pitch, int koff, int L,
                                              ScanStage<CoT>& B, int part, int l) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {   // 4 rows of 256 B per instruction
        const int i = 4 * part + k, r = 4 * i + (l >> 4), j = (l & 15) ^ swz256(r);
        const _Float16* qr = qb + (size_t)min(r, L - 1) * pitch;
        __builtin_amdgcn_global_load_lds((const void*)(qr + koff + 8 * j), (lds_void*)(B.K + 4 * i * SD), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(qr + 8 * j), (lds_void*)(B.Q + 4 * i * SD), 16, 0, 0);
    }
}
constexpr int SCAN_KQ_LOADS = 8;   // instructions of scan_stage_kq per loader wave
constexpr int SCAN_TOUCH_AHEAD = 3;   // chunks between a chunk's L2 touch and its staging

template <typename CoT>
__device__ __forceinline__ void scan_stage_rest(const char* __restrict__ rec, const CoT* __restrict__ vb, int cts,
                                                int L, ScanStage<CoT>& B, int part, int l) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {   // Kh^T: 8 rows of 128 B per instruction
        const int i = 4 * part + k, r = 8 * i + (l >> 3), j = (l & 7) ^ swz128(r);
        __builtin_amdgcn_global_load_lds(rec + OFF_KH + r * C * 2 + 16 * j, (lds_void*)(B.KHT + 8 * i * C), 16, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {   // P: 8 rows of 128 B
        const int i = 2 * part + k, r = 8 * i + (l >> 3), j = (l & 7) ^ swz128(r);
        __builtin_amdgcn_global_load_lds(rec + OFF_P + r * C * 2 + 16 * j, (lds_void*)(B.P + 8 * i * C), 16, 0, 0);
    }
    constexpr int VL = CW * (int)sizeof(CoT) / 16;   // 16-byte lanes per V row
    constexpr int NVI = C * VL / 64;                  // V instructions in all (2 or 4)
    for (int i = part; i < NVI; i += 4) {             // uniform
        const int r = (64 / VL) * i + l / VL;
        __builtin_amdgcn_global_load_lds((const void*)(vb + (size_t)min(r, L - 1) * cts + 16 / sizeof(CoT) * (l % VL)),
                                         (lds_void*)(B.V + (64 / VL) * i * CW), 16, 0, 0);
    }
    if (part == 0) __builtin_amdgcn_global_load_lds(rec + OFF_T + 16 * l, (lds_void*)B.T, 16, 0, 0);
}

// Scan workgroup: 8 compute waves + 4 loader waves. The dependency chain per chunk is
// Y = V - e^G K S0 and S1 = e^{G_last} S0 + Kh^T Y; the output O = e^G Q S0 + P Y hangs off it.
// Waves 0-3 ("chain") run the chain for chunk c while waves 4-7 ("output") compute O of chunk c-1
// from the previous chunk's S0 and Y (both double buffered in LDS). Waves 8-11 ("loaders") stage
// the operands and touch chunk c+3's lines so that the staging hits L2; only they ever wait for
// global loads, so no compute wave stalls on load issue. A stage's k and q rows are read only
// before the step's second barrier (the chain's Y phase, the output waves' operand copy), so the
// loaders issue chunk c+2's k and q rows after that barrier and the rest of chunk c+1 after the
// first: the ~60 KB a step passes through the CU's load path in both halves of the step.
// An f16 conv output (CoT = _Float16) gives q and k in place; from an f32 one they are the
// prep's f16 rows in the record. V is read in place either way.
constexpr int SCAN_THREADS = 768;

template <typename CoT>
__global__ __launch_bounds__(SCAN_THREADS) void gdn_chunk_scan(const char* __restrict__ scr, const CoT* __restrict__ co,
                                                      int cts, int nch, float* __restrict__ state, float* __restrict__ out,
                                                      int ots, int nt, int nv, int nk) {
    constexpr bool DIRECT = sizeof(CoT) == 2;
    constexpr size_t REC = rec_bytes<DIRECT>();
    constexpr int SP = SD + 8, VP = C + 8;
    __shared__ __align__(16) ScanStage<CoT> B0;
    __shared__ __align__(16) ScanStage<CoT> B1;
    __shared__ __align__(16) _Float16 S0T[2][2][CW][SP];   // [chunk & 1][hi|lo][state column][key dim]
    __shared__ __align__(16) _Float16 YT[2][2][CW][VP];    // [chunk & 1][hi|lo][state column][token]
    __shared__ uint32_t PfSink[64];                         // landing words of the L2 touches, never read

    // XCD-aware placement: workgroups are dealt to the 8 XCDs round-robin by linear id, so id L
    // runs on XCD L % 8. All column blocks of one head go to the same XCD (head = xcd + 8*(slot/NCB))
    // and re-read that head's chunk records from the XCD's L2 instead of HBM; with nk a multiple of
    // 8, the V heads that share a q/k head (h % nk) are on one XCD too.
    const int L_id = blockIdx.x, xcd = L_id & 7, slot = L_id >> 3;
    const int h = xcd + 8 * (slot / NCB), cb = slot % NCB;
    if (h >= nv) return;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 4, li = l & 15;
    const int n0 = CW * cb;
    const char* hrec = scr + (size_t)h * nch * REC;
    const int kh = h % nk;
    // chunk cc's q rows: row r at qbase(cc) + min(r, rows(cc) - 1) * pitch, its k row koff further;
    // its V rows (this block's columns) at vbase(cc) + min(r, rows(cc) - 1) * cts
    auto qbase = [&](int cc) -> const _Float16* {
        if constexpr (DIRECT) return co + (size_t)cc * C * cts + kh * SD;
        else return (const _Float16*)(hrec + (size_t)cc * REC + OFF_Q);
    };
    auto vbase = [&](int cc) { return co + (size_t)cc * C * cts + 2 * nk * SD + h * SD + n0; };
    const int pitch = DIRECT ? cts : SD, koff = DIRECT ? nk * SD : C * SD;
    auto rows = [&](int cc) { return min(C, nt - cc * C); };
    auto stage_kq = [&](int cc, ScanStage<CoT>& B, int part) {
        scan_stage_kq<CoT>(qbase(cc), pitch, koff, rows(cc), B, part, l);
    };
    auto stage_rest = [&](int cc, ScanStage<CoT>& B, int part) {
        scan_stage_rest<CoT>(hrec + (size_t)cc * REC, vbase(cc), cts, rows(cc), B, part, l);
    };

    // Barrier schedule: step c (0 <= c <= nch) holds barriers A_c and B_c. The chain writes S0T[c&1]
    // before A_c, reads stage c&1 and writes YT[c&1] between A_c and B_c, reads stage c&1's Kh^T and
    // table after B_c. The output waves read S0T/YT[(c-1)&1] and stage c&1 between A_c and B_c. The
    // loaders fill stage (c+1)&1's Kh^T, P, V and table after A_c and stage c&1's k and q rows (for
    // chunk c+2) after B_c, and have chunk c+1 landed before A_{c+1}. Step nch only finishes the
    // last chunk's output.
    if (wv >= 8) {
        const int part = wv - 8;
        constexpr int RL = (int)(REC / 128);                        // 128-byte lines of a record
        constexpr int QL = DIRECT ? 2 * C * (SD * 2 / 128) : 0;     // lines of the chunk's q and k rows
        constexpr int VLN = SD * (int)sizeof(CoT) / 128;            // lines of one V row of the head
        // this block's share of chunk cc's 128-byte lines, 32 per loader wave (1024 per head): the
        // record's, then (f16 conv output) those of the q and k rows, then those of the V rows
        auto touch = [&](int cc) {
            cc = min(cc, nch - 1);
            const int u = cb * 128 + part * 32 + (l & 31), L = rows(cc);
            const char* p = hrec + (size_t)cc * REC + 128 * min(u, RL - 1);
            if (u >= RL && u < RL + QL) {
                const int v = u - RL, r = (v >> 1) & (C - 1);
                p = (const char*)(qbase(cc) + (size_t)min(r, L - 1) * pitch + (v >= C * 2 ? koff : 0)) + 128 * (v & 1);
            } else if (u >= RL + QL) {
                const int v = min(u - RL - QL, C * VLN - 1), r = v / VLN;
                p = (const char*)(vbase(cc) - n0 + (size_t)min(r, L - 1) * cts) + 128 * (v % VLN);
            }
            __builtin_amdgcn_global_load_lds((const void*)p, (lds_void*)PfSink, 4, 0, 0);
        };
        stage_kq(0, B0, part);
        stage_rest(0, B0, part);
        if (nch > 1) stage_kq(1, B1, part);
#pragma unroll
        for (int k = 1; k < SCAN_TOUCH_AHEAD; ++k) touch(k);
        // chunk 0 landed; chunk 1's k and q rows and the touches may still be in flight
        if (nch > 1) IT_SCAN_WAIT_VMCNT(SCAN_KQ_LOADS + SCAN_TOUCH_AHEAD - 1);
        else IT_SCAN_WAIT_VMCNT(SCAN_TOUCH_AHEAD - 1);
        for (int c = 0; c <= nch; ++c) {
            lds_barrier();   // A_c
            if (c + 1 < nch) stage_rest(c + 1, (c & 1) ? B0 : B1, part);
            touch(c + SCAN_TOUCH_AHEAD);
            lds_barrier();   // B_c
            // chunk c+1 landed (its k and q rows went out a step earlier); the touch and chunk
            // c+2's k and q rows may still be in flight
            if (c + 2 < nch) {
                stage_kq(c + 2, (c & 1) ? B1 : B0, part);
                IT_SCAN_WAIT_VMCNT(SCAN_KQ_LOADS + 1);
            } else {
                IT_SCAN_WAIT_VMCNT(1);
            }
        }
        return;
    }
    const int w = wv & 3;
    if (wv < 4) {
        float* sh = state + (size_t)h * SD * SD;
        // state slice in accumulator layout: st[mi][ni][i] = S[16(2w+mi) + 4g + i][n0 + 16ni + li]
        f4 st[2][NI];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int i = 0; i < 4; ++i) st[mi][ni][i] = sh[(size_t)(16 * (2 * w + mi) + 4 * g + i) * SD + n0 + 16 * ni + li];
        const int rw = 16 * w + li;
        for (int c = 0; c < nch; ++c) {
            const int b = c & 1;
            const ScanStage<CoT>& B = b ? B1 : B0;
            // ---- S0 -> LDS as hi/lo, transposed to [column][key dim]
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v = st[mi][ni][i];
                        const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
                        const int col = 16 * ni + li, dk = 16 * (2 * w + mi) + 4 * g + i;
                        S0T[b][0][col][dk] = hi;
                        S0T[b][1][col][dk] = lo;
                    }
            lds_barrier();   // A_c
            // ---- Y = V - e^G (K S0) for tokens 16w..16w+15 (k row 16w+li, dims 32ks+8g..). Every
            // operand and V read is issued before the first product (the reads queue behind the
            // loaders' LDS writes, so one round trip instead of one per product), the hi and lo
            // products go to separate accumulators, and Y^T goes out as 8-byte pieces (tokens
            // 16w + 4g + 0..3 of column li are contiguous).
            static_assert(NI == 1, "one 16-column tile per workgroup");
            h8 ka[4], sh[4], sl[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                ka[ks] = ld_h8(B.K + rw * SD + 8 * ((4 * ks + g) ^ swz256(rw)));
                sh[ks] = ld_h8(&S0T[b][0][li][32 * ks + 8 * g]);
                sl[ks] = ld_h8(&S0T[b][1][li][32 * ks + 8 * g]);
            }
            CoT vv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = B.V[(16 * w + 4 * g + i) * CW + li];
            const f4 eg = *(const f4*)&B.T[C + 16 * w + 4 * g];
            f4 xh = {0.f, 0.f, 0.f, 0.f}, xl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                xh = mfma16x16x32(ka[ks], sh[ks], xh);
                xl = mfma16x16x32(ka[ks], sl[ks], xl);
            }
            h4 yh, yl;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = (float)vv[i] - eg[i] * (xh[i] + xl[i]);
                yh[i] = (_Float16)v;
                yl[i] = (_Float16)(v - (float)yh[i]);
            }
            *(h4*)&YT[b][0][li][16 * w + 4 * g] = yh;
            *(h4*)&YT[b][1][li][16 * w + 4 * g] = yl;
            lds_barrier();   // B_c
            // ---- S1 = e^{G_last} S0 + Kh^T Y (Kh^T rows 16(2w+mi)+li, tokens 32ks+8g..), every
            // operand read issued first
            h8 kt[2][2], yv[2][2];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const int rk = 16 * (2 * w + mi) + li;
                    kt[ks][mi] = ld_h8(B.KHT + rk * C + 8 * ((4 * ks + g) ^ swz128(rk)));
                }
#pragma unroll
                for (int hl = 0; hl < 2; ++hl) yv[ks][hl] = ld_h8(&YT[b][hl][li][32 * ks + 8 * g]);
            }
            const float gc = B.T[3 * C];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) st[mi][0] *= gc;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl)
#pragma unroll
                    for (int mi = 0; mi < 2; ++mi) st[mi][0] = mfma16x16x32(kt[ks][mi], yv[ks][hl], st[mi][0]);
        }
        lds_barrier();   // A_nch
        lds_barrier();   // B_nch
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int i = 0; i < 4; ++i) sh[(size_t)(16 * (2 * w + mi) + 4 * g + i) * SD + n0 + 16 * ni + li] = st[mi][ni][i];
        return;
    }
    // ---- output waves: O of chunk c-1 in step c, for tokens 16w..16w+15; the A operands of chunk
    // c (q and P rows) and e^G of the output rows are copied from stage c&1 into registers in step
    // c, used in step c+1
    const float rs = 1.0f / sqrtf((float)SD);
    const int rw = 16 * w + li;
    h8 qg[4], pa[2];
    f4 eg = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c <= nch; ++c) {
        lds_barrier();   // A_c
        const int b = c & 1, pb = b ^ 1;
        f4 oa[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) oa[ni] = f4{0.f, 0.f, 0.f, 0.f};
        if (c > 0) {
            // every operand read first, then the products (hi and lo of S0 in separate accumulators)
            h8 sh[4], sl[4], yv[2][2];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                sh[ks] = ld_h8(&S0T[pb][0][li][32 * ks + 8 * g]);
                sl[ks] = ld_h8(&S0T[pb][1][li][32 * ks + 8 * g]);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl) yv[ks][hl] = ld_h8(&YT[pb][hl][li][32 * ks + 8 * g]);
            f4 qh = {0.f, 0.f, 0.f, 0.f}, ql = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                qh = mfma16x16x32(qg[ks], sh[ks], qh);
                ql = mfma16x16x32(qg[ks], sl[ks], ql);
            }
            oa[0] = (qh + ql) * eg;   // e^{G_t} of rows 16w + 4g + i
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int hl = 0; hl < 2; ++hl) oa[0] = mfma16x16x32(pa[ks], yv[ks][hl], oa[0]);
        }
        if (c < nch) {
            // chunk c's operands, before B_c: the loaders overwrite stage c&1's q rows after it
            const ScanStage<CoT>& B = b ? B1 : B0;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qg[ks] = ld_h8(B.Q + rw * SD + 8 * ((4 * ks + g) ^ swz256(rw)));
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) pa[ks] = ld_h8(B.P + rw * C + 8 * ((4 * ks + g) ^ swz128(rw)));
            eg = *(const f4*)&B.T[C + 16 * w + 4 * g];
        }
        lds_barrier();   // B_c
        if (c > 0) {
            // (stores guarded per token only in a partial last chunk: per-lane conditions split
            // the code into small blocks)
            const int t0 = (c - 1) * C, L = min(C, nt - t0);
            float* orow = out + (size_t)t0 * ots + (size_t)h * SD + n0 + li;
            if (L == C) {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                    for (int i = 0; i < 4; ++i) orow[(size_t)(16 * w + 4 * g + i) * ots + 16 * ni] = oa[ni][i] * rs;
            } else {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = 16 * w + 4 * g + i;
                        if (t < L) orow[(size_t)t * ots + 16 * ni] = oa[ni][i] * rs;
                    }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
template <typename CoT>
hipError_t launch_gdn_chunked(const CoT* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                              const float* a, float* state, float* out, int ots, int nt, int nv, int nk, void* scratch,
                              hipStream_t st) {
    const int nch = (nt + C - 1) / C;
    gdn_chunk_prep<<<dim3(nch * nv), PREP_THREADS, 0, st>>>(co, cts, br, ar, bts, dt, a, nt, nv, nk, (char*)scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // linear grid of 8 * NCB * ceil(nv / 8) workgroups, mapped to (head, column block) in-kernel
    gdn_chunk_scan<CoT><<<dim3(8 * NCB * ((nv + 7) / 8)), SCAN_THREADS, 0, st>>>((const char*)scratch, co, cts, nch, state,
                                                                                 out, ots, nt, nv, nk);
    return hipGetLastError();
}
template hipError_t launch_gdn_chunked<float>(const float*, int, const float*, const float*, int, const float*,
                                              const float*, float*, float*, int, int, int, int, void*, hipStream_t);
template hipError_t launch_gdn_chunked<_Float16>(const _Float16*, int, const float*, const float*, int, const float*,
                                                 const float*, float*, float*, int, int, int, int, void*, hipStream_t);

}  // namespace it
