// Chunk-64 WY/UT form of the gated delta rule on the matrix cores (a new algorithm: the reference
// runs the recurrence token by token, kernels/src/lib.rs:285-331, cpu.rs:216-232). Per V head h
// and chunk of L <= 64 tokens with in-chunk cumulative log-decay G (G_t = g_0 + ... + g_t) and
// D[t,s] = exp(G_t - G_s), starting from the state S0 (key x value):
//   A'  = strict_lower(diag(beta) (D * K K^T))        (I + A') [W | U] = diag(beta) [e^G K | V]
//   V'  = U - W S0
//   O   = (diag(e^G) Q S0 + lower_incl(D * Q K^T) V') / sqrt(128)
//   S1  = e^{G_last} S0 + (diag(e^{G_last - G}) K)^T V'
// which is the token-sequential recurrence S <- e^g S + beta k (v - e^g S^T k)^T regrouped; only
// decay differences G_t - G_s <= 0 (t >= s) are exponentiated, so nothing overflows.
//
// Kernel 1 (gdn_chunk_prep, one workgroup per (chunk, V head), all chunks in parallel) produces
// everything that does not depend on S0 and is not a row of q or k: W (f16), U (f32), the masked
// Q K^T block (f16) and a table of the chunk's decays (G, e^G, e^{G_last - G}, e^{G_last}).
// K K^T / Q K^T are f16 MFMA products of hi+lo splits (three products, ~f32 accurate); the solve
// is blocked by 16 rows: small substitutions for the diagonal blocks, MFMA hi+lo products for the
// rest. From an f32 conv output it also writes the chunk's q and k rows as f16; an f16 conv
// output is read in place by kernel 2.
// Kernel 2 (gdn_chunk_scan, one workgroup per (16-column block of the state, V head)) walks the
// chunks in order with its 128x16 slice of S in MFMA accumulators; S0 and V' enter the products
// as f16 hi+lo pairs through LDS, so the state path keeps f32 accuracy. It takes e^G Q S0 as
// (Q S0) scaled per row, and the decayed K^T as the k rows read transposed from LDS and scaled
// per token, so neither is kept in the records.
#include "common.h"
#include "internal.h"

namespace it {

namespace {
constexpr int C = 64;      // chunk length
constexpr int SD = 128;    // state size (d_k = d_v)
// per-(V head, chunk) record in scratch, byte offsets
constexpr size_t OFF_W = 0;                        // f16 [C][SD]   W (token-major)
constexpr size_t OFF_U = OFF_W + C * SD * 2;        // f32 [C][SD]   U
constexpr size_t OFF_T = OFF_U + C * SD * 4;        // f32 [4][C]    G, e^G, e^{G_last - G}, e^{G_last} (x64)
constexpr size_t OFF_AQK = OFF_T + 4 * C * 4;       // f16 [C][C]    lower_incl(D * Q K^T)
constexpr size_t OFF_Q = OFF_AQK + C * C * 2;       // f16 [C][SD]   q rows (f32 conv output only)
constexpr size_t OFF_K = OFF_Q + C * SD * 2;        // f16 [C][SD]   k rows (f32 conv output only)
constexpr size_t REC_DIRECT = OFF_Q;                // the scan reads an f16 conv output in place
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
// 8 waves, 60 KB of LDS (two workgroups per CU, so one's loads overlap the other's products): the
// K rows as f16 hi/lo pairs (the V rows pass through the same tile once K is dead), A' and the
// diagonal-block inverses. Q never enters LDS: the Q K^T operands and e^G q are read from global
// (the chunk's q rows stay in L2). The triangular solve runs in registers.
constexpr int PREP_THREADS = 512;
constexpr int KP = SD + 8;     // f16 row pitch of the K tile (272 B: 16 rows at one column hit distinct bank groups)

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
__global__ __launch_bounds__(PREP_THREADS) __attribute__((amdgpu_waves_per_eu(4))) void gdn_chunk_prep(const CoT* __restrict__ co, int cts,
                                                               const float* __restrict__ br, const float* __restrict__ ar,
                                                               int bts, const float* __restrict__ dt,
                                                               const float* __restrict__ A, int nt, int nv, int nk,
                                                               char* __restrict__ scr) {
    __shared__ __align__(16) _Float16 Kx[2][C][KP];          // K rows hi / lo, then the V rows (f32)
    __shared__ __align__(16) float Ap[C][C + 4];
    __shared__ float sG[C], sB[C];
    __shared__ __align__(16) float Td[4][16][20];            // inverses of the 16x16 diagonal blocks
    static_assert(2 * C * KP * 2 >= C * SD * 4, "the V rows fit in the K tile");

    // an f16 conv output is exact in f16, so its hi/lo splits have lo == 0 and the K K^T product
    // needs only the hi x hi term (bit-identical to the three-term form)
    constexpr bool F16 = sizeof(CoT) == 2;
    const int nch = (nt + C - 1) / C;
    int c, h;
    prep_wg(blockIdx.x, nch, nv, nk, c, h);
    const int t0 = c * C, L = min(C, nt - t0);
    const int kh = h % nk, qk = nk * SD;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, li = l & 15;
    char* rec = scr + ((size_t)h * nch + c) * rec_bytes<F16>();
    const int col = 16 * w + li;                 // this lane's column of the solve

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
        *(h8*)&Kx[0][t][d8] = hi; *(h8*)&Kx[1][t][d8] = lo;
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
    f4 qv[2][8];
    if (w < 3) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nb) break;   // uniform
            const int ta = 16 * (mb0 - b) + li;
            const CoT* qr = co + (size_t)(t0 + min(ta, L - 1)) * cts + kh * SD;
            const float qm = ta < L ? 1.f : 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                ld8(qr + 32 * ks + 8 * g, qv[b][2 * ks], qv[b][2 * ks + 1]);
                qv[b][2 * ks] *= qm;
                qv[b][2 * ks + 1] *= qm;
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
    // take the 10 K K^T tiles, two each.
    _Float16* aqk = (_Float16*)(rec + OFF_AQK);
    auto store_tile = [&](bool isq, int mt, int nt_, f4 acc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * mt + 4 * g + i, s = 16 * nt_ + li;
            const float d = exp_hw(fminf(sG[t] - sG[s], 0.f));
            if (!isq) Ap[t][s] = s < t ? sB[t] * d * acc[i] : 0.f;
            else aqk[t * C + s] = (_Float16)(s <= t ? d * acc[i] : 0.f);
        }
    };
    if (w < 3) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b >= nb) break;   // uniform
            const int mt = mb0 - b;
            h8 ah[4], al[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) split_hi_lo(qv[b][2 * ks], qv[b][2 * ks + 1], ah[ks], al[ks]);
            for (int nt_ = 0; nt_ <= mt; ++nt_) {
                f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int d = 32 * ks + 8 * g;
                    const h8 bh = ld_h8(&Kx[0][16 * nt_ + li][d]);
                    acc = mfma16x16x32(ah[ks], bh, acc);
                    if constexpr (!F16) {
                        const h8 bl = ld_h8(&Kx[1][16 * nt_ + li][d]);
                        acc = mfma16x16x32(ah[ks], bl, acc);
                        acc = mfma16x16x32(al[ks], bh, acc);
                    }
                }
                store_tile(true, mt, nt_, acc);
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
                    const h8 al = ld_h8(&Kx[1][ta][d]), bl = ld_h8(&Kx[1][16 * nt_ + li][d]);
                    acc = mfma16x16x32(ah, bl, acc);
                    acc = mfma16x16x32(al, bh, acc);
                }
            }
            store_tile(false, mt, nt_, acc);
        }
    }
    // upper tiles of the Q K^T block are zero (16-byte stores)
    {
        u4* aq = (u4*)(rec + OFF_AQK);
        for (int idx = tid; idx < C * C / 8; idx += PREP_THREADS) {
            const int t = idx >> 3, s8 = 8 * (idx & 7);
            if ((s8 >> 4) > (t >> 4)) aq[idx] = u4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();   // A' complete
    // ---- (I + A') [W | U] = diag(beta) [e^G K | V], blocked by 16 rows:
    //   T_i = (I + A'_ii)^-1 (16x16, one wave, forward substitution per column)
    //   X_i = T_i (diag(beta) B_i - sum_{k<i} A'_ik X_k)          (MFMA, hi+lo products)
    // W and U are solved one after the other (128 columns each, one 16-column block per wave).
    if (w == 0) {
        const int kb = l >> 4, ci = l & 15;
        float y[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float acc = r == ci ? 1.0f : 0.0f;
#pragma unroll
            for (int q = 0; q < r; ++q) acc -= Ap[16 * kb + r][16 * kb + q] * y[q];
            y[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) Td[kb][r][ci] = y[r];
    }
    // V rows, coalesced (thread: row tid >> 3, 16 columns); they reach their solve lanes through
    // LDS once the K tile is dead. Rows past the prompt repeat the last row and are zeroed through
    // beta = 0. (The other workgroup on the CU covers their latency.)
    f4 vreg[4];
    {
        const CoT* src = co + (size_t)(t0 + min(tid >> 3, L - 1)) * cts + 2 * qk + h * SD + 16 * (tid & 7);
        ld8(src, vreg[0], vreg[1]);
        ld8(src + 8, vreg[2], vreg[3]);
    }
    // right-hand sides of this lane's 16 (row, column) cells: W from the K tile, U from V
    float rhs[2][4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 16 * i + 4 * g + e;
            rhs[0][i][e] = sB[t] * (exp_hw(sG[t]) * ((float)Kx[0][t][col] + (float)Kx[1][t][col]));
        }
    __syncthreads();   // the K tile is dead: V passes through it to its solve lanes
    float* const Vs = (float*)&Kx[0][0][0];   // [C][SD] f32, 32 KB of the 36 KB tile
#pragma unroll
    for (int j = 0; j < 4; ++j) *(f4*)(Vs + (tid >> 3) * SD + 16 * (tid & 7) + 4 * j) = vreg[j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 16 * i + 4 * g + e;
            rhs[1][i][e] = sB[t] * Vs[t * SD + col];
        }
    // Each wave solves its own 16 columns in registers, no LDS and no barrier: the accumulator of a
    // 16x16x16 MFMA (lane = column li, rows 4g..4g+3) is exactly its B-operand layout (k = 4g..4g+3),
    // so X_k feeds the next block rows and R_i feeds T_i R_i straight from registers.
    //   R_i = beta B_i - sum_{k<i} A'_ik X_k,   X_i = T_i R_i   (hi+lo products on both sides)
    for (int hf = 0; hf < 2; ++hf) {
        f4 X[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f4 acc = {rhs[hf][i][0], rhs[hf][i][1], rhs[hf][i][2], rhs[hf][i][3]};
#pragma unroll
            for (int k = 0; k < i; ++k) {
                const f4 a = -*(const f4*)&Ap[16 * i + li][16 * k + 4 * g];
                h4 ah, al, xh, xl;
                split_hi_lo4(a, ah, al);
                split_hi_lo4(X[k], xh, xl);
                acc = mfma16x16x16(ah, xh, acc);
                acc = mfma16x16x16(ah, xl, acc);
                acc = mfma16x16x16(al, xh, acc);
            }
            h4 th, tl, rh, rl;
            split_hi_lo4(*(const f4*)&Td[i][li][4 * g], th, tl);
            split_hi_lo4(acc, rh, rl);
            f4 z = {0.f, 0.f, 0.f, 0.f};
            z = mfma16x16x16(th, rh, z);
            z = mfma16x16x16(th, rl, z);
            z = mfma16x16x16(tl, rh, z);
            X[i] = z;
            // X_i -> scratch (W f16 / U f32)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * i + 4 * g + e;
                if (hf == 0) ((_Float16*)(rec + OFF_W))[t * SD + col] = (_Float16)z[e];
                else ((float*)(rec + OFF_U))[t * SD + col] = z[e];
            }
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
// are XOR-swizzled by 16-byte chunk so the operand reads hit distinct banks: W and q rows by
// row & 15, the 128-byte Q K^T rows by (row >> 1) & 7 (two rows share a 256-byte bank window), k
// rows by kswz (even, see below). U holds only this block's CW columns; T the chunk's decay table
// (G, e^G, e^{G_last - G}, e^{G_last} x64).
struct ScanStage {
    _Float16 W[C * SD];      // [token][dim]
    _Float16 Q[C * SD];      // [token][dim]
    _Float16 K[C * SD];      // [token][dim]
    _Float16 AQK[C * C];     // [token][token]
    float U[C * CW];         // [token][column]
    float T[4 * C];
};
__device__ __forceinline__ int swz256(int r) { return r & 15; }
__device__ __forceinline__ int swz128(int r) { return (r >> 1) & 7; }
// Even, so 16-byte chunks 2m and 2m+1 stay adjacent and in order (a transpose read takes 32
// aligned bytes per 4 lanes). The 16 rows of one transpose read (8g + 0..3, or 8g + 4..7, for
// g = 0..3, plus a multiple of 32) take each of the 8 values twice, as do 16 consecutive rows.
__device__ __forceinline__ int kswz(int r) { return 2 * ((r & 3) | (((r >> 3) & 1) << 2)); }

// Issue loads of one chunk into stage B as the share `part` (0-3) of the loader waves: W from the
// record `rec`, q and k rows from `qb` (row r at qb + min(r, L-1) * pitch, its k row koff halves
// further), the Q K^T block, this block's U columns and (part 0) the decay table. Instructions of
// 64 lanes x 16 bytes, per wave W 4, q 4, k 4, Q K^T 2, U CW/16 (+1); lane l lands at byte 16*l of
// its instruction's 1 KB.
__device__ __forceinline__ void scan_stage_loads(const char* __restrict__ rec, const _Float16* __restrict__ qb, int pitch,
                                                 int koff, int L, ScanStage& B, int n0, int part, int l) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {   // 4 rows of 256 B per instruction
        const int i = 4 * part + k, r = 4 * i + (l >> 4), j = l & 15;
        const _Float16* qr = qb + (size_t)min(r, L - 1) * pitch;
        __builtin_amdgcn_global_load_lds(rec + OFF_W + r * SD * 2 + 16 * (j ^ swz256(r)), (lds_void*)(B.W + 4 * i * SD), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(qr + 8 * (j ^ swz256(r))), (lds_void*)(B.Q + 4 * i * SD), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(qr + koff + 8 * (j ^ kswz(r))), (lds_void*)(B.K + 4 * i * SD), 16, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {   // Q K^T: 8 rows of 128 B per instruction
        const int i = 2 * part + k, r = 8 * i + (l >> 3), j = (l & 7) ^ swz128(r);
        __builtin_amdgcn_global_load_lds(rec + OFF_AQK + r * C * 2 + 16 * j, (lds_void*)(B.AQK + 8 * i * C), 16, 0, 0);
    }
    constexpr int UL = CW / 4;       // 16-byte lanes per U row (CW floats)
#pragma unroll
    for (int k = 0; k < CW / 16; ++k) {   // this block's U columns: 64/UL rows per instruction
        const int i = (CW / 16) * part + k, r = (64 / UL) * i + l / UL;
        __builtin_amdgcn_global_load_lds(rec + OFF_U + (r * SD + n0) * 4 + 16 * (l % UL), (lds_void*)(B.U + (64 / UL) * i * CW), 16, 0, 0);
    }
    if (part == 0) __builtin_amdgcn_global_load_lds(rec + OFF_T + 16 * l, (lds_void*)B.T, 16, 0, 0);
}

// Scan workgroup: 8 compute waves + 4 loader waves. The dependency chain per chunk is
// V' = U - W S0 and S1 = e^{G_last} S0 + K~^T V'; the output O = e^G Q S0 + Aqk V' hangs off it.
// Waves 0-3 ("chain") run the chain for chunk c while waves 4-7 ("output") compute O of chunk c-1
// from the previous chunk's S0 and V' (both double buffered in LDS). Waves 8-11 ("loaders") stage chunk c+1's operands into the
// other LDS stage and touch chunk c+3's lines so that the staging hits L2; only they ever wait
// for global loads, so no compute wave stalls on load issue.
// DIRECT: q and k rows come from the f16 conv output co (token stride cts), else from the record.
constexpr int SCAN_THREADS = 768;

template <bool DIRECT>
__global__ __launch_bounds__(SCAN_THREADS) void gdn_chunk_scan(const char* __restrict__ scr, const _Float16* __restrict__ co,
                                                      int cts, int nch, float* __restrict__ state, float* __restrict__ out,
                                                      int ots, int nt, int nv, int nk) {
    constexpr size_t REC = rec_bytes<DIRECT>();
    constexpr int SP = SD + 8, VP = C + 8;
    __shared__ __align__(16) ScanStage B0;
    __shared__ __align__(16) ScanStage B1;
    __shared__ __align__(16) _Float16 S0T[2][2][CW][SP];   // [chunk & 1][hi|lo][state column][key dim]
    __shared__ __align__(16) _Float16 VpT[2][2][CW][VP];   // [chunk & 1][hi|lo][state column][token]
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
    // chunk cc's q rows: row r at qbase(cc) + min(r, rows(cc) - 1) * pitch, its k row koff further
    auto qbase = [&](int cc) -> const _Float16* {
        if constexpr (DIRECT) return co + (size_t)cc * C * cts + kh * SD;
        else return (const _Float16*)(hrec + (size_t)cc * REC + OFF_Q);
    };
    const int pitch = DIRECT ? cts : SD, koff = DIRECT ? nk * SD : C * SD;
    auto rows = [&](int cc) { return DIRECT ? min(C, nt - cc * C) : C; };

    // Barrier schedule: step c (0 <= c <= nch) holds barriers A_c and B_c. The chain writes S0T[c&1]
    // before A_c, reads stage c&1 and writes VpT[c&1] between A_c and B_c, reads stage c&1 again
    // after B_c. The output waves read S0T/VpT[(c-1)&1] between A_c and B_c and stage c&1 after
    // B_c. The loaders fill stage (c+1)&1 after A_c and have it landed before A_{c+1}. Step nch
    // only finishes the last chunk's output.
    if (wv >= 8) {
        const int part = wv - 8;
        constexpr int RL = (int)(REC / 128);   // 128-byte lines of a record
        // this block's share of chunk cc's 128-byte lines, 32 per loader wave (1024 per head):
        // the record's, then (DIRECT) those of the q and k rows, 2 per row
        auto touch = [&](int cc) {
            cc = min(cc, nch - 1);
            const int u = cb * 128 + part * 32 + (l & 31);
            const char* p = hrec + (size_t)cc * REC + 128 * min(u, RL - 1);
            if (DIRECT && u >= RL) {
                const int v = min(u - RL, 255), r = (v >> 1) & 63;
                p = (const char*)(qbase(cc) + (size_t)min(r, rows(cc) - 1) * pitch + (v >= 128 ? koff : 0)) + 128 * (v & 1);
            }
            __builtin_amdgcn_global_load_lds((const void*)p, (lds_void*)PfSink, 4, 0, 0);
        };
        scan_stage_loads(hrec, qbase(0), pitch, koff, rows(0), B0, n0, part, l);
        touch(1);
        touch(2);
        IT_SCAN_WAIT_VMCNT(2);
        for (int c = 0; c <= nch; ++c) {
            lds_barrier();   // A_c
            if (c + 1 < nch)
                scan_stage_loads(hrec + (size_t)(c + 1) * REC, qbase(c + 1), pitch, koff, rows(c + 1), (c & 1) ? B0 : B1, n0, part, l);
            touch(c + 3);
            lds_barrier();   // B_c
            IT_SCAN_WAIT_VMCNT(1);   // stage (c+1)&1 landed; the newest touch may still be in flight
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
        // K^T operand by transpose reads: source lane li addresses k row 8g + li/4 (+ 32ks, + 4),
        // dims 16(2w+mi) + 4(li & 3) + 0..3; lane li receives dim 16(2w+mi) + li of 4 tokens
        int ktoff[2];
        {
            const int r = 8 * g + (li >> 2);   // kswz(r + 32ks + 4) == kswz(r)
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const int lj = 2 * (2 * w + mi) + ((li >> 1) & 1);
                ktoff[mi] = r * SD + 8 * (lj ^ kswz(r)) + 4 * (li & 1);
            }
        }
        for (int c = 0; c < nch; ++c) {
            const int b = c & 1;
            const ScanStage& B = b ? B1 : B0;
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
            // ---- V' = U - W S0 for tokens 16w..16w+15 (W row 16w+li, dims 32ks+8g..)
            f4 vp[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) vp[ni] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const h8 a = ld_h8(B.W + rw * SD + 8 * ((4 * ks + g) ^ swz256(rw)));
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) {
                    vp[ni] = mfma16x16x32(a, ld_h8(&S0T[b][0][16 * ni + li][32 * ks + 8 * g]), vp[ni]);
                    vp[ni] = mfma16x16x32(a, ld_h8(&S0T[b][1][16 * ni + li][32 * ks + 8 * g]), vp[ni]);
                }
            }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * w + 4 * g + i, col = 16 * ni + li;
                    const float v = B.U[t * CW + col] - vp[ni][i];
                    const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
                    VpT[b][0][col][t] = hi;
                    VpT[b][1][col][t] = lo;
                }
            lds_barrier();   // B_c
            // ---- S1 = e^{G_last} S0 + (diag(e^{G_last - G}) K)^T V': the K^T operand (dims
            // 16(2w+mi) + li, tokens 32ks + 8g + 0..7) is two transpose reads, scaled per token
            const float gc = B.T[3 * C];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) st[mi][ni] *= gc;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const h8 dk = to_h8(*(const f4*)&B.T[2 * C + 32 * ks + 8 * g], *(const f4*)&B.T[2 * C + 32 * ks + 8 * g + 4]);
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const _Float16* kp = B.K + ktoff[mi] + 32 * ks * SD;
                    const h8 a = cat_h4(lds_tr4(kp), lds_tr4(kp + 4 * SD)) * dk;
#pragma unroll
                    for (int ni = 0; ni < NI; ++ni) {
                        st[mi][ni] = mfma16x16x32(a, ld_h8(&VpT[b][0][16 * ni + li][32 * ks + 8 * g]), st[mi][ni]);
                        st[mi][ni] = mfma16x16x32(a, ld_h8(&VpT[b][1][16 * ni + li][32 * ks + 8 * g]), st[mi][ni]);
                    }
                }
            }
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
    // c (q and Q K^T rows) and e^G of the output rows are copied from stage c&1 into registers in
    // step c, used in step c+1
    const float rs = 1.0f / sqrtf((float)SD);
    const int rw = 16 * w + li;
    h8 qg[4], aqk[2];
    f4 eg = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c <= nch; ++c) {
        lds_barrier();   // A_c
        const int b = c & 1, pb = b ^ 1;
        f4 oa[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) oa[ni] = f4{0.f, 0.f, 0.f, 0.f};
        if (c > 0) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) {
                    oa[ni] = mfma16x16x32(qg[ks], ld_h8(&S0T[pb][0][16 * ni + li][32 * ks + 8 * g]), oa[ni]);
                    oa[ni] = mfma16x16x32(qg[ks], ld_h8(&S0T[pb][1][16 * ni + li][32 * ks + 8 * g]), oa[ni]);
                }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) oa[ni] *= eg;   // e^{G_t} of rows 16w + 4g + i
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) {
                    oa[ni] = mfma16x16x32(aqk[ks], ld_h8(&VpT[pb][0][16 * ni + li][32 * ks + 8 * g]), oa[ni]);
                    oa[ni] = mfma16x16x32(aqk[ks], ld_h8(&VpT[pb][1][16 * ni + li][32 * ks + 8 * g]), oa[ni]);
                }
        }
        if (c < nch) {
            const ScanStage& B = b ? B1 : B0;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qg[ks] = ld_h8(B.Q + rw * SD + 8 * ((4 * ks + g) ^ swz256(rw)));
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) aqk[ks] = ld_h8(B.AQK + rw * C + 8 * ((4 * ks + g) ^ swz128(rw)));
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
    constexpr bool DIRECT = sizeof(CoT) == 2;
    const int nch = (nt + C - 1) / C;
    gdn_chunk_prep<<<dim3(nch * nv), PREP_THREADS, 0, st>>>(co, cts, br, ar, bts, dt, a, nt, nv, nk, (char*)scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const _Float16* co16 = nullptr;
    if constexpr (DIRECT) co16 = co;
    // linear grid of 8 * NCB * ceil(nv / 8) workgroups, mapped to (head, column block) in-kernel
    gdn_chunk_scan<DIRECT><<<dim3(8 * NCB * ((nv + 7) / 8)), SCAN_THREADS, 0, st>>>((const char*)scratch, co16, cts, nch, state,
                                                                                    out, ots, nt, nv, nk);
    return hipGetLastError();
}
template hipError_t launch_gdn_chunked<float>(const float*, int, const float*, const float*, int, const float*,
                                              const float*, float*, float*, int, int, int, int, void*, hipStream_t);
template hipError_t launch_gdn_chunked<_Float16>(const _Float16*, int, const float*, const float*, int, const float*,
                                                 const float*, float*, float*, int, int, int, int, void*, hipStream_t);

}  // namespace it
