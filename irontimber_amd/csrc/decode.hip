// Split-K partials for decode and MTP verify: short dependency chain after the loads land.
//
// Reference behaviour: src/cpu.rs:260-272 (math), kernels/src/lib.rs:753-798 (split-K partial
// record {m, l, pad, pad, o[256]} per (token, head, split), merged by the combine kernel).
//
// One workgroup = one KV head x one split of `chunk` keys x up to 8*NB query rows (rows r = t*G + g,
// token t, head g of the KV group: they all read the same K/V, so each key is loaded once for all
// of them). 4 waves; keys are processed in 64-key tiles, wave w scoring keys 16w..16w+15.
//
//   K      : loaded straight into MFMA A-operand registers (key row = lane & 15, 8 dims per lane
//            group), never staged in LDS.
//   V      : copied to LDS by the DMA path (global_load_lds, 16 bytes a lane, two 512-byte rows an
//            instruction) with its 16-byte chunks XOR-swizzled by row, read back with the LDS
//            transpose read as the P.V B operand.
//   q      : staged once in LDS as f16 hi + lo planes (hi + lo == q to ~2^-22), the B operand of
//            S^T = K q^T: MFMA columns 0-7 carry q_hi, 8-15 q_lo of the block's 8 rows, so the two
//            halves of one score sit in lanes c and c ^ 8 and one DPP row rotate sums them.
//   softmax: in registers. Each lane holds 4 keys of one row; the row maximum of the tile needs the
//            other 48 keys, exchanged through a 4x8-float LDS table (barrier A).
//   P.V    : P (hi + lo f16 rows, as for q) goes to a small LDS plane in MFMA A layout (barrier B,
//            which also covers V); wave w then owns output dims 64w..64w+63 for all 64 keys, and
//            one more MFMA per k-step against a ones column gives it the full row sums.
//   records: stored straight from the accumulators (no staging, no barrier), as the 260-word
//            record or, for the wave merge inside it_attn_f16, the same values in the piece layout
//            below.
// Per tile that is two barriers. First tile: q and K go out first, the q planes are built while K
// is in flight, then V goes out and the scores and softmax run while it lands; later tiles are
// prefetched while P.V runs. MULTI = false (splits of one tile) declares a single V buffer, which
// lets two or three workgroups share a CU.
#include <algorithm>
#include <atomic>

#include "common.h"
#include "internal.h"

namespace it {

namespace {

constexpr int HD = 256;
constexpr int PART = idx::PART;
constexpr int TK = 64;          // keys per tile
constexpr int QST = HD + 8;     // q plane row stride (halves)
constexpr int PST = TK + 8;     // P plane row stride (halves): 144 bytes
constexpr float LOG2E_F = 1.4426950408889634f;
constexpr float LN2_F = 0.6931471805599453f;
constexpr int COMB_SPL = idx::COMB_SPL;   // splits per merge split lane per batch of loads

// V tile chunk swizzle. The transpose read of one 16-lane group covers rows r0..r0+3 (r0 % 4 == 0)
// x 32 bytes (two chunks of one 128-byte line); unswizzled, the four 512-byte-apart rows would hit
// the same banks. XOR-ing the chunk index with 2*(r & 3) moves the four rows to four different
// 32-byte bank groups of the same 128 bytes and keeps the chunk pair together.
__device__ __forceinline__ int vswz(int r) { return (r & 3) << 1; }

typedef __attribute__((address_space(3))) void lds_void;

// DMA one 64-key V tile (rows kb .. kb+63 of KV head `head_off`, clamped to kend-1) into LDS.
// Wave w copies rows 16w .. 16w+15, two rows per instruction; lane l lands at LDS chunk (l & 31) of
// its row, so it fetches logical chunk (l & 31) ^ vswz(row).
__device__ __forceinline__ void v_tile_to_lds(const uint16_t* __restrict__ vc, int kvd, size_t head_off, int kb,
                                              int kend, _Float16* lds, int w, int l) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 16 * w + 2 * i + (l >> 5);
        const int j = (l & 31) ^ vswz(r);
        const uint16_t* g = vc + (size_t)min(kb + r, kend - 1) * kvd + head_off + 8 * j;
        __builtin_amdgcn_global_load_lds(g, (lds_void*)(lds + (16 * w + 2 * i) * HD), 16, 0, 0);
    }
}

// The same V tile into registers (lane l of wave w: the 16 bytes v_tile_to_lds would land at its
// slot of rows 16w + 2i + (l >> 5)), written to that slot once the scores and softmax are done.
__device__ __forceinline__ void v_tile_to_regs(const uint16_t* __restrict__ vc, int kvd, size_t head_off, int kb,
                                               int kend, u4 (&vr)[8], int w, int l) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 16 * w + 2 * i + (l >> 5);
        const int j = (l & 31) ^ vswz(r);
        vr[i] = *(const u4*)(vc + (size_t)min(kb + r, kend - 1) * kvd + head_off + 8 * j);
    }
}
__device__ __forceinline__ void v_regs_to_lds(const u4 (&vr)[8], _Float16* lds, int w, int l) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *(u4*)(lds + (16 * w + 2 * i + (l >> 5)) * HD + 8 * (l & 31)) = vr[i];
}

// K rows as the A operand of S^T = K q^T: lane l holds key kb + 16w + (l & 15), dims 32ks + 8*(l >> 4).
__device__ __forceinline__ void k_tile_to_regs(const uint16_t* __restrict__ kc, int kvd, size_t head_off, int kb,
                                               int kend, u4 (&kr)[8], int w, int l) {
    const uint16_t* g = kc + (size_t)min(kb + 16 * w + (l & 15), kend - 1) * kvd + head_off + 8 * (l >> 4);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kr[ks] = *(const u4*)(g + 32 * ks);
}

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// Mailbox for decode in one launch. The split records go, per 16-dim block, into 96-byte pieces
// {o[16], m, l, unused} of a caller-owned buffer whose words all hold MB_EMPTY between calls (an f32
// NaN pattern no arithmetic produces: generated NaNs are the canonical quiet NaN, and an f16 NaN
// widened keeps its low 13 bits zero). Pieces are written and read device-coherently (past the
// per-XCD L2), and each word is checked on its own, so no flag, fence or store ordering is needed:
// a piece is complete when none of its 18 words is MB_EMPTY. The merging wave then writes
// MB_EMPTY back, which leaves the buffer ready for the next call. Word 0 of the buffer is the
// poison flag, set by a merge that gave up waiting; word 1 holds MAILBOX_MAGIC once the buffer is
// initialised, so a buffer that never was (or was overwritten) fails loudly instead of passing its
// stale words off as records; words 2-3 the address of a host-visible report word that a merge
// which finds the mailbox poisoned sets to 1.
constexpr int MB_PIECE = idx::MB_PIECE;   // floats per piece: o[16], {m, l}, unused; whole 32-byte sectors
constexpr int MB_HEAD = idx::MB_HEAD;     // floats before the first piece
constexpr uint32_t MB_EMPTY = 0xFFFFFFFFu;
constexpr int MB_COHERENT = 16;     // buffer cache-policy bit: device-coherent access
constexpr uint64_t MB_SPIN_TICKS = 1000000;   // 10 ms of the 100 MHz real-time counter
typedef __amdgpu_buffer_rsrc_t MbRsrc;

__device__ __forceinline__ MbRsrc mb_rsrc(float* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, (int)bytes, 0x00020000);
}
// float index of piece (row th, dim block db, split s)
__device__ __forceinline__ int mb_piece(int th, int db, int s, int smax) { return idx::mb_piece(th, db, s, smax); }
// A record value is stored as a word that can never equal MB_EMPTY: any NaN (which could carry a
// payload from a NaN in q, K or V, such as 0xFFFFFFFF) is written as the canonical quiet NaN, so a
// non-finite input gives NaN outputs for that call instead of a piece that never looks complete.
__device__ __forceinline__ uint32_t mb_word(float v) {
    return v != v ? 0x7FC00000u : __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ void mb_store1(MbRsrc r, int idx, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(mb_word(v), r, 4 * idx, 0, MB_COHERENT);
}
__device__ __forceinline__ void mb_store2(MbRsrc r, int idx, f2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(u2{mb_word(v[0]), mb_word(v[1])}, r, 4 * idx, 0, MB_COHERENT);
}
__device__ __forceinline__ void mb_clear2(MbRsrc r, int idx) {
    __builtin_amdgcn_raw_buffer_store_b64(u2{MB_EMPTY, MB_EMPTY}, r, 4 * idx, 0, MB_COHERENT);
}
__device__ __forceinline__ void mb_store4(MbRsrc r, int idx, u4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, 4 * idx, 0, MB_COHERENT);
}
__device__ __forceinline__ u4 mb_load4(MbRsrc r, int idx) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, 4 * idx, 0, MB_COHERENT);
}
__device__ __forceinline__ u2 mb_load2(MbRsrc r, int idx) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, 4 * idx, 0, MB_COHERENT);
}

// VR (one-tile splits only): V is loaded into registers right behind K and written to LDS after
// the softmax, instead of the direct global->LDS copy issued after the q planes. With the copy in
// flight the compiler waits for every outstanding load before the first score product (it treats a
// pending global->LDS copy and ordinary loads as completing out of order), so the scores and the
// softmax could not start until V had landed; with ordinary loads the counter stays in order and
// the scores wait for K only. Decode at ctx 8192: partial kernel 5.95 -> 5.65 us, layer 9.41 ->
// 9.13 us; with few workgroups (ctx 512, 16 of them) the copy is faster (6.09 against 6.27 us per
// layer), so the launch takes VR from 64 workgroups up.
template <int NB, bool MULTI, bool MB = false, bool VR = false, bool CR = false>
__device__ __forceinline__ void decode_partial(const float* __restrict__ q, int qts, const uint16_t* __restrict__ kc,
                                               const uint16_t* __restrict__ vc, int kvd, int pos0, int nh, int nkv,
                                               int nt, float scale, float* __restrict__ part, int chunk, int smax,
                                               int s, int kh, int rg, float* mb = nullptr, uint32_t mbb = 0) {
    constexpr int ROWS = 8 * NB;
    __shared__ __align__(16) _Float16 V0[TK * HD];
    __shared__ __align__(16) _Float16 V1[MULTI ? TK * HD : 8];   // only when a split has several tiles
    __shared__ __align__(16) _Float16 Qs[2][ROWS][QST];   // [hi|lo][row][dim]
    __shared__ __align__(16) _Float16 Ps[NB][16][PST];    // rows 0-7 P_hi, 8-15 P_lo of a row block
    __shared__ float Mx[4][ROWS];                          // per-wave tile maxima
    __shared__ float Al[ROWS];                             // per-row rescale of the tile

    const int G = nh / nkv, R = nt * G, r0 = rg * ROWS;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
    const int tmax = (min(R, r0 + ROWS) - 1) / G;
    const int p0 = s * chunk;
    const int pend = min(p0 + chunk, pos0 + tmax + 1);
    if (p0 >= pend) return;   // no row of this group sees these keys; the combine never reads them
    const float sc2 = scale * LOG2E_F;
    const size_t head_off = (size_t)kh * HD;

    // ---- issue every load of the first tile: q rows (raw f32), K rows (registers), V rows (DMA)
    constexpr int QPT = ROWS * HD / 8 / 256;   // 8-float q pieces per thread (NB)
    f4 qx[QPT][2];
#pragma unroll
    for (int it = 0; it < QPT; ++it) {
        // unconditional loads (padding rows read row R-1 and are zeroed below) keep the wait for q
        // from also waiting for the K and V loads issued after it
        const int idx = tid + 256 * it, rr = min(r0 + (idx >> 5), R - 1);
        const float* src = q + (size_t)(rr / G) * qts + (size_t)(kh * G + rr % G) * 2 * HD + 8 * (idx & 31);
        qx[it][0] = ld_f4(src);
        qx[it][1] = ld_f4(src + 4);
    }
    u4 kr[8];
    k_tile_to_regs(kc, kvd, head_off, p0, pend, kr, w, l);
    static_assert(!(VR && MULTI), "V in registers is for one-tile splits");
    u4 vr[VR ? 8 : 1];
    if constexpr (VR) v_tile_to_regs(vc, kvd, head_off, p0, pend, vr, w, l);
#pragma unroll
    for (int it = 0; it < QPT; ++it) {
        const int idx = tid + 256 * it, row = idx >> 5, d0 = 8 * (idx & 31);
        h8 hi, lo;
        if (r0 + row >= R) qx[it][0] = qx[it][1] = f4{0.f, 0.f, 0.f, 0.f};
        split_hi_lo(qx[it][0], qx[it][1], hi, lo);
        *(h8*)&Qs[0][row][d0] = hi;
        *(h8*)&Qs[1][row][d0] = lo;
    }

    // per-lane row facts for the S^T columns: lane column c is row 8b + (c & 7) of block b
    int lim[NB];
    float m_run[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int rr = r0 + 8 * b + (c & 7);
        lim[b] = rr < R ? pos0 + rr / G + 1 : 0;
        m_run[b] = -INFINITY;
    }
    f4 acc[NB][4], lacc[NB];   // O over this wave's 64 dims, and P times a ones column (row sums)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        lacc[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[b][n] = f4{0.f, 0.f, 0.f, 0.f};
    }
    h8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = (_Float16)1.0f;

    // transpose-read source offsets (halves) of this lane inside a V tile, for key rows
    // 32ks + 8g + 4e' + (c >> 2) and the 16-dim column block of output tile n of wave w
    int voff[2][4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int rlo = 8 * g + 4 * e + (c >> 2);   // + 32ks, which keeps vswz (multiple of 4)
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int col = 64 * w + 16 * n + 4 * (c & 3);
            voff[e][n] = rlo * HD + 8 * ((col >> 3) ^ vswz(rlo)) + (col & 7);
        }
    }

    __syncthreads();   // q planes
    h8 qb[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qb[b][ks] = ld_h8(&Qs[c >> 3][8 * b + (c & 7)][32 * ks + 8 * g]);
    // V goes out only now: the q planes were built while the K rows were in flight, and the scores
    // and softmax below run while V lands (the memory system is kept busy by the other waves' K)
    if constexpr (!VR) v_tile_to_lds(vc, kvd, head_off, p0, pend, V0, w, l);

    int it = 0;
    for (int kb = p0; kb < pend; kb += TK, ++it) {
        const _Float16* Vt = (MULTI && (it & 1)) ? V1 : V0;
        // ---- scores S^T (rows = this wave's 16 keys, columns = q hi/lo rows)
        f4 sacc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            sacc[b] = f4{0.f, 0.f, 0.f, 0.f};
            if (r0 + 8 * b < R) {   // wave-uniform
#pragma unroll
                for (int ks = 0; ks < 8; ++ks)
                    sacc[b] = mfma16x16x32(__builtin_bit_cast(h8, kr[ks]), qb[b][ks], sacc[b]);
            }
        }
        // ---- hi + lo, scale to log2 units, mask; wave-local maxima
        float x[NB][4], mx[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int lb = min(lim[b], pend);
            mx[b] = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = sacc[b][i] + dpp_f<0x128>(sacc[b][i]);   // row_ror:8 -> column c ^ 8
                const int key = kb + 16 * w + 4 * g + i;
                x[b][i] = key < lb ? v * sc2 : -INFINITY;
                mx[b] = fmaxf(mx[b], x[b][i]);
            }
        }
        // maxima over the four 16-lane rows by lane swaps (no LDS). With several blocks the swaps
        // fold them: blocks (0, 1) and (2, 3) share a row-pair swap, the two results share the
        // half-wave swap, and 16-lane row g ends with block g's maxima.
        if constexpr (NB == 1) {
            const float m1 = max_xor32(max_xor16(mx[0]));
            if (g == 0 && c < 8) Mx[w][c] = m1;
        } else {
            float a0 = mx[0], b0 = mx[1];
            swap16(a0, b0);
            float t0 = fmaxf(a0, b0), t1 = t0;
            if constexpr (NB > 2) {
                float a1 = mx[2], b1 = NB > 3 ? mx[NB - 1] : -INFINITY;
                swap16(a1, b1);
                t1 = fmaxf(a1, b1);
            }
            swap32(t0, t1);
            const float m = fmaxf(t0, t1);
            if (g < NB && c < 8) Mx[w][8 * g + c] = m;
        }
        __syncthreads();   // A: tile maxima
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int row = 8 * b + (c & 7);
            const float mt = fmaxf(fmaxf(Mx[0][row], Mx[1][row]), fmaxf(Mx[2][row], Mx[3][row]));
            const float mnew = fmaxf(m_run[b], mt);
            const float a = (mnew == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[b] - mnew);
            const float msub = (mnew == -INFINITY) ? 0.0f : mnew;
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(x[b][i] - msub);
            m_run[b] = mnew;
            h4 ph;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 hi = (_Float16)p[i];
                ph[i] = c < 8 ? hi : (_Float16)(p[i] - (float)hi);
            }
            *(h4*)&Ps[b][c][16 * w + 4 * g] = ph;
            if (MULTI && w == 0 && g == 0 && c < 8) Al[row] = a;   // (one tile: nothing to rescale)
        }
        if constexpr (VR) v_regs_to_lds(vr, V0, w, l);   // (the compiler waits for V's loads)
        else IT_WAIT_VMCNT(0);   // this tile's V
        __syncthreads();    // B: P planes, alpha, V tile
        // prefetch the next tile (K registers are free, the other V buffer was last read two
        // barriers ago)
        if (MULTI && kb + TK < pend) {
            k_tile_to_regs(kc, kvd, head_off, kb + TK, pend, kr, w, l);
            v_tile_to_lds(vc, kvd, head_off, kb + TK, pend, (it & 1) ? V0 : V1, w, l);
        }
        // ---- O = diag(alpha) O + P V over output dims 64w .. 64w+63
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (r0 + 8 * b >= R) continue;   // wave-uniform
            if constexpr (MULTI) {   // with one tile per split O and l are still zero here
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float a = Al[8 * b + ((4 * g + i) & 7)];
#pragma unroll
                    for (int n = 0; n < 4; ++n) acc[b][n][i] *= a;
                    lacc[b][i] *= a;
                }
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const h8 pa = ld_h8(&Ps[b][c][32 * ks + 8 * g]);
                lacc[b] = mfma16x16x32(pa, ones, lacc[b]);
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    const h8 vb = cat_h4(lds_tr4(Vt + 32 * ks * HD + voff[0][n]), lds_tr4(Vt + 32 * ks * HD + voff[1][n]));
                    acc[b][n] = mfma16x16x32(pa, vb, acc[b][n]);
                }
            }
        }
    }

    // ---- records {m (natural log units), l, 0, 0, o[256]} straight from registers: adding lanes l
    // and l ^ 32 sums the P_hi and P_lo halves. One swap per pair of dim blocks (n, n + 1) leaves
    // the sum of block n in the lower half-wave and of block n + 1 in the upper, so lane (c, g)
    // holds row 4(g & 1) + i at dims 64w + 16(2k + (g >> 1)) + c for k = 0, 1 (16 lanes store 64
    // contiguous bytes of a row), and the ones product gives every wave the full row sums. Wave 0's
    // lower half adds the headers.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (r0 + 8 * b >= R) continue;   // wave-uniform
        // (token, q-head) of row r0 + 8b + 4g, then walked over i (one division per block)
        const int rb = r0 + 8 * b + 4 * (g & 1);
        int tq = rb / G, gq = rb - tq * G;
        float mh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) mh[i] = __shfl(m_run[b], (4 * g + i) & 7);   // lane row = c & 7
        // row sums of rows 4(g & 1) + i: rows i = 0, 2 in the lower half-wave, 1, 3 in the upper
        const float lsp[2] = {fold32(lacc[b][0], lacc[b][1]), fold32(lacc[b][2], lacc[b][3])};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hi = l >> 5;
            const float v[2] = {fold32(acc[b][0][i], acc[b][1][i]), fold32(acc[b][2][i], acc[b][3][i])};
            const float ls = lsp[i >> 1];
            const bool hdr = hi == (i & 1) && c == 0;   // the lanes that hold row 4(g & 1) + i's sum
            if (rb + i < R) {
                const int th = tq * nh + kh * G + gq;
                if constexpr (MB) {
                    // mailbox pieces of dim blocks 4w .. 4w+3: dims from every lane, {m, l} from
                    // lanes c < 4 (one piece each); only for rows that see this split's keys
                    // (the merge reads exactly those pieces and clears them)
                    const MbRsrc mbr = mb_rsrc(mb, mbb);
                    if (p0 <= pos0 + tq) {
#pragma unroll
                        for (int k = 0; k < 2; ++k) mb_store1(mbr, mb_piece(th, 4 * w + 2 * k + hi, s, smax) + c, v[k]);
                        if (hi == (i & 1) && c < 4) mb_store2(mbr, mb_piece(th, 4 * w + c, s, smax) + 16, f2{mh[i] * LN2_F, ls});
                    }
                } else if constexpr (CR) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        float* dst = prec_o(part, th, 4 * w + 2 * k + hi, s, smax) + c;
                        if constexpr (NB >= 2) __builtin_nontemporal_store(v[k], dst);   // as below
                        else *dst = v[k];
                    }
                    if (w == 0 && hdr) *(f2*)prec_h(part, nt * nh, th, s, smax) = f2{mh[i] * LN2_F, ls};
                } else if constexpr (NB >= 2) {
                    // blocks of 16 or more rows (verify at nt = 4) store their records
                    // non-temporally: measured faster there (15.7 -> 14.6 us per layer), slower for
                    // decode (10.3 -> 11.1)
                    float* rec = part + idx::rec(th, s, smax) * PART;
#pragma unroll
                    for (int k = 0; k < 2; ++k) __builtin_nontemporal_store(v[k], rec + 4 + 64 * w + 16 * (2 * k + hi) + c);
                    if (w == 0 && hdr) __builtin_nontemporal_store(f4{mh[i] * LN2_F, ls, 0.f, 0.f}, (f4*)rec);
                } else {
                    float* rec = part + idx::rec(th, s, smax) * PART;
#pragma unroll
                    for (int k = 0; k < 2; ++k) rec[4 + 64 * w + 16 * (2 * k + hi) + c] = v[k];
                    if (w == 0 && hdr) *(f4*)rec = f4{mh[i] * LN2_F, ls, 0.f, 0.f};
                }
            }
            if (++gq == G) { gq = 0; ++tq; }
        }
    }
}

template <int NB, bool MULTI, bool VR = false, bool CR = false>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float* __restrict__ q, int qts,
                                                          const uint16_t* __restrict__ kc,
                                                          const uint16_t* __restrict__ vc, int kvd, int pos0, int nh,
                                                          int nkv, int nt, float scale, float* __restrict__ part,
                                                          int chunk, int smax) {
    decode_partial<NB, MULTI, false, VR, CR>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, smax, blockIdx.x, blockIdx.y,
                       blockIdx.z);
}

// ------------------------------------------------------------------------------------------------
// Merge of the partial records of one query row over its visible splits:
// M = max m_s, den = sum l_s e^(m_s-M), out = sum o_s e^(m_s-M) / den * sigmoid(gate)
// (kernels/src/lib.rs:722-740). Thread = (split lane sg of SL, dim lane of 256/SL, 4 dims each).
// Each thread loads the headers and its dims of up to 8 of its splits in one batch before using any
// of them; the maxima and sums reduce through LDS.
//   SL = 16: a quarter of the dims per workgroup (4 per row), for rows with many splits (decode).
//   SL = 4 : the whole row per workgroup, for rows with at most 32 splits (chunked prefill).
//   Q16: the flash key-split records (O as int16 in units of k, headers {m, l, k, 0} in their own
//        region: rec_index.h flash_o / flash_h).
template <int SL, bool Q16 = false>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ q, int qts, int pos0, int nh,
                                                          const float* __restrict__ part, int chunk, int smax,
                                                          float* __restrict__ out, int ots) {
    constexpr int RW = PART;                 // record words (f32 records)
    constexpr int DLN = 256 / SL;            // dim lanes, 4 dims each
    constexpr int DW = 4 * DLN;              // dims per workgroup
    __shared__ float red_m[SL];
    __shared__ f4 red_o[SL][DLN];
    __shared__ float red_d[SL];
    const int dq = blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int sg = tid / DLN, dl = tid % DLN, d0 = DW * dq + 4 * dl;
    const int ns = idx::splits_seen(pos0, t, chunk);
    const float* base = part + idx::rec(t * nh + h, 0, smax) * RW;
    const int rows = (int)gridDim.z * nh;
    const f4 gt = ld_f4(q + (size_t)t * qts + (size_t)h * 2 * HD + HD + d0);
    float M = -INFINITY, den = 0.f;
    f4 o = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += SL * COMB_SPL) {
        const int nb = idx::comb_count(ns, s0, sg, SL);   // this lane's splits in the batch
        f2 hv[COMB_SPL];
        f4 ov[COMB_SPL];
        float kv[COMB_SPL];
        u2 qv[COMB_SPL];
        // branch-free batch: slots past the lane's count reload its last split and are masked after.
        // Headers load as {m, l} only: a wider load with dead lanes lets the register allocator
        // reuse them while the load is in flight, which costs a wait per load.
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) {
            // a lane with no split left in the batch (nb <= 0) reloads split ns - 1: every index
            // stays inside this row's records, so a buffer sized exactly for them is never overrun
            const int sj = idx::comb_split(s0, sg, SL, j, nb, ns);
            if (Q16) {
                const float* hd = part + idx::flash_h(rows, t * nh + h, sj, smax);
                hv[j] = *(const f2*)hd;
                kv[j] = hd[2];
                qv[j] = *((const u2*)(part + idx::flash_o(t * nh + h, sj, smax)) + (d0 >> 2));
            } else {
                const float* rec = base + (size_t)sj * RW;
                hv[j] = *(const f2*)rec;
                ov[j] = ld_f4(rec + 4 + d0);
            }
        }
        if (Q16) {
#pragma unroll
            for (int j = 0; j < COMB_SPL; ++j) {
                // int16 pairs, low half first: sign-extend, convert, scale by k
                const int32_t a = (int32_t)qv[j][0], b = (int32_t)qv[j][1];
                ov[j] = f4{(float)((a << 16) >> 16), (float)(a >> 16), (float)((b << 16) >> 16), (float)(b >> 16)} * kv[j];
            }
        }
        float mloc = M;
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) {
            if (j >= nb) { hv[j] = f2{-INFINITY, 0.f}; ov[j] = f4{0.f, 0.f, 0.f, 0.f}; }
            mloc = fmaxf(mloc, hv[j][0]);
        }
        if (dl == 0) red_m[sg] = mloc;
        __syncthreads();
        float Mn = red_m[0];
#pragma unroll
        for (int j = 1; j < SL; ++j) Mn = fmaxf(Mn, red_m[j]);
        __syncthreads();
        const float r = (M == -INFINITY) ? 0.f : __expf(M - Mn);
        den *= r;
        o *= r;
#pragma unroll
        for (int j = 0; j < COMB_SPL; ++j) {
            const float wgt = hv[j][0] == -INFINITY ? 0.f : __expf(hv[j][0] - Mn);
            den += hv[j][1] * wgt;
            o += ov[j] * wgt;
        }
        M = Mn;
    }
    red_o[sg][dl] = o;
    if (dl == 0) red_d[sg] = den;
    __syncthreads();
    if (sg == 0) {
        f4 acc = red_o[0][dl];
        float dd = red_d[0];
#pragma unroll
        for (int j = 1; j < SL; ++j) { acc += red_o[j][dl]; dd += red_d[j]; }
        f4 res;
#pragma unroll
        for (int j = 0; j < 4; ++j) res[j] = acc[j] / dd * sigmoidf_(gt[j]);
        *(f4*)(out + (size_t)t * ots + (size_t)h * HD + d0) = res;
    }
}

// Merge of the rows of a prefill chunk (at most NS <= 64 splits a row): one wave per query row,
// lane l owning dims 4l .. 4l+3. Lane j also loads the header of split j, so the row maximum and
// the denominator are one wave reduction each and split j's weight is read from lane j; every
// header and O load is issued before any is used (one memory round trip; O slots past the row's
// ns reload its last split and are skipped). No LDS, no barrier. Same formula as
// attn_combine_kernel, the splits' O summed in order.
template <int NS, bool Q16>
__global__ __launch_bounds__(256) void attn_combine_row_kernel(const float* __restrict__ q, int qts, int pos0, int nh,
                                                               int nt, const float* __restrict__ part, int chunk,
                                                               int smax, float* __restrict__ out, int ots) {
    const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
    if (row >= nt * nh) return;
    const int l = threadIdx.x & 63;
    const int t = row / nh, h = row - t * nh;
    const int ns = idx::splits_seen(pos0, t, chunk);   // splits holding keys <= pos0 + t (1 .. smax)
    const float* base = part + idx::rec(row, 0, smax) * PART;   // f32 records
    // lane l: header of split l (int16 records: the packed header region, 16 bytes a split)
    const f4 hl = Q16 ? *(const f4*)(part + idx::flash_h(nt * nh, row, idx::row_split(l, ns), smax))
                      : *(const f4*)(base + (size_t)idx::row_split(l, ns) * PART);
    f4 ov[NS];
    u2 qv[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        if constexpr (Q16) qv[j] = *((const u2*)(part + idx::flash_o(row, idx::row_split(j, ns), smax)) + l);
        else ov[j] = ld_f4(base + (size_t)idx::row_split(j, ns) * PART + 4 + 4 * l);
    }
    const f4 gt = ld_f4(q + (size_t)t * qts + (size_t)h * 2 * HD + HD + 4 * l);
    const float M = wave_max(l < ns ? hl[0] : -INFINITY);   // finite: split 0 holds key 0
    const float wl = l < ns ? __expf(hl[0] - M) : 0.f;
    const float den = wave_sum(hl[1] * wl);
    const float wk = Q16 ? wl * hl[2] : wl;   // int16 records: the scale k folded into the weight
    f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        // lanes at or past ns hold weight 0; their slots reloaded split ns - 1, which the row sees,
        // so a non-finite O there reaches the output through that split's own term anyway
        const float wj = readlane_f(wk, j);
        if constexpr (Q16) {
            // int16 pairs, low half first: sign-extend, convert
            const int32_t a = (int32_t)qv[j][0], b = (int32_t)qv[j][1];
            o += f4{(float)((a << 16) >> 16), (float)(a >> 16), (float)((b << 16) >> 16), (float)(b >> 16)} * wj;
        } else {
            o += ov[j] * wj;
        }
    }
    f4 res;
#pragma unroll
    for (int e = 0; e < 4; ++e) res[e] = o[e] / den * sigmoidf_(gt[e]);
    *(f4*)(out + (size_t)t * ots + (size_t)h * HD + 4 * l) = res;
}

// Merge without barriers: one wave per (token, head, 16-dim block). Lane l takes splits l, l + 64,
// ... (SPL of them, loads clamped to the last valid split and masked), merges them in registers,
// then the 64 lanes are reduced by a halving butterfly: the swap across lane halves (and across
// 16-lane rows) hands each lane of a pair the half of the other's values it keeps, so 16 dims
// need 8 + 4 + 2 + 1 + 2 exchanges instead of 16 full reductions. Lane l ends holding dim
// 8*b5 + 4*b4 + 2*b3 + b2 (bits of l) summed over all lanes.

// Given lane l's headers hv[j] = {m, l} and dims d0 .. d0+15 ov[j] of splits l + 64j (those at or
// past ns masked here), merge them over the wave and store the 16 gated outputs of row (t, h).
// The gate input of the output dim lane l ends up holding (see the butterfly below).
__device__ __forceinline__ float merge_gate(const float* __restrict__ q, int qts, int t, int h, int d0, int l) {
    return q[(size_t)t * qts + (size_t)h * 2 * HD + HD + d0 + 8 * (l >> 5) + 4 * ((l >> 4) & 1) + 2 * ((l >> 3) & 1) +
             ((l >> 2) & 1)];
}
template <int SPL>
__device__ __forceinline__ void merge_wave_store(float gv, int nh, int t, int h, int ns, f2 (&hv)[SPL],
                                                 const f4 (&ov)[SPL][4], float* __restrict__ out, int ots, int d0,
                                                 int l) {
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        if (l + 64 * j >= ns) hv[j][0] = -INFINITY;
        M = fmaxf(M, hv[j][0]);
    }
    M = wave_max(M);   // finite: split 0 always holds key 0
    float den = 0.f, o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.f;
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const float wgt = hv[j][0] == -INFINITY ? 0.f : __expf(hv[j][0] - M);
        den += hv[j][1] * wgt;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[4 * k + e] += ov[j][k][e] * wgt;
    }
    den = wave_sum(den);
    // lanes 0-31 keep dims 0-7, lanes 32-63 dims 8-15
    float r8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float a = o[i], b = o[8 + i];
        swap32(a, b);
        r8[i] = a + b;
    }
    // within each half: rows 0 and 2 keep the lower 4, rows 1 and 3 the upper 4
    float r4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a = r8[i], b = r8[4 + i];
        swap16(a, b);
        r4[i] = a + b;
    }
    // within each 16-lane row by DPP (no LDS): the partner of lane i is 15 - i (row_mirror, the
    // other b3) and then 7 - i within its half (row_half_mirror, the other b2), so the partner
    // sets of lanes i, i ^ 1, i ^ 2, i ^ 3 together cover the row; each lane keeps the half its own
    // bits select, and the quad sums finish by quad_perm
    const bool b3 = (l >> 3) & 1, b2 = (l >> 2) & 1;
    float r2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float keep = b3 ? r4[2 + i] : r4[i], give = b3 ? r4[i] : r4[2 + i];
        r2[i] = keep + dppc<0x140>(give);   // row_mirror
    }
    float v;
    {
        const float keep = b2 ? r2[1] : r2[0], give = b2 ? r2[0] : r2[1];
        v = keep + dppc<0x141>(give);       // row_half_mirror
    }
    v += dppc<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dppc<0xB1>(v);   // quad_perm [1,0,3,2]
    if ((l & 3) == 0) {
        const int d = d0 + 8 * (l >> 5) + 4 * ((l >> 4) & 1) + 2 * ((l >> 3) & 1) + ((l >> 2) & 1);
        out[(size_t)t * ots + (size_t)h * HD + d] = v / den * sigmoidf_(gv);
    }
}

// One wave merges the records of query row th (token t = th / nh, head h) for output dims
// d0 .. d0+15; lane l = the wave's lane. CR: the records in the piece layout.
template <int SPL, bool CR>
__device__ __forceinline__ void combine_wave_row(const float* __restrict__ q, int qts, int pos0, int nh, int nt,
                                                 const float* __restrict__ part, int chunk, int smax,
                                                 float* __restrict__ out, int ots, int th, int d0, int l) {
    if (th >= nt * nh) return;   // whole wave
    const int t = th / nh, h = th - t * nh;
    const int ns = idx::splits_seen(pos0, t, chunk);   // splits that hold keys <= pos0 + t
    f2 hv[SPL];
    f4 ov[SPL][4];
    if constexpr (CR) {
        float* pp = const_cast<float*>(part);
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const int sj = idx::wave_split(l, j, ns);
            hv[j] = *(const f2*)prec_h(pp, nt * nh, th, sj, smax);
            const float* src = prec_o(pp, th, d0 >> 4, sj, smax);
#pragma unroll
            for (int k = 0; k < 4; ++k) ov[j][k] = ld_f4(src + 4 * k);
        }
    } else {
        const float* base = part + idx::rec(th, 0, smax) * PART;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const float* rec = base + (size_t)idx::wave_split(l, j, ns) * PART;
            hv[j] = *(const f2*)rec;
#pragma unroll
            for (int k = 0; k < 4; ++k) ov[j][k] = ld_f4(rec + 4 + d0 + 4 * k);
        }
    }
    merge_wave_store<SPL>(merge_gate(q, qts, t, h, d0, l), nh, t, h, ns, hv, ov, out, ots, d0, l);
}

template <int SPL>
__global__ __launch_bounds__(256) void attn_combine_wave_kernel(const float* __restrict__ q, int qts, int pos0,
                                                                int nh, int nt, const float* __restrict__ part,
                                                                int chunk, int smax, float* __restrict__ out,
                                                                int ots) {
    // workgroup = 4 waves = 64 dims of one row; the 4 workgroups of a row read the same record
    // lines, so they get ids 8 apart (one XCD under the round-robin dispatch) when the row count
    // allows it, and each line comes from HBM into that XCD's L2 once
    int row, quarter;
    if ((nt * nh) % 8 == 0) {
        const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
        row = ((slot >> 2) << 3) | xcd;
        quarter = slot & 3;
    } else {
        row = blockIdx.x >> 2;
        quarter = blockIdx.x & 3;
    }
    combine_wave_row<SPL, false>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots, row,
                          16 * (4 * quarter + (threadIdx.x >> 6)), threadIdx.x & 63);
}

// The same merge with one wave per workgroup, for the piece layout: (row, 16-dim block) units spread
// over rows x 16 workgroups instead of a quarter as many. With 260-word records it was slower (each
// wave's loads touched a line per split); with pieces it is faster: ctx-8192 decode layer 8.53 /
// 8.54 -> 8.26 / 8.28 us, verify nt = 4 12.51 -> 12.47 us, ctx 512 5.81 -> 5.77 us (same box).
template <int SPL>
__global__ __launch_bounds__(64) void attn_combine_wave1_kernel(const float* __restrict__ q, int qts, int pos0,
                                                                int nh, int nt, const float* __restrict__ part,
                                                                int chunk, int smax, float* __restrict__ out,
                                                                int ots) {
    int row, db;
    idx::wave1_unit((int)blockIdx.x, nt * nh, row, db);
    combine_wave_row<SPL, true>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots, row, 16 * db, threadIdx.x & 63);
}

// One wave merges mailbox unit (row th, dim block db): lane l polls its pieces of splits l + 64j
// until every word has arrived (bounded by a deadline on the real-time counter), merges as
// combine_wave_row does, and clears the pieces it read. A poisoned mailbox, or a wait that ran out
// (which poisons it), gives NaN outputs.
template <int SPL>
__device__ __forceinline__ void mailbox_merge(const float* __restrict__ q, int qts, int pos0, int nh, int chunk,
                                              int smax, MbRsrc r, float* __restrict__ out, int ots, int th, int db,
                                              int l) {
    const int t = th / nh, h = th - t * nh, d0 = 16 * db;
    const int ns = idx::splits_seen(pos0, t, chunk);
    f2 hv[SPL];
    f4 ov[SPL][4];
    bool ok[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        ok[j] = l + 64 * j >= ns;
        hv[j] = f2{-INFINITY, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) ov[j][k] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const float gv = merge_gate(q, qts, t, h, d0, l);   // issued before the wait, used after it
    const u2 hdr = mb_load2(r, 0);
    bool bad = hdr[0] != 0u || hdr[1] != MAILBOX_MAGIC;
    const uint64_t deadline = __builtin_amdgcn_s_memrealtime() + MB_SPIN_TICKS;
    while (!bad) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            if (ok[j]) continue;
            const int base = mb_piece(th, db, l + 64 * j, smax);
            u4 w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) w[k] = mb_load4(r, base + 4 * k);
            const u2 hw = mb_load2(r, base + 16);
            bool full = hw[0] != MB_EMPTY && hw[1] != MB_EMPTY;
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) full = full && w[k][e] != MB_EMPTY;
            if (full) {
                ok[j] = true;
                hv[j] = __builtin_bit_cast(f2, hw);
#pragma unroll
                for (int k = 0; k < 4; ++k) ov[j][k] = __builtin_bit_cast(f4, w[k]);
            }
        }
        bool mine = true;
#pragma unroll
        for (int j = 0; j < SPL; ++j) mine = mine && ok[j];
        if (__all(mine)) break;
        if (__builtin_amdgcn_s_memrealtime() > deadline) {
            bad = true;
            if (l == 0) mb_store2(r, 0, f2{1.f, 1.f});
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (bad) {
        if (l < 16) out[(size_t)t * ots + (size_t)h * HD + d0 + l] = __builtin_nanf("");
        // tell the host (an initialised header holds the address of its report word), so the
        // next it_attn_f16_mailbox call with this mailbox fails instead of returning NaN again
        if (l == 0 && hdr[1] == MAILBOX_MAGIC) {
            const u2 a = mb_load2(r, 2);
            uint32_t* rep = (uint32_t*)(uintptr_t)(((uint64_t)a[1] << 32) | a[0]);
            if (rep) __hip_atomic_store(rep, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        return;
    }
    // clear the pieces for the next call, then merge (clearing first measured faster: the clears
    // are issued before the merge and drain while it runs)
    const u4 empty = u4{MB_EMPTY, MB_EMPTY, MB_EMPTY, MB_EMPTY};
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        if (l + 64 * j >= ns) continue;
        const int base = mb_piece(th, db, l + 64 * j, smax);
#pragma unroll
        for (int k = 0; k < 4; ++k) mb_store4(r, base + 4 * k, empty);
        mb_clear2(r, base + 16);
    }
    merge_wave_store<SPL>(gv, nh, t, h, ns, hv, ov, out, ots, d0, l);
}

// Decode / verify attention in one launch: the split-K partials of decode_partial (one 64-key tile
// per split) into the mailbox, then every wave merges its share of the (row, 16-dim block) units.
// The host launches it only when the whole grid is co-resident, so every piece a merge waits for is
// being produced.
template <int NB, int SPL>
__global__ __launch_bounds__(256) void attn_decode_mailbox_kernel(const float* __restrict__ q, int qts,
                                                                  const uint16_t* __restrict__ kc,
                                                                  const uint16_t* __restrict__ vc, int kvd, int pos0,
                                                                  int nh, int nkv, int nt, float scale, int chunk,
                                                                  int smax, float* mb, uint32_t mbb,
                                                                  float* __restrict__ out, int ots) {
    decode_partial<NB, false, true, true>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, nullptr, chunk, smax, blockIdx.x,
                                    blockIdx.y, blockIdx.z, mb, mbb);
    const int nwg = gridDim.x * gridDim.y * gridDim.z;
    const int wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const MbRsrc r = mb_rsrc(mb, mbb);
    for (int u = wg + nwg * (threadIdx.x >> 6); u < nt * nh * 16; u += 4 * nwg)
        mailbox_merge<SPL>(q, qts, pos0, nh, chunk, smax, r, out, ots, u >> 4, u & 15, threadIdx.x & 63);
}

// Header words 2-3 hold the device address of the mailbox's host-visible report word (0 if none);
// the fill clears that word too, in stream order after every earlier call.
__global__ __launch_bounds__(256) void mailbox_fill_kernel(uint32_t* p, size_t words, uint32_t* report) {
    const uint64_t rp = (uint64_t)(uintptr_t)report;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (size_t)gridDim.x * 256)
        p[i] = i == 1 ? MAILBOX_MAGIC : i == 2 ? (uint32_t)rp : i == 3 ? (uint32_t)(rp >> 32)
             : i < (size_t)MB_HEAD ? 0u : MB_EMPTY;
    if (report && blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(report, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

bool piece_records(int pos0, int nt, int nh, int chunk) {
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    // 9-256 splits, at most 256 rows: the wave merge on the piece layout (from 9 splits it beats the
    // row merge on 260-word records: 4 tokens at 1024 keys, 16 splits, 8.77 -> 7.79 us per call)
    return smax > 8 && smax <= 256 && (long)nt * nh <= 256;
}

hipError_t launch_attn_partials(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd,
                                       int pos0, int nh, int nkv, int nt, float scale, float* part, int chunk,
                                       hipStream_t st, bool pieces) {
    const int G = nh / nkv, R = nt * G;
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    // one tile per split (chunk <= 64 keys) needs one V buffer, so two or three workgroups share a
    // CU; verify rows are then spread over more workgroups (8 rows each up to 16 rows, 16 rows up to
    // 32: measured best at nt = 2 and nt = 4), with the K/V tile of a split read by each of them
    // from the same XCD's L2 when smax * nkv (the id distance of a split's row groups) is a
    // multiple of 8. Splits of several tiles keep the smallest block that holds all rows.
    const bool multi = chunk > TK;
    const int rows = multi ? (R <= 8 ? 8 : R <= 16 ? 16 : R <= 24 ? 24 : 32) : (R <= 16 ? 8 : R <= 32 ? 16 : 32);
    const dim3 grid(smax, nkv, (R + rows - 1) / rows);
#define IT_DECODE_LAUNCH2(NB_, CR_)                                                                                   \
    (multi ? attn_decode_kernel<NB_, true, false, CR_><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt,     \
                                                                            scale, part, chunk, smax)                   \
           : attn_decode_kernel<NB_, false, false, CR_><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt,    \
                                                                             scale, part, chunk, smax))
#define IT_DECODE_LAUNCH(NB_) (pieces ? IT_DECODE_LAUNCH2(NB_, true) : IT_DECODE_LAUNCH2(NB_, false))
    // decode rows (one block of 8) over 64 or more workgroups load V into registers (see
    // decode_partial); verify blocks measured equal either way and keep the copy
    const bool vr = !multi && rows == 8 && (long)grid.x * grid.y * grid.z >= 64;
    switch (rows / 8) {
        case 1:
            if (vr && pieces)
                attn_decode_kernel<1, false, true, true><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt,
                                                                              scale, part, chunk, smax);
            else if (vr)
                attn_decode_kernel<1, false, true><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale,
                                                                        part, chunk, smax);
            else
                IT_DECODE_LAUNCH(1);
            break;
        case 2: IT_DECODE_LAUNCH(2); break;
        case 3: IT_DECODE_LAUNCH(3); break;
        default: IT_DECODE_LAUNCH(4); break;
    }
#undef IT_DECODE_LAUNCH
#undef IT_DECODE_LAUNCH2
    return hipGetLastError();
}

size_t mailbox_bytes(long ctx, int nt, int nh) {
    const long smax = idx::split_count(ctx, TK);
    return 4 * ((size_t)MB_HEAD + (size_t)nt * nh * 16 * smax * MB_PIECE);
}

namespace {
// workgroups of one mailbox kernel instantiation that fit the device at once (cached per device)
template <int NB, int SPL>
int mailbox_capacity() {
    static std::atomic<int> cap[64];   // 0 = not yet queried
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int c = cap[dev].load(std::memory_order_relaxed);
    if (c) return c;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_decode_mailbox_kernel<NB, SPL>, 256, 0) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    c = per_cu * cus > 0 ? per_cu * cus : -1;
    cap[dev].store(c, std::memory_order_relaxed);
    return c;
}
}  // namespace

hipError_t launch_attn_decode_mailbox(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd,
                                      int pos0, int nh, int nkv, int nt, float scale, float* out, int ots, float* mb,
                                      size_t mbb, hipStream_t st, bool* launched, bool dry_run) {
    *launched = false;
    const int G = nh / nkv, R = nt * G;
    const long total = (long)pos0 + nt;
    const int smax = idx::split_count(total, TK);
    const size_t need = mailbox_bytes(total, nt, nh);
    // one group of at most 8 rows (decode): with more rows the merging waves wait beside
    // workgroups still computing, and two launches measured faster (nt = 2: 12.1 against 13.8 us,
    // nt = 4: 18.5 against 21.3 at ctx 8192)
    if (smax > 256 || R > 8 || need > mbb || need >= (1u << 31) || !mb) return hipSuccess;
    const int rows = 8;
    const dim3 grid(smax, nkv, (R + rows - 1) / rows);
    const long wgs = (long)grid.x * grid.y * grid.z;
    // every merge unit needs a wave of its own: a wave that merges several units waits a memory
    // round trip per unit (ctx 512, 16 workgroups for 256 units: 11.3 against 7.8 us for two launches)
    if ((long)nt * nh * 16 > 4 * wgs) return hipSuccess;
    const int spl = smax <= 64 ? 1 : smax <= 128 ? 2 : 4;
#define IT_MB_CASE(SPL_)                                                                                            \
    if (spl == SPL_) {                                                                                              \
        if (mailbox_capacity<1, SPL_>() < wgs) return hipSuccess;                                                   \
        *launched = true;                                                                                           \
        if (dry_run) return hipSuccess;                                                                             \
        attn_decode_mailbox_kernel<1, SPL_><<<grid, 256, 0, st>>>(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale,    \
                                                                  TK, smax, mb, (uint32_t)need, out, ots);          \
        return hipGetLastError();                                                                                   \
    }
    IT_MB_CASE(1) IT_MB_CASE(2) IT_MB_CASE(4)
#undef IT_MB_CASE
    return hipSuccess;
}

hipError_t launch_mailbox_fill(void* mb, size_t bytes, uint32_t* report, hipStream_t st) {
    const size_t words = bytes / 4;
    const unsigned blocks = (unsigned)std::min<size_t>((words + 255) / 256, 2048);
    mailbox_fill_kernel<<<blocks, 256, 0, st>>>((uint32_t*)mb, words, report);
    return hipGetLastError();
}

hipError_t launch_attn_combine(const float* q, int qts, const float* part, int pos0, int nh, int nt, int chunk,
                               float* out, int ots, hipStream_t st, bool pieces) {
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    if (pieces) {   // piece_records() holds: 8 < smax <= 256, at most 256 rows
        const unsigned wgs = (unsigned)((long)nt * nh * 16);   // one wave each
        if (smax <= 64)
            attn_combine_wave1_kernel<1><<<wgs, 64, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
        else if (smax <= 128)
            attn_combine_wave1_kernel<2><<<wgs, 64, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
        else
            attn_combine_wave1_kernel<4><<<wgs, 64, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
        return hipGetLastError();
    }
    const unsigned wgs = (unsigned)(((long)nt * nh * 16 + 3) / 4);   // 4 waves each
    // the wave merge for the few rows of decode and verify; the workgroup merge (fewer, longer
    // waves) for the many rows of a prefill chunk
    const unsigned rwgs = (unsigned)(((long)nt * nh + 3) / 4);   // one wave per row
    if (smax <= 8)
        attn_combine_row_kernel<8, false><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if (smax <= 16)
        attn_combine_row_kernel<16, false><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if ((long)nt * nh > 256 && smax <= 32)
        attn_combine_row_kernel<32, false><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if ((long)nt * nh > 256)
        attn_combine_kernel<16><<<dim3(4, nh, nt), 256, 0, st>>>(q, qts, pos0, nh, part, chunk, smax, out, ots);
    else if (smax <= 64)
        attn_combine_wave_kernel<1><<<wgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if (smax <= 128)
        attn_combine_wave_kernel<2><<<wgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if (smax <= 256)
        attn_combine_wave_kernel<4><<<wgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else
        attn_combine_kernel<16><<<dim3(4, nh, nt), 256, 0, st>>>(q, qts, pos0, nh, part, chunk, smax, out, ots);
    return hipGetLastError();
}

hipError_t launch_attn_combine_q16(const float* q, int qts, const float* part, int pos0, int nh, int nt, int chunk,
                                   float* out, int ots, hipStream_t st) {
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    const unsigned rwgs = (unsigned)(((long)nt * nh + 3) / 4);   // one wave per row
    if (smax <= 8)
        attn_combine_row_kernel<8, true><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if (smax <= 16)
        attn_combine_row_kernel<16, true><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else if (smax <= 32)
        attn_combine_row_kernel<32, true><<<rwgs, 256, 0, st>>>(q, qts, pos0, nh, nt, part, chunk, smax, out, ots);
    else
        attn_combine_kernel<16, true><<<dim3(4, nh, nt), 256, 0, st>>>(q, qts, pos0, nh, part, chunk, smax, out, ots);
    return hipGetLastError();
}

hipError_t launch_attn_splitk(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                              int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                              hipStream_t st) {
    const bool cr = piece_records(pos0, nt, nh, chunk);
    hipError_t e = launch_attn_partials(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, st, cr);
    if (e != hipSuccess) return e;
    return launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, st, cr);
}

}  // namespace it
