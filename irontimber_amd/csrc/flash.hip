// Causal GQA attention for prefill on the matrix cores (flash form: one pass over the keys, online
// softmax, no scratch). Same math as src/cpu.rs:260-272 for every query row; the reference's GPU
// counterparts are the multi-query split-K tiles of kernels/src/prefill_attention*.rs and
// kernels/src/prefill_gqa.rs.
//
// Workgroup = 128 query rows sharing one KV head (rows r = t*G + g: token t, head g of the group,
// G = nh/nkv). Per 64-key tile, in the transposed form so that every lane owns one query row:
//   S^T  = K Q^T          A = K rows from LDS, B = q (f16, pre-scaled by scale*log2 e) held in
//                         registers for the whole kernel
//   softmax              running max / sum per query in the log2 domain, lane exchanges only
//   O^T += V^T P^T        A = V^T through the LDS transpose read of the row-major V tile, B = P^T
//                         straight from the S^T accumulator (f16); O^T stays in accumulators
// K/V tiles go straight from HBM/L2 into double-buffered LDS (global_load_lds, 16 bytes per lane,
// no registers): tile t+1 streams in while tile t is computed, one barrier per tile.
// Two forms of the same tile:
//   attn_flash_kernel     4 waves of 32 rows, 32x32x16 matrix ops, one wave per SIMD: each
//                         transpose read of V serves 32 queries. One-pass launches of at least
//                         a workgroup per CU (long prompts), which the LDS bytes per tile bound.
//   attn_flash_w8_kernel  8 waves of 16 rows, 16x16x32 matrix ops, two waves per SIMD, so one
//                         wave's softmax and waits overlap the other's matrix ops. Key-split
//                         launches and short one-pass launches, bound by latency.
//
// Key-split form (part != null, attn_flash_w8_kernel): workgroup (row tile, KV head, split s)
// covers keys [s*chunk, (s+1)*chunk) only and writes a partial record of each of its rows for the
// merge kernel: the {m, l} of the decode partials (kernels/src/lib.rs:753-798) plus a scale k, and
// O as int16 in units of k (FLASH_REC words a record: the O runs and the headers in two regions,
// rec_index.h flash_o / flash_h). Used when one pass would leave most CUs idle: a 64-token
// chunk after a long context has only 2 * ceil(64*G/128) row tiles.
#include "common.h"
#include "internal.h"

namespace it {

namespace {
constexpr int HD = 256;
constexpr int BM = 128, BN = 64, RW = 16;   // rows per workgroup, keys per tile, rows per wave
constexpr float RESCALE_SLACK = 8.0f;   // log2 units
}

// ---- four waves of 32 query rows (32x32x16 matrix ops)
// LDS tiles are unpadded 512-byte rows of 32 16-byte chunks; logical chunk j of row r lives at
// physical chunk j ^ swz32(r). With 512-byte rows a chunk's bank group is (chunk mod 16), so swz32
// gives 16 consecutive rows 16 distinct values (K operand reads: one row per lane) and 4
// consecutive rows distinct chunk pairs (V transpose reads: 4 rows x 2 chunks per 16 lanes).
__device__ __forceinline__ int swz32(int r) { return ((r & 3) << 1) | ((r >> 2) & 1) | (((r >> 3) & 1) << 3); }

// Issue the direct-to-LDS loads of one 64-row tile: wave w moves rows 16w..16w+15, two rows
// (64 lanes x 16 bytes) per instruction, each lane fetching the logical chunk that belongs at its
// physical slot. Rows past kend-1 repeat row kend-1 (a tile issued past the end only refetches it).
// Addresses are a uniform row base plus a 32-bit lane offset, so each instruction needs two VALU
// ops; the chunk part of the offsets (cj, including the head's column) is computed once.
__device__ __forceinline__ void tile_to_lds32(const uint16_t* __restrict__ src, int kvd, int kb, int kend,
                                            const int (&cj)[8], _Float16* lds, int w, int l) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int ts = min(kb, kend - 1);                      // first row of the tile, clamped
    const char* base = (const char*)(src + (size_t)ts * kvd);
    const int rmax = kend - 1 - ts;                        // >= 0
    const unsigned rowb = 2u * (unsigned)kvd;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 16 * w + 2 * i + (l >> 5);
        const unsigned off = (unsigned)min(r, rmax) * rowb + (unsigned)cj[i];
        __builtin_amdgcn_global_load_lds((const void*)(base + off), (lds_void*)(lds + (16 * w + 2 * i) * HD), 16, 0, 0);
    }
}

// acc *= a for an MFMA accumulator tile held in AGPRs, element by element in place (read to a VGPR,
// multiply, write back). Written out so the accumulators never need a VGPR home: with a plain
// multiply in the (rare) rescale branch the register allocator keeps them in VGPRs at the branch
// merge and the common path copies all of them to VGPRs and back on every tile.
__device__ __forceinline__ void scale_acc(f16v& acc, float a) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float x = acc[i], t;
        asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32_e32 %1, %2, %1\n\tv_accvgpr_write_b32 %0, %1"
                     : "+a"(x), "=&v"(t)
                     : "v"(a));
        acc[i] = x;
    }
}

// One pass over the keys (no records), for launches of at least a workgroup per CU, where each
// V transpose read serving 32 queries keeps the tile below the LDS bound of the 16-row form.
// QM: where the q operand comes from. 0: the f32 q rows, scaled and converted here. 2: q16,
// pre-converted (q16[t][h][d] = f16(q * scale * log2 e), exactly what that conversion makes, from
// it_attn_prep_f16_q16), half the bytes, read as whole rows and transposed through LDS as QM 0
// does; q still provides the gates.
template <int QM>
__global__ __launch_bounds__(256) void attn_flash_kernel(
    const float* __restrict__ q, int qts, const _Float16* __restrict__ q16, int q16ts, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int kvd, int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ out,
    int ots) {
    static_assert(QM == 0 || QM == 2, "one-pass launches read q as whole rows");
    // two K and two V buffers as distinct objects, so the compiler can tell that the loads
    // streaming into one buffer never alias the reads of the other (no conservative waits)
    __shared__ __align__(16) _Float16 K0[BN * HD];
    __shared__ __align__(16) _Float16 K1[BN * HD];
    __shared__ __align__(16) _Float16 V0[BN * HD];
    __shared__ __align__(16) _Float16 V1[BN * HD];

    const int G = nh / nkv, R = nt * G;
    const int nrt = (R + BM - 1) / BM;
    const int rt = nrt - 1 - (int)blockIdx.x;          // heaviest row tile first
    const int kh = blockIdx.y;
    // the wave index as a scalar: row counts, row walks and branches on them stay in SGPRs
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, hh = l >> 5, c = l & 31;
    const int r = rt * BM + 32 * w + c;                 // this lane's query row
    const bool rvalid = r < R;
    const int t = rvalid ? r / G : 0;
    const int tmin = (rt * BM) / G, tmax = (min(R, rt * BM + BM) - 1) / G;
    const int kb0 = 0, kend = pos0 + tmax + 1;          // this workgroup's keys: [0, kend)
    const int kfull = pos0 + tmin + 1;                  // keys every row of the tile sees
    const int qlim = pos0 + t;                          // this row sees keys <= qlim
    const size_t head_off = (size_t)kh * HD;

    // q as the B operand: column = query c, k = dims 16*ks + 8*hh + 0..7, scaled into log2 units.
    // Wave w reads its 32 rows whole (one 1 KB row per load instruction: a per-lane gather of the
    // operand layout would touch 32 rows per instruction), then transposes them through its own
    // 16 KB of the second K/V buffers, which the first tile does not use (rows XOR-swizzled by
    // 16-byte chunk so the operand reads of 32 rows hit distinct banks). The q loads go out before
    // the first tile's, so the prologue costs one memory round trip.
    // byte offset of the logical chunk each lane's DMA slot holds, plus the KV head's column
    int cj[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cj[i] = 2 * (int)head_off + 16 * ((l & 31) ^ swz32(16 * w + 2 * i + (l >> 5)));
    h8 qb[16];
    if constexpr (QM == 2) {
        // two 512-byte rows per load instruction (lanes 0-31 row 2j, lanes 32-63 row 2j + 1 of the
        // wave's 32; rows past R zero), then the transpose through LDS the f32 rows take below: whole
        // rows keep the loads coalesced (a per-lane gather of the operand layout touches 32 rows per
        // instruction)
        h8 qx[16];
        const int rw = __builtin_amdgcn_readfirstlane(rt * BM + 32 * w);   // even: BM, 32 are
        int te = __builtin_amdgcn_readfirstlane(rw / G), ge = rw - te * G;   // row 2j
        int to = te, go = ge + 1;                                           // row 2j + 1
        if (go == G) { go = 0; ++to; }
        const int hi = l >> 5;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const size_t oe = uniform_off((size_t)te * q16ts + (size_t)(kh * G + ge) * HD);
            const size_t oo = uniform_off((size_t)to * q16ts + (size_t)(kh * G + go) * HD);
            const bool valid = rw + 2 * j + hi < R;
            const h8 v = ld_h8(q16 + (valid ? (hi ? oo : oe) : 0) + 8 * (l & 31));
            qx[j] = valid ? v : h8{};
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (++ge == G) { ge = 0; ++te; }
                if (++go == G) { go = 0; ++to; }
            }
        }
        tile_to_lds32(kc, kvd, kb0, kend, cj, K0, w, l);
        tile_to_lds32(vc, kvd, kb0, kend, cj, V0, w, l);
        _Float16* qs = (w < 2 ? K1 : V1) + (w & 1) * (32 * HD);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = 2 * j + hi;
            *(h8*)(qs + i * HD + 8 * ((l & 31) ^ i)) = qx[j];
        }
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qb[ks] = ld_h8(qs + c * HD + 8 * ((2 * ks + hh) ^ c));
    } else {
        f4 qx[32];
        const int rw = __builtin_amdgcn_readfirstlane(rt * BM + 32 * w);
        // row rr = token rr / G, q-head kh*G + rr % G: one division, then a walk over the 32 rows
        // (a division per row costs ~40 instructions, ~10k cycles over the unrolled loop). The
        // row offsets are scalar (uniform_off): per-row 64-bit vector address arithmetic cost
        // ~60 cycles a row.
        int tq = __builtin_amdgcn_readfirstlane(rw / G), gq = rw - tq * G;
        const float* qlast = q + uniform_off((size_t)((R - 1) / G) * qts + (size_t)(kh * G + (R - 1) % G) * 2 * HD);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            // rows past R: any valid row (the last), zeroed below
            const float* src = rw + i < R ? q + uniform_off((size_t)tq * qts + (size_t)(kh * G + gq) * 2 * HD) : qlast;
            qx[i] = ld_f4(src + 4 * l);
            if (++gq == G) { gq = 0; ++tq; }
        }
        tile_to_lds32(kc, kvd, kb0, kend, cj, K0, w, l);
        tile_to_lds32(vc, kvd, kb0, kend, cj, V0, w, l);
        _Float16* qs = (w < 2 ? K1 : V1) + (w & 1) * (32 * HD);
        const float sc = scale * LOG2E;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float si = rw + i < R ? sc : 0.0f;
            const h4 hv = {(_Float16)(qx[i][0] * si), (_Float16)(qx[i][1] * si), (_Float16)(qx[i][2] * si),
                           (_Float16)(qx[i][3] * si)};
            *(h4*)(qs + i * HD + 8 * ((l >> 1) ^ i) + 4 * (l & 1)) = hv;
        }
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qb[ks] = ld_h8(qs + c * HD + 8 * ((2 * ks + hh) ^ c));
    }
    f16v o[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] = f16v{};
    float m_run = -INFINITY, l_run = 0.f;

    // Per-lane LDS offsets (halves). K operand: row c (+32 per block), logical chunk 2ks+hh.
    int koff[8];
    {
        const int sw = swz32(c);          // swz32(32b + c) == swz32(c)
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) koff[k2] = c * HD + 8 * ((2 * k2 + hh) ^ sw);
    }
    // V transpose read: source lane provides row 4hh + vrow (+16ks, +8 for the second half) and
    // logical column 32db + vcol; swz of those rows is (vrow << 1) | hh for every ks.
    int voff[4][2];
    {
        const int vrow = (l & 15) >> 2, vcol = 16 * ((l >> 4) & 1) + 4 * (l & 3);
        const int jj = vcol >> 3, inner = vcol & 7;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            // rows 16ks + 4hh + vrow (+8 for the second transpose read): swz depends on bit 3 too
            const int r = 4 * hh + vrow + 8 * half;
            const int sv = swz32(r);
#pragma unroll
            for (int par = 0; par < 4; ++par) voff[par][half] = r * HD + 8 * ((4 * par + jj) ^ sv) + inner;
        }
    }

    // one 64-key tile: K/V hold tile kb (issued one tile earlier); tile kb+BN streams into Kn/Vn
    auto tile = [&](int kb, const _Float16* K, const _Float16* V, _Float16* Kn, _Float16* Vn) {
        // tile kb has landed for this wave; after the barrier for every wave, and every wave is
        // done with the buffers that tile kb+BN goes into
        IT_WAIT_VMCNT(0);
        __syncthreads();
        // the next tile streams in while this one is computed; issued unconditionally (past the end
        // it refetches row kend-1 into the idle buffers) so the loads stay in the same basic block
        // as the S^T matrix ops and the scheduler can spread them between those
        tile_to_lds32(kc, kvd, kb + BN, kend, cj, Kn, w, l);
        tile_to_lds32(vc, kvd, kb + BN, kend, cj, Vn, w, l);
        // ---- S^T = K Q^T for two 32-key blocks. Logical chunk 2ks+hh of row rr sits at physical
        // chunk 16*(ks/8) + ((2*(ks%8) + hh) ^ swz32(rr)): eight per-lane offsets plus immediates.
        f16v sc[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) sc[b] = f16v{};
#pragma unroll
        for (int ks = 0; ks < 16; ++ks)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                sc[b] = mfma32x32x16(ld_h8(K + (32 * b) * HD + koff[ks & 7] + 128 * (ks >> 3)), qb[ks], sc[b]);
        // eight operand reads in flight ahead of the matrix cores, and the next tile's 16 loads
        // spread one per two matrix ops (each occupies the CU's load path for ~16 cycles per wave)
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 24; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (i < 16) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        // ---- causal mask (only tiles that reach past the first row's diagonal)
        if (kb + BN > kfull) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kb + 32 * b + 8 * (i >> 2) + 4 * hh + (i & 3);
                    if (!rvalid || key > qlim) sc[b][i] = -INFINITY;
                }
        }
        // ---- online softmax in the log2 domain with a lazily raised reference max: m_run only
        // moves when a row's max exceeds it by more than RESCALE_SLACK, so O and l are rescaled
        // on few tiles; P = 2^(s - m_run) <= 2^RESCALE_SLACK stays exact enough in f16 and the
        // final O / l does not depend on the reference.
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sc[b][i]);
        mx = max_xor32(mx);
        const bool grow = mx > m_run + RESCALE_SLACK;
        if (__any(grow)) {
            const float mnew = grow ? mx : m_run;
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - mnew);
            l_run *= alpha;
            // the previous tile's last P.V matrix ops may still be writing O. The ISA requires, after
            // an XDL matrix op that writes accumulation registers, (passes + 2) wait states before a
            // v_accvgpr_read of them: 18 for the 16-pass 32x32x16 f16 op. scale_acc is inline assembly,
            // which the compiler's hazard recognizer does not look into, so the wait is explicit:
            // four s_nop 7 give 32 wait states. Too few would scale a stale O on the rare tiles
            // where a row's reference max grows (every prefill parity test crosses such tiles).
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
#pragma unroll
            for (int db = 0; db < 8; ++db) scale_acc(o[db], alpha);
            m_run = mnew;
        }
        const float msub = (m_run == -INFINITY) ? 0.0f : m_run;
        float lsum = 0.f;
        h8 pb[4];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(sc[b][8 * kk + j] - msub);
                    lsum += p;
                    pb[2 * b + kk][j] = (_Float16)p;
                }
        l_run += lsum;   // this lane half's keys only; the halves are added after the loop
        // ---- O^T += V^T P^T: k-step ks covers keys 16ks + {4hh + 0..3, 8 + 4hh + 0..3}; the
        // transpose-read address is voff[db & 3][half] plus immediates
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const _Float16* v = V + (16 * ks) * HD + 128 * (db >> 2);
                const h8 va = cat_h4(lds_tr4(v + voff[db & 3][0]), lds_tr4(v + voff[db & 3][1]));
                o[db] = mfma32x32x16(va, pb[ks], o[db]);
            }
        // four operands (eight transpose reads) in flight ahead of the matrix cores
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 28; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    };
    for (int kb = kb0; kb < kend; kb += 2 * BN) {
        tile(kb, K0, V0, K1, V1);
        if (kb + BN < kend) tile(kb + BN, K1, V1, K0, V0);
    }
    // ---- epilogue. Lane (c, hh) holds O^T of query c at dims 32db + 8*(i/4) + 4hh + (i&3); wave w
    // stages its 32 rows x 256 f32 in its own 32 KB of the tile buffers (16-byte chunk index XOR
    // row, conflict-free), then writes whole rows: one 1 KB row per store instruction.
    IT_WAIT_VMCNT(0);  // the loads issued past the end land in the buffers staged below
    __syncthreads();   // every wave is done with the last tile
    float* os = (float*)(w == 0 ? K0 : w == 1 ? K1 : w == 2 ? V0 : V1);
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const int ch = (32 * db + 8 * i4 + 4 * hh) >> 2;   // 16-byte chunk of the row
            *(f4*)(os + c * HD + 4 * (ch ^ c)) = f4{o[db][4 * i4], o[db][4 * i4 + 1], o[db][4 * i4 + 2], o[db][4 * i4 + 3]};
        }
    __shared__ __align__(16) float ml[4][32];   // per wave: the sum of each of its 32 queries
    l_run = sum_xor32(l_run);
    if (hh == 0) ml[w][c] = l_run;
    const int rw = __builtin_amdgcn_readfirstlane(rt * BM + 32 * w);
    const int nrow = min(32, R - rw);
    int tq = __builtin_amdgcn_readfirstlane(rw / G), gq = rw - tq * G;   // (token, q-head) of row rw + i
    // out = O / l * sigmoid(gate), gate rows read whole as well; eight rows per step (their gate
    // loads wait for the previous step's stores, which share the counter: 14.0k / 12.0k / 11.3k
    // cycles per workgroup at 2 / 4 / 8 rows per step; all 32 gates issued up front measured 24.7k)
#pragma unroll 8
    for (int i = 0; i < nrow; ++i) {
        const int tt = tq, hd = kh * G + gq;
        if (++gq == G) { gq = 0; ++tq; }
        const f4 gt = ld_f4(q + (size_t)tt * qts + (size_t)hd * 2 * HD + HD + 4 * l);
        const f4 ov = *(const f4*)(os + i * HD + 4 * (l ^ i));
        // the gate through the hardware exp2 and reciprocal: with accurate expf and division this
        // loop (128 gates a lane) took ~19k cycles per workgroup, more than a whole short chunk's
        // tiles; the output changes by ~1e-7 relative
        const float inv = __builtin_amdgcn_rcpf(ml[w][i]);
        f4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = ov[j] * inv * sigmoid_hw(gt[j]);
        *(f4*)(out + (size_t)tt * ots + (size_t)hd * HD + 4 * l) = v;
    }
}

// ---- eight waves of 16 query rows (16x16x32 matrix ops)
// LDS tiles are unpadded 512-byte rows of 32 16-byte chunks; logical chunk j of row r lives at
// physical chunk j ^ swz16(r) (swz16 < 16). A chunk's bank group is (chunk mod 16). The score reads
// (one K row per lane, 16 lanes at a time) take rows that differ in bits 0, 1, 3 and 4, and the V
// transpose reads (4 rows x 2 chunks per 16 lanes, 32 lanes at a time) rows that differ in bits 0,
// 1 and 3: swz16 maps bits 0, 1, 3 to its bits 1-3 and bit 4 to its bit 0, so both patterns hit 16
// distinct bank groups.
__device__ __forceinline__ int swz16(int r) { return ((r & 3) << 1) | (((r >> 3) & 1) << 3) | ((r >> 4) & 1); }

// Issue the direct-to-LDS loads of one 64-row tile: wave w moves rows 8w..8w+7, two rows (64 lanes
// x 16 bytes) per instruction, each lane fetching the logical chunk that belongs at its physical
// slot. Rows past kend-1 repeat row kend-1 (a tile issued past the end only refetches it).
// Addresses are a uniform row base plus a 32-bit lane offset; the chunk part of the offsets (cj,
// including the head's column) is computed once.
__device__ __forceinline__ void tile_to_lds16(const uint16_t* __restrict__ src, int kvd, int kb, int kend,
                                            const int (&cj)[4], _Float16* lds, int w, int l) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int ts = min(kb, kend - 1);                      // first row of the tile, clamped
    const char* base = (const char*)(src + (size_t)ts * kvd);
    const int rmax = kend - 1 - ts;                        // >= 0
    const unsigned rowb = 2u * (unsigned)kvd;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * w + 2 * i + (l >> 5);
        const unsigned off = (unsigned)min(r, rmax) * rowb + (unsigned)cj[i];
        __builtin_amdgcn_global_load_lds((const void*)(base + off), (lds_void*)(lds + (8 * w + 2 * i) * HD), 16, 0, 0);
    }
}

// Two waves per SIMD (about 210 registers each), so one wave's softmax, waits and barrier overlap
// the other's matrix ops; each V transpose read serves 16 queries, so a tile moves twice the LDS
// bytes of the 32-row form. For key-split launches and one-pass launches of fewer workgroups than
// CUs, which are bound by each workgroup's chain of dependent phases rather than by LDS.
// F32REC: the key-split records in the split-K kernels' lossless f32 form instead ({m, l, 0, 0} +
// O as 256 floats, 260 words, merged by the f32 combine), selectable through it_attn_f16_ex.
// QM: where the q operand comes from. 0: the f32 q rows, scaled and converted here. 1 and 2: q16,
// pre-converted (q16[t][h][d] = f16(q * scale * log2 e), exactly what that conversion makes, from
// it_attn_prep_f16_q16), half the bytes; q still provides the gates. 1 gathers each lane's operand
// straight from global, no transpose through LDS: for key-split launches, whose q rows are re-read
// by every split from L2. 2 reads whole rows and transposes them through LDS as QM 0 does: for
// one-pass launches, which read q once from memory, where a per-lane gather touches 16 rows per
// instruction.
template <bool F32REC, int QM>
__global__ __launch_bounds__(512) void attn_flash_w8_kernel(
    const float* __restrict__ q, int qts, const _Float16* __restrict__ q16, int q16ts, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int kvd, int pos0, int nh, int nkv, int nt, float scale, float* __restrict__ out,
    int ots, float* __restrict__ part, int chunk, int smax) {
    // two K and two V buffers as distinct objects, so the compiler can tell that the loads
    // streaming into one buffer never alias the reads of the other (no conservative waits)
    __shared__ __align__(16) _Float16 K0[BN * HD];
    __shared__ __align__(16) _Float16 K1[BN * HD];
    __shared__ __align__(16) _Float16 V0[BN * HD];
    __shared__ __align__(16) _Float16 V1[BN * HD];

    const int G = nh / nkv, R = nt * G;
    const int nrt = (R + BM - 1) / BM;
    const int rt = nrt - 1 - (int)blockIdx.x;          // heaviest row tile first
    const int kh = blockIdx.y;
    // the wave index as a scalar: row counts, row walks and branches on them stay in SGPRs
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 4, c = l & 15;
    const int r = rt * BM + RW * w + c;                 // this lane's query row
    const bool rvalid = r < R;
    const int t = rvalid ? r / G : 0;
    const int tmin = (rt * BM) / G, tmax = (min(R, rt * BM + BM) - 1) / G;
    const int split = blockIdx.z;
    const int kb0 = part ? split * chunk : 0;           // this workgroup's keys: [kb0, kend)
    const int kend = part ? min(pos0 + tmax + 1, kb0 + chunk) : pos0 + tmax + 1;
    if (kb0 >= kend) return;                            // no row of the tile sees these keys
    const int kfull = pos0 + tmin + 1;                  // keys every row of the tile sees
    const int qlim = pos0 + t;                          // this row sees keys <= qlim
    const size_t head_off = (size_t)kh * HD;

    // byte offset of the logical chunk each lane's DMA slot holds, plus the KV head's column
    int cj[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cj[i] = 2 * (int)head_off + 16 * ((l & 31) ^ swz16(8 * w + 2 * i + (l >> 5)));
    // q as the B operand of S^T = K Q^T: lane (c, g) holds dims 32ks + 8g .. +7 of query row c,
    // scaled into log2 units. QM 0 and 2 read the wave's 16 rows whole and transpose them through
    // the wave's own 8 KB of the second K/V buffers, which the first tile does not use (16-byte
    // chunk index XOR row, so the operand reads of 16 rows hit distinct banks). The q loads go out
    // before the first tile's, so the prologue costs one memory round trip.
    h8 qb[8];
    _Float16* qs = (w < 4 ? K1 : V1) + (w & 3) * (RW * HD);
    if constexpr (QM == 1) {
        const int rr = rvalid ? r : R - 1;
        const _Float16* qrow = q16 + (size_t)(rr / G) * q16ts + (size_t)(kh * G + rr % G) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const h8 v = ld_h8(qrow + 32 * ks);
            qb[ks] = rvalid ? v : h8{};
        }
        tile_to_lds16(kc, kvd, kb0, kend, cj, K0, w, l);
        tile_to_lds16(vc, kvd, kb0, kend, cj, V0, w, l);
    } else if constexpr (QM == 2) {
        // two 512-byte rows per load instruction (lanes 0-31 row 2j, lanes 32-63 row 2j + 1 of the
        // wave's 16; rows past R zero)
        h8 qx[8];
        const int rw = __builtin_amdgcn_readfirstlane(rt * BM + RW * w);   // even: BM, RW are
        int te = __builtin_amdgcn_readfirstlane(rw / G), ge = rw - te * G;   // row 2j
        int to = te, go = ge + 1;                                           // row 2j + 1
        if (go == G) { go = 0; ++to; }
        const int hi = l >> 5;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const size_t oe = uniform_off((size_t)te * q16ts + (size_t)(kh * G + ge) * HD);
            const size_t oo = uniform_off((size_t)to * q16ts + (size_t)(kh * G + go) * HD);
            const bool valid = rw + 2 * j + hi < R;
            const h8 v = ld_h8(q16 + (valid ? (hi ? oo : oe) : 0) + 8 * (l & 31));
            qx[j] = valid ? v : h8{};
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (++ge == G) { ge = 0; ++te; }
                if (++go == G) { go = 0; ++to; }
            }
        }
        tile_to_lds16(kc, kvd, kb0, kend, cj, K0, w, l);
        tile_to_lds16(vc, kvd, kb0, kend, cj, V0, w, l);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = 2 * j + hi;
            *(h8*)(qs + i * HD + 8 * ((l & 31) ^ i)) = qx[j];
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qb[ks] = ld_h8(qs + c * HD + 8 * ((4 * ks + g) ^ c));
    } else {
        f4 qx[RW];
        const int rw = __builtin_amdgcn_readfirstlane(rt * BM + RW * w);
        // row rr = token rr / G, q-head kh*G + rr % G: one division, then a walk over the 16 rows.
        // The row offsets are scalar (uniform_off): per-row 64-bit vector address arithmetic costs
        // ~60 cycles a row.
        int tq = __builtin_amdgcn_readfirstlane(rw / G), gq = rw - tq * G;
        const float* qlast = q + uniform_off((size_t)((R - 1) / G) * qts + (size_t)(kh * G + (R - 1) % G) * 2 * HD);
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            // rows past R: any valid row (the last), zeroed below
            const float* src = rw + i < R ? q + uniform_off((size_t)tq * qts + (size_t)(kh * G + gq) * 2 * HD) : qlast;
            qx[i] = ld_f4(src + 4 * l);
            if (++gq == G) { gq = 0; ++tq; }
        }
        tile_to_lds16(kc, kvd, kb0, kend, cj, K0, w, l);
        tile_to_lds16(vc, kvd, kb0, kend, cj, V0, w, l);
        const float sc = scale * LOG2E;
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const float si = rw + i < R ? sc : 0.0f;
            const h4 hv = {(_Float16)(qx[i][0] * si), (_Float16)(qx[i][1] * si), (_Float16)(qx[i][2] * si),
                           (_Float16)(qx[i][3] * si)};
            *(h4*)(qs + i * HD + 8 * ((l >> 1) ^ i) + 4 * (l & 1)) = hv;
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qb[ks] = ld_h8(qs + c * HD + 8 * ((4 * ks + g) ^ c));
    }
    f4 o[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) o[db] = f4{};
    float m_run = -INFINITY, l_run = 0.f;

    // Score block b (16 keys) puts key 32(b>>1) + 4(b&1) + 8(m>>2) + (m&3) in matrix row m, so the
    // accumulator of lane (c, g), rows 4g..4g+3, holds keys 32(b>>1) + 4(b&1) + 8g + 0..3: blocks
    // 2kk and 2kk+1 together give the 8 consecutive keys 32kk + 8g .. +7 that the P^T operand of
    // the kk-th P.V step needs in the lane. K operand: row krow(b, c), logical chunk 4ks + g; swz of
    // those rows does not depend on b.
    int koff[4];
    {
        const int rk = 8 * (c >> 2) + (c & 3);
        const int sw = swz16(rk);
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) koff[k4] = rk * HD + 8 * ((4 * k4 + g) ^ sw);
    }
    // V transpose read: source lane s = l & 15 of group g provides row 8g + (s>>2) (+4 for the
    // second read, +32 per P.V step) and logical columns 16db + 4(s&3) .. +3; swz of those rows
    // does not depend on the +4 / +32.
    int voff[8];
    {
        const int s = l & 15, rv = 8 * g + (s >> 2), sw = swz16(rv);
#pragma unroll
        for (int d8 = 0; d8 < 8; ++d8) voff[d8] = rv * HD + 8 * ((2 * d8 + ((s & 3) >> 1)) ^ sw) + 4 * (s & 1);
    }

    // one 64-key tile: K/V hold tile kb (issued one tile earlier); tile kb+BN streams into Kn/Vn
    auto tile = [&](int kb, const _Float16* K, const _Float16* V, _Float16* Kn, _Float16* Vn) {
        // tile kb has landed for this wave; after the barrier for every wave, and every wave is
        // done with the buffers that tile kb+BN goes into
        IT_WAIT_VMCNT(0);
        __syncthreads();
        // the next tile streams in while this one is computed; issued unconditionally (past the end
        // it refetches row kend-1 into the idle buffers)
        tile_to_lds16(kc, kvd, kb + BN, kend, cj, Kn, w, l);
        tile_to_lds16(vc, kvd, kb + BN, kend, cj, Vn, w, l);
        // ---- S^T = K Q^T, four 16-key blocks
        f4 sc[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) sc[b] = f4{};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                sc[b] = mfma16x16x32(ld_h8(K + (4 * (b & 1) + 32 * (b >> 1)) * HD + koff[ks & 3] + 128 * (ks >> 2)),
                                     qb[ks], sc[b]);
        // eight operand reads in flight ahead of the matrix ops, and the next tile's 8 loads spread
        // one per three matrix ops
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 24; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (i % 3 == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        // ---- causal mask (only tiles that reach past the first row's diagonal)
        if (kb + BN > kfull) {
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb + 32 * (b >> 1) + 4 * (b & 1) + 8 * g + i;
                    if (!rvalid || key > qlim) sc[b][i] = -INFINITY;
                }
        }
        // ---- online softmax in the log2 domain with a lazily raised reference max: m_run only
        // moves when a row's max exceeds it by more than RESCALE_SLACK, so O and l are rescaled
        // on few tiles; P = 2^(s - m_run) <= 2^RESCALE_SLACK stays exact enough in f16 and the
        // final O / l does not depend on the reference.
        float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                         fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
        mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(sc[2][0], sc[2][1]), fmaxf(sc[2][2], sc[2][3])),
                             fmaxf(fmaxf(sc[3][0], sc[3][1]), fmaxf(sc[3][2], sc[3][3]))));
        mx = max_xor32(max_xor16(mx));
        const bool grow = mx > m_run + RESCALE_SLACK;
        if (__any(grow)) {
            const float mnew = grow ? mx : m_run;
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - mnew);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 16; ++db) o[db] *= alpha;
            m_run = mnew;
        }
        const float msub = (m_run == -INFINITY) ? 0.0f : m_run;
        float lsum = 0.f;
        h8 pb[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(sc[2 * kk + (j >> 2)][j & 3] - msub);
                lsum += p;
                pb[kk][j] = (_Float16)p;
            }
        l_run += lsum;   // this lane group's keys only; the groups are added after the loop
        // ---- O^T += V^T P^T: step kk covers keys 32kk + 8g + 0..7 in lane group g
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int db = 0; db < 16; ++db) {
                const _Float16* v = V + (32 * kk) * HD + 128 * (db >> 3);
                const h8 va = cat_h4(lds_tr4(v + voff[db & 7]), lds_tr4(v + 4 * HD + voff[db & 7]));
                o[db] = mfma16x16x32(va, pb[kk], o[db]);
            }
        // four operands (eight transpose reads) in flight ahead of the matrix ops
#pragma unroll
        for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 28; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    };
    for (int kb = kb0; kb < kend; kb += 2 * BN) {
        tile(kb, K0, V0, K1, V1);
        if (kb + BN < kend) tile(kb + BN, K1, V1, K0, V0);
    }
    // ---- epilogue. Lane (c, g) holds O^T of query c at dims 16db + 4g + 0..3; wave w stages its
    // 16 rows x 256 f32 in its own 16 KB of the tile buffers (16-byte chunk index XOR row,
    // conflict-free), then writes whole rows: one 1 KB row per store instruction.
    IT_WAIT_VMCNT(0);  // the loads issued past the end land in the buffers staged below
    __syncthreads();   // every wave is done with the last tile
    float* os = (float*)(w < 2 ? K0 : w < 4 ? K1 : w < 6 ? V0 : V1) + (w & 1) * (RW * HD);
    // max |O| over the lane's 64 dims of its row (the int16 record scale), taken on the bit
    // patterns of |O|: NaN patterns sort above infinity, so a NaN or infinite O (from a NaN or
    // infinite V) reaches the record's scale and the merged output instead of being quantised
    // away (a float maximum would skip a NaN)
    uint32_t abits = 0u;
#pragma unroll
    for (int db = 0; db < 16; ++db) {
        const int ch = 4 * db + g;   // 16-byte chunk of the row
        *(f4*)(os + c * HD + 4 * (ch ^ c)) = o[db];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = __builtin_bit_cast(u4, o[db])[j] & 0x7fffffffu;
            abits = b > abits ? b : abits;
        }
    }
    __shared__ __align__(16) float ml[8][3][RW];   // per wave: running max, sum and max |O| of its 16 queries
    l_run = sum_xor32(sum_xor16(l_run));
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        float a = __builtin_bit_cast(float, abits), b = a;
        if (k == 0) swap16(a, b); else swap32(a, b);   // this lane's and its partner's, in some order
        const uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
        abits = ua > ub ? ua : ub;
    }
    const float amax = __builtin_bit_cast(float, abits);
    if (g == 0) { ml[w][0][c] = m_run; ml[w][1][c] = l_run; ml[w][2][c] = amax; }
    const int rw = __builtin_amdgcn_readfirstlane(rt * BM + RW * w);
    const int nrow = min(RW, R - rw);
    int tq = __builtin_amdgcn_readfirstlane(rw / G), gq = rw - tq * G;   // (token, q-head) of row rw + i
    if (F32REC && part) {
        // f32 records of (token, head, split), 260 words each: {m, l, 0, 0}, then O
        if (l < nrow) {
            const int tl = (rw + l) / G, gl = rw + l - tl * G;
            float* rec = part + idx::rec(tl * nh + kh * G + gl, split, smax) * idx::PART;
            __builtin_nontemporal_store(f4{ml[w][0][l] * 0.6931471805599453f, ml[w][1][l], 0.f, 0.f}, (f4*)rec);
        }
        size_t ridx = idx::rec(tq * nh + kh * G + gq, split, smax);
        const size_t rnext = (size_t)(nh - G + 1) * smax;
        for (int i = 0; i < nrow; ++i) {
            const f4 ov = *(const f4*)(os + i * HD + 4 * (l ^ i));
            __builtin_nontemporal_store(ov, (f4*)(part + uniform_off(ridx * idx::PART + 4)) + l);
            if (++gq == G) { gq = 0; ridx += rnext; } else { ridx += smax; }
        }
        return;
    }
    if (part) {
        // partial records of (token, head, split), FLASH_REC words each: O as 256 int16 in a
        // 512-byte run of its own (whole cache lines: no line is shared with another split's
        // record, which another workgroup writes), the header in a packed region: {m, l, k, 0} with m in
        // natural-log units of the scaled score and k = max|O| / 32767, then O as int16 in units of
        // k (v_cvt_pk_norm_i16_f32 of O / max|O|): error <= max|O| / 65534 per value, half the
        // bytes of an f32 record. Stored non-temporally.
        // All 16 staged rows are read before any store (the accumulators are dead, so the
        // registers are free). Lane i < nrow writes row i's header. Each row's record base is
        // scalar and its 1 / max|O| comes from a lane that owns the row (lanes c, c + 16, c + 32
        // and c + 48 all hold row c's maximum), so a row costs a few vector instructions.
        if (l < nrow) {
            const int tl = (rw + l) / G, gl = rw + l - tl * G;
            float* rec = part + idx::flash_h(nt * nh, tl * nh + kh * G + gl, split, smax);
            __builtin_nontemporal_store(f4{ml[w][0][l] * 0.6931471805599453f, ml[w][1][l], ml[w][2][l] * (1.0f / 32767.0f), 0.f},
                                        (f4*)rec);
        }
        const float inv_c = amax > 0.f ? __builtin_amdgcn_rcpf(amax) : 0.f;   // row c
        f4 ov[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) ov[i] = *(const f4*)(os + i * HD + 4 * (l ^ i));
        // record index of row rw + i, walked in scalar registers: +smax within a token, and past
        // the other KV heads' q-heads at a token boundary
        size_t ridx = idx::rec(tq * nh + kh * G + gq, split, smax);
        const size_t rnext = (size_t)(nh - G + 1) * smax;
        auto put = [&](int i) {
            u2* dst = (u2*)(part + uniform_off(ridx * 128));   // idx::flash_o of record ridx
            const float inv = readlane_f(inv_c, i);
            u2 pk;
            pk[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(ov[i][0] * inv, ov[i][1] * inv));
            pk[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pknorm_i16(ov[i][2] * inv, ov[i][3] * inv));
            __builtin_nontemporal_store(pk, dst + l);
            if (++gq == G) { gq = 0; ridx += rnext; } else { ridx += smax; }
        };
        // a full 16-row wave (every wave when the row count is a multiple of 128) runs the rows
        // as one straight block, so their conversions and stores interleave
        if (nrow == RW) {
#pragma unroll
            for (int i = 0; i < RW; ++i) put(i);
        } else {
#pragma unroll
            for (int i = 0; i < RW; ++i)
                if (i < nrow) put(i);
        }
        return;
    }
    // out = O / l * sigmoid(gate), gate rows read whole as well; eight rows per step (their gate
    // loads wait for the previous step's stores, which share the counter)
#pragma unroll 8
    for (int i = 0; i < nrow; ++i) {
        const int tt = tq, hd = kh * G + gq;
        if (++gq == G) { gq = 0; ++tq; }
        const f4 gt = ld_f4(q + (size_t)tt * qts + (size_t)hd * 2 * HD + HD + 4 * l);
        const f4 ov = *(const f4*)(os + i * HD + 4 * (l ^ i));
        // the gate through the hardware exp2 and reciprocal (the accurate forms cost more than a
        // short chunk's tiles); the output changes by ~1e-7 relative
        const float inv = __builtin_amdgcn_rcpf(ml[w][1][i]);
        f4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = ov[j] * inv * sigmoid_hw(gt[j]);
        *(f4*)(out + (size_t)tt * ots + (size_t)hd * HD + 4 * l) = v;
    }
}

hipError_t launch_attn_flash(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                             int nh, int nkv, int nt, float scale, float* out, int ots, hipStream_t st,
                             const uint16_t* q16, int q16ts) {
    const int R = nt * (nh / nkv);
    const dim3 grid((R + BM - 1) / BM, nkv);
    const _Float16* qh = (const _Float16*)q16;
    // a workgroup per CU or more: the 32-row form (at 8192 tokens 4-6 % faster; below ~128
    // workgroups the 16-row form, e.g. 64 tokens 14.1 -> 10.6 us)
    if (grid.x * grid.y >= 256) {
        if (q16)
            attn_flash_kernel<2><<<grid, 256, 0, st>>>(q, qts, qh, q16ts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots);
        else
            attn_flash_kernel<0><<<grid, 256, 0, st>>>(q, qts, qh, q16ts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots);
    } else if (q16) {
        attn_flash_w8_kernel<false, 2><<<grid, 512, 0, st>>>(q, qts, qh, q16ts, kc, vc, kvd, pos0, nh, nkv, nt, scale,
                                                             out, ots, nullptr, 0, 1);
    } else {
        attn_flash_w8_kernel<false, 0><<<grid, 512, 0, st>>>(q, qts, qh, q16ts, kc, vc, kvd, pos0, nh, nkv, nt, scale,
                                                             out, ots, nullptr, 0, 1);
    }
    return hipGetLastError();
}

int flash_split_chunk(int pos0, int nt, int nh, int nkv) {
    const int R = nt * (nh / nkv);
    const int wgs = (R + BM - 1) / BM * nkv;
    const int keys = pos0 + nt;
    if (wgs >= 128 || keys <= 4 * BN) return 0;
    const int want = (256 + wgs - 1) / wgs;                       // splits to reach ~256 workgroups
    int chunk = ((keys + want - 1) / want + BN - 1) / BN * BN;    // multiple of the 64-key tile
    chunk = chunk < 2 * BN ? 2 * BN : chunk;
    return chunk >= keys ? 0 : chunk;
}

hipError_t launch_attn_flash_split(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                                   int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                                   hipStream_t st, bool f32rec, const uint16_t* q16, int q16ts) {
    const int R = nt * (nh / nkv);
    const int smax = idx::split_count((long)pos0 + nt, chunk);
    const dim3 grid((R + BM - 1) / BM, nkv, smax);
    const _Float16* qh = (const _Float16*)q16;
#define IT_FLASH_SPLIT(F32_, Q16_)                                                                                     \
    attn_flash_w8_kernel<F32_, Q16_><<<grid, 512, 0, st>>>(q, qts, qh, q16ts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, \
                                                        ots, part, chunk, smax)
    if (f32rec) {
        if (q16) IT_FLASH_SPLIT(true, 1);
        else IT_FLASH_SPLIT(true, 0);
    } else {
        if (q16) IT_FLASH_SPLIT(false, 1);
        else IT_FLASH_SPLIT(false, 0);
    }
#undef IT_FLASH_SPLIT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return f32rec ? launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, st)
                  : launch_attn_combine_q16(q, qts, part, pos0, nh, nt, chunk, out, ots, st);
}

}  // namespace it
