// Index arithmetic of the split-K records, the mailbox pieces and the merges that read them. The
// kernels (decode.hip, attn_f32kv.hip, flash.hip) compute every record address through these
// functions, and tests/csrc/index_sweep.cpp compiles the same header for the host and walks them
// over many geometries: every load and store stays inside the buffer the planner sizes, the piece
// layout is one-to-one, and every visible split is merged exactly once.
#pragma once
#include <stddef.h>

#if defined(__HIP__)
#define IT_IDX __host__ __device__ __forceinline__
#else
#define IT_IDX inline
#endif

namespace it {
namespace idx {

constexpr int PART = 260;          // words of a split-K record {m, l, 0, 0, o[256]}
constexpr int FLASH_REC = 4 + 128; // words of a flash key-split record {m, l, k, 0} + 256 int16
constexpr int COMB_SPL = 8;        // splits a split lane of attn_combine_kernel loads per batch
constexpr int MB_PIECE = 24;       // floats per mailbox piece: o[16], {m, l}, unused
constexpr int MB_HEAD = 64;        // floats before the first mailbox piece

IT_IDX int imin(int a, int b) { return a < b ? a : b; }
IT_IDX int imax(int a, int b) { return a > b ? a : b; }

// Splits of `chunk` keys over `total` keys (the record count per row), and the splits that hold
// keys <= pos0 + t, i.e. the ones token t of a call at pos0 merges (1 .. split_count).
IT_IDX int split_count(long total, int chunk) { return (int)((total + chunk - 1) / chunk); }
IT_IDX int splits_seen(int pos0, int t, int chunk) { return (pos0 + t + chunk) / chunk; }

// Record (row th = token * nh + head, split s) in the row-major record layouts: its first word is
// rec(th, s, smax) * words (PART or FLASH_REC).
IT_IDX size_t rec(int th, int s, int smax) { return (size_t)th * smax + s; }

// Piece layout of the f32 split-K records (for the wave merge): O of (row th, 16-dim block db,
// split s) as 16 floats at piece_o, then {m, l} of (th, s) at piece_h; piece_words floats in all.
IT_IDX size_t piece_o(int th, int db, int s, int smax) { return ((size_t)(th * 16 + db) * smax + s) * 16; }
IT_IDX size_t piece_h(int rows, int th, int s, int smax) {
    return (size_t)rows * smax * 256 + 2 * ((size_t)th * smax + s);
}
IT_IDX size_t piece_words(int rows, int smax) { return (size_t)rows * smax * 258; }

// Flash key-split records (O as int16 in units of k): O of (row th, split s) as 256 int16 at
// flash_o, a 512-byte-aligned run of whole cache lines, then the headers {m, l, k, 0} of all
// (row, split) packed after them at flash_h; flash_words floats in all (FLASH_REC per record).
IT_IDX size_t flash_o(int th, int s, int smax) { return ((size_t)th * smax + s) * 128; }
IT_IDX size_t flash_h(int rows, int th, int s, int smax) {
    return (size_t)rows * smax * 128 + ((size_t)th * smax + s) * 4;
}
IT_IDX size_t flash_words(int rows, int smax) { return (size_t)rows * smax * FLASH_REC; }

// Mailbox piece (row th, dim block db, split s): its first float.
IT_IDX int mb_piece(int th, int db, int s, int smax) { return MB_HEAD + ((th * 16 + db) * smax + s) * MB_PIECE; }

// Wave merge (one wave per row and 16 dims): split lane l loads split wave_split(l, j, ns) in slot
// j; slots with l + 64 j >= ns reload the row's last split and are masked.
IT_IDX int wave_split(int l, int j, int ns) { return imin(l + 64 * j, ns - 1); }

// Wave merge with one wave per workgroup: workgroup id -> (row th, 16-dim block db) of rows x 16
// units. With rows a multiple of 8, the 16 workgroups of a row get ids 8 apart (one XCD under the
// round-robin dispatch), so the row's header run is fetched into one L2.
IT_IDX void wave1_unit(int id, int rows, int& th, int& db) {
    if (rows % 8 == 0) {
        const int xcd = id & 7, slot = id >> 3;
        th = ((slot >> 4) << 3) | xcd;
        db = slot & 15;
    } else {
        th = id >> 4;
        db = id & 15;
    }
}

// Row merge (one wave per row): slot j loads split row_split(j, ns), masked past ns.
IT_IDX int row_split(int j, int ns) { return imin(j, ns - 1); }

// attn_combine_kernel<SL>: in the batch starting at split s0, split lane sg holds comb_count
// splits (<= 0: none) and loads comb_split(...) in slot j; slots past the count reload its last
// split (or split ns - 1) and are masked.
IT_IDX int comb_count(int ns, int s0, int sg, int SL) { return imin(COMB_SPL, (ns - s0 - sg + SL - 1) / SL); }
IT_IDX int comb_split(int s0, int sg, int SL, int j, int nb, int ns) {
    return imin(s0 + sg + SL * imax(0, imin(j, nb - 1)), ns - 1);
}

}  // namespace idx
}  // namespace it
