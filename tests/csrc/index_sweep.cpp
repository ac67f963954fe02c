// Host build of irontimber_amd/csrc/rec_index.h, the index functions through which the kernels
// address every split record, mailbox piece and merge load, walked over many geometries:
//   - f32 split-K records, flash int16 records and the piece layout lie inside the bytes the planner
//     sizes for them (api.hip: splitk_scratch, flash_scratch), and the piece layout maps every
//     (row, dim, split) and every header to its own word;
//   - the merges (wave merge, row merge, workgroup merge) load only splits 0 .. ns-1 of a row, with
//     ns <= smax, and merge each of them exactly once;
//   - mailbox pieces of every (row, dim block, visible split) are disjoint and inside the buffer.
// The loops restate the kernels' grids and the launch policy (which merge, how many slots); the
// arithmetic is the header's. Prints "ok <checks>" or the first failure and exits nonzero.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "../../irontimber_amd/csrc/rec_index.h"

using namespace it::idx;

static long checks = 0;
#define REQUIRE(cond, ...)                  \
    do {                                    \
        ++checks;                           \
        if (!(cond)) {                      \
            std::printf("FAIL: ");          \
            std::printf(__VA_ARGS__);       \
            std::printf("\n");              \
            return 1;                       \
        }                                   \
    } while (0)

// every split a merge of ns splits loads (and which slots it keeps) covers 0 .. ns-1 once
static int check_merge_cover(const char* what, const std::vector<std::pair<int, bool>>& loads, int ns) {
    std::vector<int> seen(ns, 0);
    for (auto& [s, keep] : loads) {
        REQUIRE(s >= 0 && s < ns, "%s: split %d loaded, ns %d", what, s, ns);
        if (keep) ++seen[s];
    }
    for (int s = 0; s < ns; ++s) REQUIRE(seen[s] == 1, "%s: split %d merged %d times (ns %d)", what, s, seen[s], ns);
    return 0;
}

// api.hip flash_scratch / 4: FLASH_REC words per (row, split)
static size_t flash_words_planned(int rows, int smax) { return (size_t)rows * smax * FLASH_REC; }

static int check_geometry(int pos0, int nt, int nh, int chunk) {
    const int rows = nt * nh;
    const int smax = split_count((long)pos0 + nt, chunk);
    const size_t part_words = (size_t)rows * smax * PART;   // splitk_scratch / 4
    const size_t fw = (size_t)rows * smax * FLASH_REC;
    // row-major records: the last word of the last record is inside the buffer
    REQUIRE(rec(rows - 1, smax - 1, smax) * PART + PART <= part_words, "f32 records pos0 %d nt %d", pos0, nt);
    REQUIRE(rec(rows - 1, smax - 1, smax) * FLASH_REC + FLASH_REC <= fw, "flash records pos0 %d", pos0);
    // flash int16 records: O runs 512-byte aligned and one-to-one, headers after them, all inside
    // flash_words (the planner's size)
    REQUIRE(flash_words(rows, smax) == flash_words_planned(rows, smax), "flash words");
    REQUIRE(flash_o(rows - 1, smax - 1, smax) + 128 <= (size_t)rows * smax * 128, "flash o corner");
    REQUIRE(flash_h(rows, rows - 1, smax - 1, smax) + 4 <= flash_words(rows, smax), "flash h corner");
    REQUIRE(flash_o(0, 1, smax) - flash_o(0, 0, smax) == 128 && flash_o(0, 0, smax) % 32 == 0, "flash o stride");
    if ((size_t)rows * smax <= 40000) {
        std::vector<uint8_t> hit(flash_words(rows, smax), 0);
        for (int th = 0; th < rows; ++th)
            for (int s = 0; s < smax; ++s) {
                for (int e = 0; e < 128; ++e) {
                    const size_t w = flash_o(th, s, smax) + e;
                    REQUIRE(w < (size_t)rows * smax * 128 && !hit[w], "flash o (%d,%d)", th, s);
                    hit[w] = 1;
                }
                for (int e = 0; e < 4; ++e) {
                    const size_t w = flash_h(rows, th, s, smax) + e;
                    REQUIRE(w >= (size_t)rows * smax * 128 && w < hit.size() && !hit[w], "flash h (%d,%d)", th, s);
                    hit[w] = 1;
                }
            }
    }
    // piece layout: inside the f32 records' bytes; one word per (row, dim, split) and per header word
    REQUIRE(piece_words(rows, smax) <= part_words, "piece words pos0 %d nt %d nh %d", pos0, nt, nh);
    if ((size_t)rows * smax <= 40000) {
        std::vector<uint8_t> hit(piece_words(rows, smax), 0);
        for (int th = 0; th < rows; ++th)
            for (int s = 0; s < smax; ++s) {
                for (int db = 0; db < 16; ++db)
                    for (int e = 0; e < 16; ++e) {
                        const size_t w = piece_o(th, db, s, smax) + e;
                        REQUIRE(w < (size_t)rows * smax * 256 && !hit[w], "piece o (%d,%d,%d,%d)", th, db, s, e);
                        hit[w] = 1;
                    }
                for (int e = 0; e < 2; ++e) {
                    const size_t w = piece_h(rows, th, s, smax) + e;
                    REQUIRE(w >= (size_t)rows * smax * 256 && w < hit.size() && !hit[w], "piece h (%d,%d)", th, s);
                    hit[w] = 1;
                }
            }
    } else {   // the far corner of each region
        REQUIRE(piece_o(rows - 1, 15, smax - 1, smax) + 16 <= (size_t)rows * smax * 256, "piece o corner");
        REQUIRE(piece_h(rows, rows - 1, smax - 1, smax) + 2 <= piece_words(rows, smax), "piece h corner");
    }
    // merges, per token (rows of one token share ns)
    for (int t = 0; t < nt; ++t) {
        const int ns = splits_seen(pos0, t, chunk);
        REQUIRE(ns >= 1 && ns <= smax, "ns %d smax %d (pos0 %d t %d chunk %d)", ns, smax, pos0, t, chunk);
        // wave merge (piece_records: 8 < smax <= 256, SPL by smax)
        if (smax > 8 && smax <= 256) {
            const int spl = smax <= 64 ? 1 : smax <= 128 ? 2 : 4;
            std::vector<std::pair<int, bool>> loads;
            for (int l = 0; l < 64; ++l)
                for (int j = 0; j < spl; ++j) loads.push_back({wave_split(l, j, ns), l + 64 * j < ns});
            if (check_merge_cover("wave merge", loads, ns)) return 1;
        }
        // row merge (smax <= NS for NS = 8, 16, 32): slots j < NS, and lane l's header
        for (int NS : {8, 16, 32}) {
            if (smax > NS) continue;
            std::vector<std::pair<int, bool>> loads, hdr;
            for (int j = 0; j < NS; ++j) loads.push_back({row_split(j, ns), j < ns});
            for (int l = 0; l < 64; ++l) hdr.push_back({row_split(l, ns), l < ns});
            if (check_merge_cover("row merge", loads, ns) || check_merge_cover("row merge headers", hdr, ns)) return 1;
        }
        // workgroup merge attn_combine_kernel<SL>
        for (int SL : {4, 16}) {
            std::vector<std::pair<int, bool>> loads;
            for (int sg = 0; sg < SL; ++sg)
                for (int s0 = 0; s0 < ns; s0 += SL * COMB_SPL) {
                    const int nb = comb_count(ns, s0, sg, SL);
                    for (int j = 0; j < COMB_SPL; ++j) loads.push_back({comb_split(s0, sg, SL, j, nb, ns), j < nb});
                }
            if (check_merge_cover("workgroup merge", loads, ns)) return 1;
        }
    }
    return 0;
}

// one-wave merge: workgroup ids 0 .. rows*16-1 map one-to-one onto (row, 16-dim block)
static int check_wave1(int rows) {
    std::vector<uint8_t> hit((size_t)rows * 16, 0);
    for (int id = 0; id < rows * 16; ++id) {
        int th = -1, db = -1;
        wave1_unit(id, rows, th, db);
        REQUIRE(th >= 0 && th < rows && db >= 0 && db < 16 && !hit[(size_t)th * 16 + db], "wave1 id %d rows %d", id, rows);
        hit[(size_t)th * 16 + db] = 1;
    }
    return 0;
}

// mailbox (64-key splits): pieces of every (row, block, visible split) disjoint, inside the buffer
// of it_attn_mailbox_bytes (MB_HEAD + rows * 16 * smax * MB_PIECE floats)
static int check_mailbox(int ctx, int nt, int nh) {
    const int pos0 = ctx - nt, rows = nt * nh, smax = split_count(ctx, 64);
    const size_t words = MB_HEAD + (size_t)rows * 16 * smax * MB_PIECE;
    std::vector<uint8_t> hit(words, 0);
    for (int th = 0; th < rows; ++th) {
        const int ns = splits_seen(pos0, th / nh, 64);
        REQUIRE(ns <= smax, "mailbox ns");
        for (int db = 0; db < 16; ++db)
            for (int s = 0; s < ns; ++s) {
                const int b = mb_piece(th, db, s, smax);
                REQUIRE(b >= MB_HEAD && (size_t)b + MB_PIECE <= words, "mailbox piece (%d,%d,%d) ctx %d", th, db, s, ctx);
                for (int e = 0; e < MB_PIECE; ++e) {
                    REQUIRE(!hit[b + e], "mailbox overlap (%d,%d,%d)", th, db, s);
                    hit[b + e] = 1;
                }
            }
    }
    return 0;
}

int main() {
    const int pos0s[] = {0, 1, 63, 64, 65, 511, 1000, 1023, 1024, 2047, 4095, 4096, 8128, 8188, 8191, 16383, 16384, 20000};
    const int nts[] = {1, 2, 3, 4, 8, 16, 17, 64};
    const int nhs[] = {1, 8, 16, 24, 32};
    const int chunks[] = {64, 128, 192, 256, 640, 1024, 8192};
    for (int pos0 : pos0s)
        for (int nt : nts)
            for (int nh : nhs)
                for (int chunk : chunks)
                    if (check_geometry(pos0, nt, nh, chunk)) return 1;
    for (int ns = 1; ns <= 300; ++ns)   // every split count of the merges at one token
        if (check_geometry(ns * 64 - 1, 1, 16, 64)) return 1;
    for (int rows = 1; rows <= 256; ++rows)
        if (check_wave1(rows)) return 1;
    for (int ctx : {1, 63, 64, 65, 1000, 2048, 8192, 16384})
        for (int nt : {1, 2, 4, 8})
            for (int nh : {4, 16, 32})
                if (ctx >= nt && check_mailbox(ctx, nt, nh)) return 1;
    std::printf("ok %ld\n", checks);
    return 0;
}
