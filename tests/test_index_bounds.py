"""Index arithmetic of the merge kernels, walked on the CPU over many geometries: every record a
merge loads lies inside its row's records (index < ns <= smax, so a scratch buffer sized exactly by
it_attn_scratch_bytes is never overrun), and every valid split is merged exactly once. The same for
the mailbox pieces of the one-launch decode against the byte size its buffer descriptor covers.
Formulas follow irontimber_amd/csrc/decode.hip (attn_combine_kernel, combine_wave_row, mb_piece)."""
import itertools
import os
import re

import pytest

_SRC = open(os.path.join(os.path.dirname(__file__), "..", "irontimber_amd", "csrc", "decode.hip")).read()


def _const(name):
    return int(re.search(rf"constexpr int {name} = (\d+);", _SRC).group(1))


COMB_SPL = _const("COMB_SPL")   # splits per lane per batch of attn_combine_kernel
MB_HEAD, MB_PIECE, TK = _const("MB_HEAD"), _const("MB_PIECE"), _const("TK")


def combine_kernel_loads(ns, SL):
    """(split index loaded, merged?) for every lane slot of attn_combine_kernel<SL>."""
    out = []
    for sg in range(SL):
        for s0 in range(0, ns, SL * COMB_SPL):
            nb = min(COMB_SPL, (ns - s0 - sg + SL - 1) // SL)
            for j in range(COMB_SPL):
                idx = min(s0 + sg + SL * max(0, min(j, nb - 1)), ns - 1)
                out.append((idx, j < nb))
    return out


def wave_loads(ns, SPL):
    out = []
    for lane in range(64):
        for j in range(SPL):
            idx = min(lane + 64 * j, ns - 1)
            out.append((idx, lane + 64 * j < ns))
    return out


@pytest.mark.parametrize("SL", [4, 16])
def test_combine_kernel_indices(SL):
    for ns in list(range(1, 300)) + [511, 512, 513, 1024, 4097]:
        loads = combine_kernel_loads(ns, SL)
        assert all(0 <= i < ns for i, _ in loads), (SL, ns)
        merged = sorted(i for i, m in loads if m)
        assert merged == list(range(ns)), (SL, ns)


@pytest.mark.parametrize("SPL", [1, 2, 4])
def test_wave_merge_indices(SPL):
    for ns in range(1, 64 * SPL + 1):
        loads = wave_loads(ns, SPL)
        assert all(0 <= i < ns for i, _ in loads)
        assert sorted(i for i, m in loads if m) == list(range(ns))


def test_mailbox_piece_indices_inside_descriptor():
    """mb_piece(th, db, s, smax) for every row, 16-dim block and visible split stays below the
    float count it_attn_mailbox_bytes gives for the call (the buffer descriptor's range), and the
    pieces of different (row, block, split) never overlap."""
    for ctx, nt, nh in itertools.product([1, 63, 64, 65, 1000, 8192, 16384], [1, 2, 4, 8], [4, 16, 32]):
        pos0 = ctx - nt
        if pos0 < 0:
            continue
        smax = (ctx + TK - 1) // TK
        words = MB_HEAD + nt * nh * 16 * smax * MB_PIECE
        seen = set()
        for th in range(nt * nh):
            t = th // nh
            ns = (pos0 + t + TK) // TK
            assert ns <= smax
            for db in range(16):
                for s in range(ns):
                    base = MB_HEAD + ((th * 16 + db) * smax + s) * MB_PIECE
                    assert base + MB_PIECE <= words
                    assert base not in seen
                    seen.add(base)
