"""Index arithmetic of the split records and the merges, checked on the compiled code: the kernels
address every record, mailbox piece and merge load through irontimber_amd/csrc/rec_index.h, and
tests/csrc/index_sweep.cpp compiles that same header for the host and walks it over many geometries
(records inside the scratch the planner sizes, the piece layout one-to-one, every visible split
merged exactly once, mailbox pieces disjoint and inside the buffer)."""
import os
import re
import subprocess

ROOT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..")
CSRC = os.path.join(ROOT, "irontimber_amd", "csrc")


def test_index_sweep(tmp_path):
    exe = tmp_path / "index_sweep"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-o", str(exe),
                    os.path.join(ROOT, "tests", "csrc", "index_sweep.cpp")], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.startswith("ok"), res.stdout + res.stderr
    assert int(res.stdout.split()[1]) > 1_000_000


def test_kernels_use_the_shared_index_functions():
    """No record, piece or merge-slot address is written out by hand in the kernels: the formulas
    the sweep checks are the ones they run."""
    for name in ("decode.hip", "attn_f32kv.hip", "flash.hip"):
        src = open(os.path.join(CSRC, name)).read()
        assert "idx::rec(" in src or name == "attn_f32kv.hip" and "idx::rec(" in src
        assert not re.search(r"\* smax \+ s(plit)?\) \* (260|PART|FLASH_REC)", src), name
        assert not re.search(r"min\(l \+ 64 \* j, ns - 1\)", src), name
    dec = open(os.path.join(CSRC, "decode.hip")).read()
    for fn in ("idx::wave_split(", "idx::row_split(", "idx::comb_split(", "idx::comb_count(", "idx::mb_piece(",
               "idx::splits_seen("):
        assert fn in dec, fn
    assert "idx::piece_o(" in open(os.path.join(CSRC, "common.h")).read()
