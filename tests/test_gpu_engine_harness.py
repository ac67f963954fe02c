"""The C++ engine-shaped caller (tests/csrc/engine_harness.cpp) drives the C ABI as the reference's
engine would (one arena, prompt split by it_prefill_chunks, scratch = the arena's dispatch room,
each chunk's GDN layer through it_gdn_prefill, then token-by-token decode with it_attn_f16 and the
one-launch GDN layer, and the MTP head's f32-KV attention as 64-token catch-up calls with the same
room) over one attention and one GDN layer; its outputs match the oracle: attention within 2e-3
with identical argmax, the MTP head's attention within 2e-5, GDN outputs within 2e-3, the final
state within 5e-3 and the conv state bit-exact."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from irontimber_amd.synth import f16_bits, gdn_inputs
from tests.gpu_util import announce, assert_argmax_agrees

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "csrc", "engine_harness")


@pytest.mark.parametrize("tp,td,ub", [(200, 3, 64), (150, 2, 128), (600, 2, 512), (2100, 2, 512)])
def test_engine_harness_matches_oracle(tmp_path, tp, td, ub):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (__graft_entry__.build() runs make -C tests/csrc)")
    T = tp + td
    rng = np.random.default_rng(7 + tp)
    q = rng.standard_normal((T, 16 * 512)).astype(np.float32)
    k = rng.standard_normal((T, 2, 256))
    k = (k / np.sqrt((k * k).mean(-1, keepdims=True) + 1e-6)).reshape(T, 512).astype(np.float32)
    v = rng.standard_normal((T, 512)).astype(np.float32)
    d = gdn_inputs(13, nt=T)
    files = {"q": q, "k": k, "v": v, "x": d["x"], "w": d["w"], "cst": d["conv_state"], "st": d["state"],
             "br": d["beta_raw"], "ar": d["alpha_raw"], "dt": d["dt"], "a": d["a"]}
    for name, arr in files.items():
        np.ascontiguousarray(arr, np.float32).tofile(tmp_path / f"{name}.bin")
    announce(f"engine harness tp={tp} td={td} ubatch={ub}")
    r = subprocess.run([EXE, str(tmp_path), str(tp), str(td), str(ub)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and r.stdout.startswith("ok "), r.stderr
    attn = np.fromfile(tmp_path / "attn_out.bin", np.float32).reshape(T, 16 * 256)
    gout = np.fromfile(tmp_path / "gdn_out.bin", np.float32).reshape(T, 32 * 128)
    st = np.fromfile(tmp_path / "state_out.bin", np.float32).reshape(32, 128, 128)
    cst = np.fromfile(tmp_path / "cst_out.bin", np.float32).reshape(d["conv_state"].shape)
    # oracle: the whole sequence as one causal pass over the RNE f16 cache (token t sees t + 1 keys)
    want = oracle.attn(q, f16_bits(k), f16_bits(v), 0, 16, 2)
    err = np.abs(attn - want).max()
    cs, ss = d["conv_state"].copy(), d["state"].copy()
    gref = np.zeros((T, 32 * 128), np.float32)
    co = np.zeros((T, d["cd"]), np.float32)
    P = lambda a_: a_.ctypes.data
    oracle.lib().it_ref_gdn_layer(P(d["x"]), d["cd"], P(d["w"]), P(cs), 4, P(d["beta_raw"]), P(d["alpha_raw"]), 32,
                                  P(d["dt"]), P(d["a"]), P(ss), P(gref), 32 * 128, P(co), T, 32, 16, 128, 1e-6,
                                  oracle.hardware_threads())
    ge, se = np.abs(gout - gref).max(), np.abs(st - ss).max()
    print(f"harness: attention {err:.3g}, gdn out {ge:.3g}, state {se:.3g}")
    assert err <= 2e-3 and ge <= 2e-3 and se <= 5e-3
    np.testing.assert_array_equal(cst, cs)
    assert assert_argmax_agrees(attn, want) == 0
    # the MTP head's f32-KV attention over the same rows (f32 cache: no f16 rounding)
    mtp = np.fromfile(tmp_path / "mtp_out.bin", np.float32).reshape(T, 16 * 256)
    mwant = oracle.attn_f32kv(q, k, v, 0, 16, 2)
    me = np.abs(mtp - mwant).max()
    print(f"harness: mtp head attention {me:.3g}")
    assert me <= 2e-5 and assert_argmax_agrees(mtp, mwant) == 0
