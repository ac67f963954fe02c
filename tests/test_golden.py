"""The committed fixtures under tests/golden/ (written by tests/golden/make_golden.py): the
reference's known-answer attention arena (src/vk/r012_parity.rs:6-28) at the BASELINE geometry and
the kernel-parity harness cases (src/vk/kparity.rs:31-36), each with float64 expected outputs.
The CPU tests check that the in-test generators still produce the frozen inputs, that the float64
statements still give the frozen outputs, and that the oracle meets the reference's bars against
them; the GPU tests hold the HIP path to the same frozen outputs."""
import os

import numpy as np
import pytest

import oracle
from irontimber_amd.synth import f16_bits_rtz
from oracle.ref_np import attn_f64, f16_to_f64, gdn_seq_f64
from tests.r012 import CASES, arena

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
R012 = np.load(os.path.join(HERE, "r012_baseline.npz"))
KP = np.load(os.path.join(HERE, "kparity.npz"))
NH, NKV, HD = 16, 2, 256
MB = 1 << 20


def rel_err(got, want):
    """kparity.rs:2-3: max |got - want| / max(1, |want|)."""
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(1.0, np.abs(want))))


def test_fixture_cases_are_the_reference_list():
    assert [tuple(c) for c in R012["cases"]] == CASES


@pytest.mark.parametrize("pos0,nt", CASES)
def test_r012_arena_and_f64_statement_reproduce_fixture(pos0, nt):
    q, k, v = arena(pos0, nt, NH, NKV, HD)
    np.testing.assert_array_equal(R012[f"qsum_{pos0}_{nt}"], [q.astype(np.float64).sum(), k.astype(np.float64).sum()])
    rows = R012[f"rows_{pos0}_{nt}"]
    want = attn_f64(q, f16_to_f64(f16_bits_rtz(k)), f16_to_f64(f16_bits_rtz(v)), pos0, NH, NKV, HD, 1.0 / 16)
    np.testing.assert_array_equal(want[rows].astype(np.float32), R012[f"out_{pos0}_{nt}"])


@pytest.mark.parametrize("pos0,nt", CASES)
def test_oracle_meets_r012_fixture(pos0, nt):
    """The sequential f32 oracle against the frozen f64 outputs (2e-5: one f32 accumulator over up
    to 8192 terms; the reference's GPU kernels are held to 2e-6 in r012_parity.rs:26)."""
    q, k, v = arena(pos0, nt, NH, NKV, HD)
    got = oracle.attn(q, f16_bits_rtz(k), f16_bits_rtz(v), pos0, NH, NKV, HD, scale=1.0 / 16)
    rows = R012[f"rows_{pos0}_{nt}"]
    assert np.abs(got[rows] - R012[f"out_{pos0}_{nt}"]).max() < 2e-5


def test_kparity_draws_reproduce_fixture_inputs():
    a, p = oracle.kparity_draws(5 << 20, 1 << 16)
    p = p.copy()
    p[16:20] = -np.abs(p[16:20]) - 0.1      # before every case, conv weights included (kparity.rs:63)
    np.testing.assert_array_equal(KP["attn_q"], a[:3 * 2048].reshape(3, 2048))
    np.testing.assert_array_equal(KP["attn_k"], a[MB:MB + 8 * 512].reshape(8, 512))
    np.testing.assert_array_equal(KP["conv_w"], p[:4000].reshape(1000, 4))
    np.testing.assert_array_equal(KP["gdn_co"], a[:6 * 1024].reshape(6, 1024))
    np.testing.assert_array_equal(KP["gdn_dt"], p[0:4])
    np.testing.assert_array_equal(KP["gdn_a"], p[16:20])
    np.testing.assert_array_equal(KP["gdn_state"], a[2 * MB:2 * MB + 4 * 128 * 128].reshape(4, 128, 128))


def test_kparity_f64_statements_reproduce_fixture():
    got = attn_f64(KP["attn_q"], KP["attn_k"].astype(np.float64), KP["attn_v"].astype(np.float64), 5, 4, 2, 256,
                   1.0 / 16)
    np.testing.assert_array_equal(got, KP["attn_out"])
    o64, s64 = gdn_seq_f64(KP["gdn_co"], KP["gdn_beta"], KP["gdn_alpha"], KP["gdn_dt"], KP["gdn_a"],
                           KP["gdn_state"], 4, 2)
    np.testing.assert_array_equal(o64, KP["gdn_out"])
    np.testing.assert_array_equal(s64.astype(np.float32), KP["gdn_state_out"])


def test_oracle_meets_kparity_fixture():
    """The oracle's attn over the f32 cache (2e-6 relative, kparity.rs:34's bar), the conv (2e-6;
    the new conv state is the last K-1 input rows, bit-exact) and the token-sequential recurrence
    (1e-4 relative on out and state: unnormalised q/k make each step's error grow by
    ~|1 - beta |k|^2|)."""
    got = oracle.attn_f32kv(KP["attn_q"], KP["attn_k"], KP["attn_v"], 5, 4, 2, scale=1.0 / 16)
    assert rel_err(got, KP["attn_out"]) <= 2e-6
    co, st = oracle.gdn_conv(KP["conv_x"], KP["conv_w"], KP["conv_state"])
    assert rel_err(co, KP["conv_out"]) <= 2e-6
    np.testing.assert_array_equal(st, KP["conv_x"][-3:])
    wo, ws = oracle.gdn_step(KP["gdn_co"], KP["gdn_beta"], KP["gdn_alpha"], KP["gdn_dt"], KP["gdn_a"],
                             KP["gdn_state"], 4, 2)
    assert rel_err(wo, KP["gdn_out"]) <= 1e-4 and rel_err(ws, KP["gdn_state_out"]) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["splitk", "flash"])
@pytest.mark.parametrize("pos0,nt", CASES)
def test_gpu_meets_r012_fixture(dev, pos0, nt, kernel):
    """Both attention kernels on the reference's known-answer inputs against the frozen float64
    outputs: the split-K path (f32 arithmetic) at the reference's 2e-6 (r012_parity.rs:26), the
    flash path (f16 q and P on the matrix cores; chosen automatically from 16 tokens, run here at
    every token count, so partial row tiles of 6 to 48 rows are covered too) at the north-star
    2e-3."""
    from irontimber_amd import ops
    from tests.gpu_util import announce, dev_f16bits, dev_f32, host
    announce(f"golden r012 pos0={pos0} nt={nt} {kernel}")
    q, k, v = arena(pos0, nt, NH, NKV, HD)
    kid, bar = (ops.KERNEL_SPLITK, 2e-6) if kernel == "splitk" else (ops.KERNEL_FLASH, 2e-3)
    got = host(ops.attn_f16(dev_f32(q, dev), dev_f16bits(f16_bits_rtz(k), dev), dev_f16bits(f16_bits_rtz(v), dev),
                            pos0, NH, NKV, scale=1.0 / 16, kernel=kid))
    rows = R012[f"rows_{pos0}_{nt}"]
    err = np.abs(got[rows] - R012[f"out_{pos0}_{nt}"]).max()
    print(f"golden r012 pos0={pos0} nt={nt} {kernel}: {err:.3g}")
    assert np.isfinite(got).all() and err <= bar


@pytest.mark.gpu
def test_gpu_meets_kparity_fixture(dev):
    """attn (f32 cache), conv and gdn of the harness on the HIP path against the frozen outputs,
    at the bars of test_oracle_meets_kparity_fixture."""
    import torch
    from irontimber_amd import ops
    from tests.gpu_util import announce, dev_f32, host
    announce("golden kparity")
    got = host(ops.attn_f32kv(dev_f32(KP["attn_q"], dev), dev_f32(KP["attn_k"], dev), dev_f32(KP["attn_v"], dev), 5,
                              4, 2, scale=1.0 / 16))
    assert rel_err(got, KP["attn_out"]) <= 2e-6
    st = dev_f32(KP["conv_state"], dev)
    co = host(ops.gdn_conv(dev_f32(KP["conv_x"], dev), dev_f32(KP["conv_w"], dev), st))
    assert rel_err(co, KP["conv_out"]) <= 2e-6
    np.testing.assert_array_equal(host(st), KP["conv_x"][-3:])
    s = dev_f32(KP["gdn_state"], dev)
    o = host(ops.gdn_step(*(dev_f32(KP[n], dev) for n in ("gdn_co", "gdn_beta", "gdn_alpha", "gdn_dt", "gdn_a")),
                          s, 4, 2))
    torch.cuda.synchronize()
    print(f"golden kparity gdn out {rel_err(o, KP['gdn_out']):.3g} state {rel_err(host(s), KP['gdn_state_out']):.3g}")
    assert rel_err(o, KP["gdn_out"]) <= 1e-4 and rel_err(host(s), KP["gdn_state_out"]) <= 1e-4
