"""Pins the attention pre-pass oracle: it_ref_rope (src/cpu.rs:145-162), it_ref_rmsnorm
(cpu.rs:14-18) and their composition it_ref_attn_prep (cpu.rs:249-257)."""
import numpy as np
import pytest

import oracle
from oracle.ref_np import rmsnorm_f64, rope_f64
from irontimber_amd.synth import ROPE_BASE, ROPE_N_ROT, ROPE_SECTIONS, prep_inputs, rope_theta_scale

U = 2.0 ** -24


def _x(n=4, hd=256, seed=0):
    return np.random.default_rng(seed).standard_normal((n, hd)).astype(np.float32) * 2


def angle_bound(pos, n_rot, tsc):
    """|f32 angle recurrence - exact angle| <= max_i i*u*pos*tsc^i (one rounding per product),
    with headroom, plus a few ulps of sin/cos."""
    i = np.arange(n_rot // 2)
    return 1.5 * U * pos * float((i * float(tsc) ** i).max()) + 4e-7


def test_theta_scale_matches_host_helper():
    for base, n in ((1e7, 64), (1e4, 128), (5e5, 32)):
        assert oracle.rope_theta_scale(base, n) == rope_theta_scale(base, n)


def test_rope_pos0_is_identity():
    x = _x()
    np.testing.assert_array_equal(oracle.rope(x, 0, 64, ROPE_BASE, ROPE_SECTIONS), x)


@pytest.mark.parametrize("pos", [1, 3, 100, 8191])
def test_rope_single_pair_is_2d_rotation(pos):
    """n_rot = 2: one frequency, angle theta_0 = pos exactly; dims past n_rot untouched."""
    x = _x(2, 8)
    y = oracle.rope(x, pos, 2, ROPE_BASE)
    c, s = np.cos(pos), np.sin(pos)
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(y[:, 0], x64[:, 0] * c - x64[:, 1] * s, atol=2e-6)
    np.testing.assert_allclose(y[:, 1], x64[:, 0] * s + x64[:, 1] * c, atol=2e-6)
    np.testing.assert_array_equal(y[:, 2:], x[:, 2:])


def test_rope_sector_rule_fixed_dims():
    """sections (1, 0, 0, 1): sect = 2, odd frequencies fall outside the text sections and keep
    angle 0 (cpu.rs:152-155), even ones rotate."""
    x = _x(3, 16)
    y = oracle.rope(x, 37, 8, ROPE_BASE, (1, 0, 0, 1))
    half = 4
    for i in range(half):
        if i % 2 == 1:
            np.testing.assert_array_equal(y[:, [i, i + half]], x[:, [i, i + half]])
        else:
            assert np.abs(y[:, [i, i + half]] - x[:, [i, i + half]]).max() > 1e-3
    np.testing.assert_allclose(y, rope_f64(x, 37, 8, rope_theta_scale(ROPE_BASE, 8), (1, 0, 0, 1)), atol=2e-6)


@pytest.mark.parametrize("pos", [7, 511, 4095, 8191])
@pytest.mark.parametrize("n_rot,sections", [(64, ROPE_SECTIONS), (64, (0, 0, 0, 0)), (256, (0, 0, 0, 0)),
                                            (128, (5, 3, 2, 6))])
def test_rope_matches_exact_angles(pos, n_rot, sections):
    """Against the float64 statement with exact angles pos*tsc^i: the only difference is the f32
    angle recurrence, bounded per frequency; a wrong sign, pair or frequency index fails by O(1)."""
    x = _x()
    tsc = rope_theta_scale(ROPE_BASE, n_rot)
    y = oracle.rope(x, pos, n_rot, ROPE_BASE, sections)
    want = rope_f64(x, pos, n_rot, tsc, sections)
    pair = np.sqrt(x[:, :n_rot // 2].astype(np.float64) ** 2 + x[:, n_rot // 2:n_rot].astype(np.float64) ** 2).max()
    err = np.abs(y - want).max()
    print(f"rope pos={pos} n_rot={n_rot} err={err:.3g} bound={angle_bound(pos, n_rot, tsc) * pair:.3g}")
    assert err <= angle_bound(pos, n_rot, tsc) * pair + 1e-6


def test_rope_preserves_pair_norms_and_relative_position():
    x, z = _x(1, 256, 1)[0], _x(1, 256, 2)[0]
    y = oracle.rope(x, 1234, 64, ROPE_BASE, ROPE_SECTIONS)
    h = 32
    n0 = x[:h].astype(np.float64) ** 2 + x[h:2 * h].astype(np.float64) ** 2
    n1 = y[:h].astype(np.float64) ** 2 + y[h:2 * h].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    # q.k after rope depends on the position difference only (every dim rotates for these sections)
    d = lambda m, n: float(np.dot(oracle.rope(x, m, 64, ROPE_BASE, ROPE_SECTIONS).astype(np.float64),
                                  oracle.rope(z, n, 64, ROPE_BASE, ROPE_SECTIONS).astype(np.float64)))
    assert abs(d(5, 2) - d(25, 22)) < 1e-4 and abs(d(5, 2) - d(3, 0)) < 1e-4
    assert abs(d(5, 2) - d(2, 5)) > 1e-3


def test_rmsnorm_closed_forms():
    x = _x(1, 256)[0]
    y = np.zeros_like(x)
    oracle.lib().it_ref_rmsnorm(x.ctypes.data, None, 256, 1e-6, y.ctypes.data)
    ms = float((x.astype(np.float64) ** 2).mean())
    assert abs(float((y.astype(np.float64) ** 2).mean()) - ms / (ms + 1e-6)) < 1e-5
    c = np.full(256, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 256).astype(np.float32)
    oracle.lib().it_ref_rmsnorm(c.ctypes.data, w.ctypes.data, 256, 1e-6, y.ctypes.data)
    np.testing.assert_allclose(y, 3.0 / np.sqrt(9.0 + 1e-6) * w, rtol=1e-6)


@pytest.mark.parametrize("pos0,nt,nh,nkv,hd", [(0, 3, 4, 2, 256), (8191, 1, 16, 2, 256), (100, 5, 8, 1, 128)])
def test_attn_prep_composition(pos0, nt, nh, nkv, hd):
    """q heads normed+roped in place at pos0+t, gates untouched; k normed+roped; against the f64
    statements (rmsnorm_f64 then rope_f64 with exact angles)."""
    d = prep_inputs(9, nt, nh, nkv, hd)
    qo, ko = oracle.attn_prep(d["q"], d["k"], d["q_norm"], d["k_norm"], 1e-6, pos0, nh, nkv, hd, ROPE_N_ROT, ROPE_BASE,
                              ROPE_SECTIONS)
    tsc = rope_theta_scale(ROPE_BASE, ROPE_N_ROT)
    q3 = d["q"].reshape(nt, nh, 2 * hd)
    np.testing.assert_array_equal(qo.reshape(nt, nh, 2 * hd)[:, :, hd:], q3[:, :, hd:])
    for t in range(nt):
        b = angle_bound(pos0 + t, ROPE_N_ROT, tsc) * 8 + 2e-6
        wq = rope_f64(rmsnorm_f64(q3[t, :, :hd], d["q_norm"]), pos0 + t, ROPE_N_ROT, tsc, ROPE_SECTIONS)
        wk = rope_f64(rmsnorm_f64(d["k"][t].reshape(nkv, hd), d["k_norm"]), pos0 + t, ROPE_N_ROT, tsc, ROPE_SECTIONS)
        assert np.abs(qo.reshape(nt, nh, 2 * hd)[t, :, :hd] - wq).max() <= b
        assert np.abs(ko[t].reshape(nkv, hd) - wk).max() <= b
