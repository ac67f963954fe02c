"""GPU parity of the fused attention pre-pass (it_attn_prep_f16: q/k RMSNorm, (I)MRoPE, f16 KV
append) against the cpu.rs restatement and the float64 statement with exact angles."""
import numpy as np
import pytest
import torch

import oracle
from oracle.ref_np import attn_f64, f16_to_f64, rmsnorm_f64, rope_f64
from irontimber_amd import ops
from irontimber_amd.synth import (ROPE_BASE, ROPE_N_ROT, ROPE_SECTIONS, f16_bits, f16_bits_rtz, prep_inputs,
                                  rope_theta_scale)
from tests.test_oracle_prep import angle_bound
from tests.gpu_util import announce, assert_argmax_agrees, dev_f32, host

pytestmark = pytest.mark.gpu
TOL = 2e-3   # BASELINE north_star bound for attention-path values


def run_prep(dev, d, pos0, nh, nkv, hd, n_rot=ROPE_N_ROT, sections=ROPE_SECTIONS, round_mode=0, weights=True,
             ctx=None):
    nt = d["q"].shape[0]
    ctx = ctx or pos0 + nt + 3
    q = dev_f32(d["q"], dev)
    kc = torch.full((ctx, nkv * hd), -1, dtype=torch.int16, device=dev)
    vc = torch.full_like(kc, -1)
    qn = dev_f32(d["q_norm"], dev) if weights else None
    kn = dev_f32(d["k_norm"], dev) if weights else None
    ops.attn_prep_f16(q, dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, vc, pos0, nh, nkv, qn, kn, 1e-6, n_rot,
                      rope_theta_scale(ROPE_BASE, n_rot), sections=sections, round_mode=round_mode)
    return host(q), host(kc).view(np.uint16), host(vc).view(np.uint16)


def exact(d, pos0, nh, nkv, hd, n_rot, sections, weights=True):
    """float64 q and k after norm and exact-angle rope."""
    nt = d["q"].shape[0]
    tsc = rope_theta_scale(ROPE_BASE, n_rot)
    qw, kw = (d["q_norm"], d["k_norm"]) if weights else (None, None)
    q3 = d["q"].reshape(nt, nh, 2 * hd)
    wq = np.stack([rope_f64(rmsnorm_f64(q3[t, :, :hd], qw), pos0 + t, n_rot, tsc, sections) for t in range(nt)])
    wk = np.stack([rope_f64(rmsnorm_f64(d["k"][t].reshape(nkv, hd), kw), pos0 + t, n_rot, tsc, sections)
                   for t in range(nt)])
    return wq, wk.reshape(nt, nkv * hd)


def check_f16_near(bits, want64, rtz=False, slack=1e-5):
    """Each f16 is the rounding of some value within `slack` (absolute) of the exact f64 value, i.e.
    lies between the roundings of want - slack and want + slack: the kernel's f32 value before the
    cast is that close to exact (the q outputs, written as f32, are checked to 2e-5)."""
    rnd = f16_bits_rtz if rtz else f16_bits
    lo = f16_to_f64(rnd((want64 - slack).astype(np.float32)))
    hi = f16_to_f64(rnd((want64 + slack).astype(np.float32)))
    got = f16_to_f64(bits)
    bad = (got < lo) | (got > hi)
    assert not bad.any(), f"{bad.sum()} f16 values outside the rounding interval"
    exact_bits = rnd(want64.astype(np.float32))
    print(f"{(bits != exact_bits).sum()} of {bits.size} f16 values differ from the exact value's rounding")


@pytest.mark.parametrize("pos0,nt,nh,nkv,hd,n_rot,sections", [
    (8191, 1, 16, 2, 256, 64, ROPE_SECTIONS),      # decode at ctx 8192
    (8188, 4, 16, 2, 256, 64, ROPE_SECTIONS),      # MTP verify
    (4096, 64, 16, 2, 256, 64, ROPE_SECTIONS),     # a prefill chunk
    (0, 37, 16, 2, 256, 64, ROPE_SECTIONS),        # ragged prompt from position 0
    (7, 3, 4, 1, 256, 64, ROPE_SECTIONS),          # the reference's rope fixture geometry (kparity.rs:33)
    (100, 5, 24, 4, 256, 256, (0, 0, 0, 0)),       # every dim rotated, plain neox rope
    (33, 6, 8, 2, 128, 64, (1, 0, 0, 1)),          # hd 128; half the frequencies outside the sections
    (70000, 2, 16, 2, 256, 64, ROPE_SECTIONS),     # far position
])
def test_prep_parity(dev, pos0, nt, nh, nkv, hd, n_rot, sections):
    announce(f"prep pos0={pos0} nt={nt} nh={nh} nkv={nkv} hd={hd} n_rot={n_rot} sections={sections}")
    d = prep_inputs(11, nt, nh, nkv, hd)
    qg, kb, vb = run_prep(dev, d, pos0, nh, nkv, hd, n_rot, sections)
    wq, wk = exact(d, pos0, nh, nkv, hd, n_rot, sections)
    q3 = qg.reshape(nt, nh, 2 * hd)
    eq = np.abs(q3[:, :, :hd] - wq).max()
    print(f"q vs exact-angle f64: {eq:.3g}")
    assert eq <= 2e-5
    np.testing.assert_array_equal(q3[:, :, hd:], d["q"].reshape(nt, nh, 2 * hd)[:, :, hd:])   # gates untouched
    rows = slice(pos0, pos0 + nt)
    check_f16_near(kb[rows], wk)
    np.testing.assert_array_equal(vb[rows], f16_bits(d["v"]))
    assert (kb[:pos0] == 0xFFFF).all() and (kb[pos0 + nt:] == 0xFFFF).all() and (vb[pos0 + nt:] == 0xFFFF).all()
    # the cpu.rs restatement within the north-star bound; past the BASELINE context (8192) its f32
    # angle recurrence alone drifts further, by at most the bound pinned in test_oracle_prep
    oq, ok = oracle.attn_prep(d["q"], d["k"], d["q_norm"], d["k_norm"], 1e-6, pos0, nh, nkv, hd, n_rot, ROPE_BASE,
                              sections)
    tol = TOL if pos0 + nt <= 8192 else TOL + 8 * angle_bound(pos0 + nt, n_rot, rope_theta_scale(ROPE_BASE, n_rot))
    assert np.abs(qg - oq).max() <= tol
    assert np.abs(f16_to_f64(kb[rows]) - f16_to_f64(f16_bits(ok))).max() <= tol


def test_prep_rtz_and_unit_weights(dev):
    nt, nh, nkv, hd = 5, 16, 2, 256
    d = prep_inputs(12, nt, nh, nkv, hd)
    qg, kb, vb = run_prep(dev, d, 50, nh, nkv, hd, round_mode=1, weights=False)
    wq, wk = exact(d, 50, nh, nkv, hd, ROPE_N_ROT, ROPE_SECTIONS, weights=False)
    assert np.abs(qg.reshape(nt, nh, 2 * hd)[:, :, :hd] - wq).max() <= 2e-5
    check_f16_near(kb[50:55], wk, rtz=True)
    np.testing.assert_array_equal(vb[50:55], f16_bits_rtz(d["v"]))


def test_prep_then_attention_matches_cpu_layer(dev):
    """cpu.rs:249-272 end to end for one decode token at position 700 over a 701-row cache: the
    pre-pass appends the new row and prepares q, then attention; against the oracle's pre-pass and
    attention over the same earlier cache rows."""
    nh, nkv, hd, pos0 = 16, 2, 256, 700
    rng = np.random.default_rng(3)
    old_k = f16_bits(rng.standard_normal((pos0, nkv * hd)).astype(np.float32))
    old_v = f16_bits(rng.standard_normal((pos0, nkv * hd)).astype(np.float32))
    d = prep_inputs(13, 1, nh, nkv, hd)
    kc = torch.zeros(pos0 + 1, nkv * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:pos0] = torch.from_numpy(old_k.view(np.int16)).to(dev)
    vc[:pos0] = torch.from_numpy(old_v.view(np.int16)).to(dev)
    q = dev_f32(d["q"], dev)
    ops.attn_prep_f16(q, dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, vc, pos0, nh, nkv, dev_f32(d["q_norm"], dev),
                      dev_f32(d["k_norm"], dev))
    got = host(ops.attn_f16(q, kc, vc, pos0, nh, nkv))
    oq, ok = oracle.attn_prep(d["q"], d["k"], d["q_norm"], d["k_norm"], 1e-6, pos0, nh, nkv, hd, ROPE_N_ROT,
                              ROPE_BASE, ROPE_SECTIONS)
    kall = np.concatenate([old_k, f16_bits(ok)]); vall = np.concatenate([old_v, f16_bits(d["v"])])
    want = oracle.attn(oq, kall, vall, pos0, nh, nkv)
    err = np.abs(got - want).max()
    print(f"prep+attn vs cpu layer: {err:.3g}")
    assert err <= TOL
    assert_argmax_agrees(got, want)



LOG2E_F32 = np.float32(1.4426950408889634)


@pytest.mark.parametrize("pos0,nt,hd", [(0, 64, 256), (4096, 64, 256), (100, 3, 256), (7, 5, 128)])
def test_prep_q16_equals_prep_and_operand_rounding(dev, pos0, nt, hd):
    """it_attn_prep_f16_q16 leaves q, K and V exactly as it_attn_prep_f16 does, and its q16 is the f16
    rounding (RNE) of q' * (scale * log2 e), the product taken in f32: the flash kernel's own
    conversion of q, so the two attention paths get the same operand bits."""
    nh, nkv = 16, 2
    announce(f"prep q16 pos0={pos0} nt={nt} hd={hd}")
    d = prep_inputs(50 + nt, nt, nh, nkv, hd)
    scale = 1.0 / hd ** 0.5
    res = []
    for with16 in (False, True):
        q = dev_f32(d["q"], dev)
        kc = torch.zeros(pos0 + nt, nkv * hd, dtype=torch.int16, device=dev)
        vc = torch.zeros_like(kc)
        args = (q, dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, vc, pos0, nh, nkv)
        qn, kn = dev_f32(d["q_norm"], dev), dev_f32(d["k_norm"], dev)
        q16 = ops.attn_prep_f16_q16(*args, scale=scale, q_norm=qn, k_norm=kn) if with16 else \
            ops.attn_prep_f16(*args, qn, kn)
        res.append((host(q), host(kc), host(vc), host(q16) if with16 else None))
    for a, b in zip(res[0][:3], res[1][:3]):
        np.testing.assert_array_equal(a, b)
    qpart = res[1][0].reshape(nt, nh, 2 * hd)[:, :, :hd]
    want = (qpart * (np.float32(scale) * LOG2E_F32)).astype(np.float16)
    np.testing.assert_array_equal(res[1][3].view(np.uint16).reshape(nt, nh, hd), want.view(np.uint16))


@pytest.mark.parametrize("pos0", [0, 300, 4096])
def test_prep_q16_then_attention_equals_prep_then_attention(dev, pos0):
    """A 64-token prefill chunk through it_attn_prep_f16_q16 + it_attn_f16_q16 gives the outputs of
    it_attn_prep_f16 + it_attn_f16 bit for bit (one pass at 0 and 300, key splits at 4096)."""
    nh, nkv, hd, nt = 16, 2, 256, 64
    announce(f"prep q16 + attn q16 pos0={pos0}")
    rng = np.random.default_rng(9 + pos0)
    old_k = f16_bits(rng.standard_normal((pos0, nkv * hd)).astype(np.float32))
    old_v = f16_bits(rng.standard_normal((pos0, nkv * hd)).astype(np.float32))
    d = prep_inputs(23, nt, nh, nkv, hd)
    outs = []
    for with16 in (False, True):
        kc = torch.zeros(pos0 + nt, nkv * hd, dtype=torch.int16, device=dev)
        vc = torch.zeros_like(kc)
        if pos0:
            kc[:pos0] = torch.from_numpy(old_k.view(np.int16)).to(dev)
            vc[:pos0] = torch.from_numpy(old_v.view(np.int16)).to(dev)
        q = dev_f32(d["q"], dev)
        args = (q, dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, vc, pos0, nh, nkv)
        qn, kn = dev_f32(d["q_norm"], dev), dev_f32(d["k_norm"], dev)
        if with16:
            q16 = ops.attn_prep_f16_q16(*args, scale=1.0 / 16, q_norm=qn, k_norm=kn)
            outs.append(host(ops.attn_f16_q16(q, q16, kc, vc, pos0, nh, nkv)))
        else:
            ops.attn_prep_f16(*args, qn, kn)
            outs.append(host(ops.attn_f16(q, kc, vc, pos0, nh, nkv)))
    np.testing.assert_array_equal(outs[0], outs[1])

def test_prep_rejects_bad_geometry(dev):
    from irontimber_amd._lib import ItError
    d = prep_inputs(1, 1, 16, 2, 256)
    kc = torch.zeros(4, 512, dtype=torch.int16, device=dev)
    with pytest.raises(ItError, match="n_rot"):
        ops.attn_prep_f16(dev_f32(d["q"], dev), dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, kc.clone(), 0, 16, 2,
                          n_rot=6)
