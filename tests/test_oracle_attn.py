"""Pins the attention oracle (oracle/cpu_ref.cpp it_ref_attn, restating src/cpu.rs:260-272)."""
import numpy as np
import pytest
import torch

import oracle
from oracle.ref_np import attn_f64, f16_to_f64
from irontimber_amd.synth import attn_inputs, f16_bits, f16_bits_rtz
from tests.r012 import CASES, GEOMS, arena


def test_f16_rne_matches_numpy():
    x = np.concatenate([np.random.default_rng(0).standard_normal(20000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 1e3, 7e4)])
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504, 65519.99, 65520, 6.1035156e-05, 5.96e-08, 2.98e-08, 2.99e-08])])
    ours = np.array([oracle.lib().it_ref_f32_to_f16_rne(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(ours, f16_bits(x))
    back = np.array([oracle.lib().it_ref_f16_to_f32(int(b)) for b in ours[::50]], np.float32)
    np.testing.assert_array_equal(back, ours[::50].view(np.float16).astype(np.float32))


def test_rtz_helper_truncates():
    x = np.float32([1.0009766, -1.0009766, 0.1, -0.1, 3.14159, 65519.0])
    b = f16_bits_rtz(x)
    h = b.view(np.float16).astype(np.float32)
    assert np.all(np.abs(h) <= np.abs(x))
    assert np.all(np.abs(x - h) < np.abs(np.spacing(h.astype(np.float16)).astype(np.float32)) + 1e-12)


@pytest.mark.parametrize("nh,nkv,hd", GEOMS)
@pytest.mark.parametrize("pos0,nt", CASES)
def test_oracle_r012_known_answer(pos0, nt, nh, nkv, hd):
    """r012_parity.rs:20-28: RTZ f16 cache, f64 softmax + f64 sigmoid gate. The reference's f32 GPU
    kernel meets 2e-6; the sequential f32 restatement sums up to 8192 terms in one f32 accumulator,
    so it is held to 2e-5 here (its worst case over the sweep is printed)."""
    q, k, v = arena(pos0, nt, nh, nkv, hd)
    kb, vb = f16_bits_rtz(k), f16_bits_rtz(v)
    got = oracle.attn(q, kb, vb, pos0, nh, nkv, hd, scale=1.0 / 16)
    want = attn_f64(q, f16_to_f64(kb), f16_to_f64(vb), pos0, nh, nkv, hd, 1.0 / 16)
    err = np.abs(got - want).max()
    print(f"r012 oracle nh={nh} pos0={pos0} nt={nt} max_abs={err:.3g}")
    assert np.isfinite(got).all() and err < 2e-5


def test_oracle_single_key_is_gated_value():
    q, kb, vb = attn_inputs(7, ctx=1, nt=1)
    got = oracle.attn(q.reshape(1, -1), kb, vb, 0, 16, 2)
    gate = q[0, :, 256:]
    v = f16_to_f64(vb).reshape(2, 256)
    want = np.stack([v[h // 8] / (1 + np.exp(-gate[h].astype(np.float64))) for h in range(16)]).reshape(1, -1)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=1e-7)


def test_oracle_zero_query_is_mean_of_values():
    q, kb, vb = attn_inputs(8, ctx=100, nt=1)
    q[:, :, :256] = 0.0
    q[:, :, 256:] = 40.0    # sigmoid(40) == 1 in f32
    got = oracle.attn(q.reshape(1, -1), kb, vb, 99, 16, 2).reshape(16, 256)
    mean = f16_to_f64(vb).reshape(100, 2, 256).mean(axis=0)
    for h in range(16):
        np.testing.assert_allclose(got[h], mean[h // 8], atol=2e-6)


def test_oracle_one_hot_query_softmax_by_hand():
    """q = c*e_0 makes the scores c*k_p[0]*scale; compute that softmax by hand."""
    q, kb, vb = attn_inputs(9, ctx=5, nt=1, nh=2, nkv=1)
    q[:] = 0.0
    q[0, :, 0] = 3.0
    q[0, :, 256:] = 40.0
    got = oracle.attn(q.reshape(1, -1), kb, vb, 4, 2, 1)
    k0 = f16_to_f64(kb)[:, 0]
    w = np.exp(3.0 * k0 / 16 - (3.0 * k0 / 16).max())
    w /= w.sum()
    want = w @ f16_to_f64(vb)
    np.testing.assert_allclose(got[0, :256], want, atol=2e-6)
    np.testing.assert_allclose(got[0, 256:], want, atol=2e-6)


@pytest.mark.parametrize("pos0,nt,nh,nkv", [(0, 16, 16, 2), (40, 24, 8, 8), (100, 3, 6, 2)])
def test_oracle_matches_torch_sdpa(pos0, nt, nh, nkv):
    """Library routine check: torch's scaled_dot_product_attention in float64 with the causal
    offset mask (token t sees keys < pos0+t+1), GQA by repeating KV heads."""
    hd = 256
    q, kb, vb = attn_inputs(11, ctx=pos0 + nt, nt=nt, nh=nh, nkv=nkv)
    got = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, nh, nkv)
    qt = torch.from_numpy(q[:, :, :hd].astype(np.float64)).permute(1, 0, 2)          # [nh, nt, hd]
    K = torch.from_numpy(f16_to_f64(kb).reshape(-1, nkv, hd)).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    V = torch.from_numpy(f16_to_f64(vb).reshape(-1, nkv, hd)).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)
    mask = torch.arange(pos0 + nt)[None, :] < (pos0 + torch.arange(nt)[:, None] + 1)
    o = torch.nn.functional.scaled_dot_product_attention(qt, K, V, attn_mask=mask, scale=1 / 16)
    gate = torch.from_numpy(q[:, :, hd:].astype(np.float64)).permute(1, 0, 2)
    want = (o * torch.sigmoid(gate)).permute(1, 0, 2).reshape(nt, -1).numpy()
    np.testing.assert_allclose(got, want, atol=3e-6)


def test_oracle_token_by_token_equals_block():
    """Calling with nt tokens equals nt single-token calls at pos0, pos0+1, ... (causal decode)."""
    pos0, nt = 30, 5
    q, kb, vb = attn_inputs(12, ctx=pos0 + nt, nt=nt)
    block = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, 16, 2)
    for t in range(nt):
        one = oracle.attn(q[t].reshape(1, -1), kb, vb, pos0 + t, 16, 2)
        np.testing.assert_array_equal(one[0], block[t])


@pytest.mark.parametrize("nh,nkv,hd", GEOMS)
@pytest.mark.parametrize("pos0,nt", CASES)
def test_oracle_f32kv_r012_known_answer(pos0, nt, nh, nkv, hd):
    """The MTP head's f32-cache attention (src/mtp.rs:122-130) on the r012 closed-form arena with
    the f32 K/V as they are (no f16 rounding), against the float64 softmax."""
    q, k, v = arena(pos0, nt, nh, nkv, hd)
    got = oracle.attn_f32kv(q, k, v, pos0, nh, nkv, hd, scale=1.0 / 16)
    want = attn_f64(q, k.astype(np.float64), v.astype(np.float64), pos0, nh, nkv, hd, 1.0 / 16)
    assert np.isfinite(got).all() and np.abs(got - want).max() < 2e-5


def test_oracle_f32kv_closed_forms():
    """Single key: output v * sigmoid(gate); zero query: the mean of V; and the f32 path equals the
    f16 path on a cache whose values are exactly f16."""
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 16 * 512)).astype(np.float32)
    k = rng.standard_normal((1, 512)).astype(np.float32)
    v = rng.standard_normal((1, 512)).astype(np.float32)
    got = oracle.attn_f32kv(q, k, v, 0, 16, 2).reshape(16, 256)
    gate = q.reshape(16, 512)[:, 256:].astype(np.float64)
    want = np.stack([v.reshape(2, 256)[h // 8] / (1 + np.exp(-gate[h])) for h in range(16)])
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=1e-7)
    q2 = q.copy().reshape(16, 512)
    q2[:, :256] = 0.0
    q2[:, 256:] = 40.0
    k = rng.standard_normal((50, 512)).astype(np.float32)
    v = rng.standard_normal((50, 512)).astype(np.float32)
    got = oracle.attn_f32kv(q2.reshape(1, -1), k, v, 49, 16, 2).reshape(16, 256)
    for h in range(16):
        np.testing.assert_allclose(got[h], v.reshape(50, 2, 256).mean(0)[h // 8], atol=2e-6)
    q3, kb, vb = attn_inputs(13, ctx=70, nt=3)
    a = oracle.attn(q3.reshape(3, -1), kb, vb, 67, 16, 2)
    b = oracle.attn_f32kv(q3.reshape(3, -1), f16_to_f64(kb).astype(np.float32), f16_to_f64(vb).astype(np.float32), 67,
                          16, 2)
    np.testing.assert_array_equal(a, b)
