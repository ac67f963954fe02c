"""GPU parity of the MTP head's f32-KV attention (it_attn_f32kv, src/mtp.rs:122-130 and
src/vk/mod.rs:942) and of its pre-pass with the slot = position - 1 cache rows."""
import numpy as np
import pytest
import torch

import oracle
from oracle.ref_np import attn_f64
from irontimber_amd import ops
from irontimber_amd.synth import ROPE_BASE, ROPE_N_ROT, ROPE_SECTIONS, prep_inputs, rope_theta_scale
from tests.gpu_util import announce, assert_argmax_agrees, dev_f32, host
from tests.r012 import CASES, GEOMS, arena

pytestmark = pytest.mark.gpu
TOL = 2e-3


def f32kv_inputs(seed, rows, nt, nh=16, nkv=2, hd=256):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((rows, nkv, hd)).astype(np.float32)
    k /= np.sqrt((k.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    v = rng.standard_normal((rows, nkv * hd)).astype(np.float32)
    q = rng.standard_normal((nt, nh * 2 * hd)).astype(np.float32)
    return q, k.reshape(rows, -1), v


@pytest.mark.parametrize("rows,nt,nh,nkv", [(8192, 1, 16, 2), (8192, 2, 16, 2), (4096 + 64, 64, 16, 2), (1, 1, 16, 2),
                                            (65, 1, 16, 2), (100, 3, 16, 2), (777, 33, 16, 2), (300, 5, 8, 8),
                                            (129, 7, 4, 1), (64, 2, 24, 4), (200, 4, 32, 2), (90, 5, 3, 1)])
def test_f32kv_matches_oracle(dev, rows, nt, nh, nkv):
    """Against the restatement of mtp.rs:122-130 (query t sees rows 0..rows-nt+t). The f32 matrix
    cores keep f32 products, so the bound is 2e-5, well inside the north-star 2e-3."""
    announce(f"f32kv rows={rows} nt={nt} nh={nh} nkv={nkv}")
    q, k, v = f32kv_inputs(rows + nt, rows, nt, nh, nkv)
    pos0 = rows - nt
    got = host(ops.attn_f32kv(dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev), pos0, nh, nkv))
    want = oracle.attn_f32kv(q, k, v, pos0, nh, nkv)
    err = np.abs(got - want).max()
    print(f"f32kv max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= 2e-5
    assert_argmax_agrees(got, want)


@pytest.mark.parametrize("nh,nkv,hd", GEOMS)
@pytest.mark.parametrize("pos0,nt", CASES)
def test_f32kv_r012_known_answer(dev, pos0, nt, nh, nkv, hd):
    """src/vk/r012_parity.rs:6-28's closed-form arena with the f32 K/V kept as they are (the MTP
    head's cache), against the float64 softmax at the reference's bound 2e-6."""
    announce(f"f32kv r012 pos0={pos0} nt={nt} nh={nh}")
    q, k, v = arena(pos0, nt, nh, nkv, hd)
    got = host(ops.attn_f32kv(dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev), pos0, nh, nkv, scale=1.0 / 16))
    want = attn_f64(q, k.astype(np.float64), v.astype(np.float64), pos0, nh, nkv, hd, 1.0 / 16)
    err = np.abs(got - want).max()
    print(f"f32kv r012 max_abs={err:.3g}")
    assert err < 2e-6


def test_f32kv_token_by_token_equals_block(dev):
    rows, nt = 500, 4
    q, k, v = f32kv_inputs(7, rows, nt)
    qd, kd, vd = dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev)
    block = host(ops.attn_f32kv(qd, kd, vd, rows - nt, 16, 2))
    for t in range(nt):
        one = host(ops.attn_f32kv(qd[t:t + 1].contiguous(), kd, vd, rows - nt + t, 16, 2))
        np.testing.assert_allclose(one[0], block[t], atol=1e-6)


def test_mtp_head_pass(dev):
    """An MTP head pass of 2 tokens at positions 300, 301 (slots 299, 300) over a 299-slot f32
    cache: the f32 pre-pass stores the new rows at the slots and ropes at the positions, then the
    attention; against mtp.rs:108-130 through the oracle (pre-pass then f32 attention)."""
    nh, nkv, hd, pos = 16, 2, 256, 300
    rng = np.random.default_rng(5)
    old_k = rng.standard_normal((pos - 1, nkv * hd)).astype(np.float32)
    old_v = rng.standard_normal((pos - 1, nkv * hd)).astype(np.float32)
    d = prep_inputs(14, 2, nh, nkv, hd)
    kc = torch.zeros(pos + 1, nkv * hd, device=dev)
    vc = torch.zeros_like(kc)
    kc[:pos - 1] = dev_f32(old_k, dev)
    vc[:pos - 1] = dev_f32(old_v, dev)
    q = dev_f32(d["q"], dev)
    ops.attn_prep_f32kv(q, dev_f32(d["k"], dev), dev_f32(d["v"], dev), kc, vc, pos, pos - 1, nh, nkv,
                        dev_f32(d["q_norm"], dev), dev_f32(d["k_norm"], dev))
    got = host(ops.attn_f32kv(q, kc, vc, pos - 1, nh, nkv))
    oq, ok = oracle.attn_prep(d["q"], d["k"], d["q_norm"], d["k_norm"], 1e-6, pos, nh, nkv, hd, ROPE_N_ROT, ROPE_BASE,
                              ROPE_SECTIONS)
    np.testing.assert_allclose(host(kc)[pos - 1:pos + 1], ok, atol=2e-5)
    np.testing.assert_array_equal(host(vc)[pos - 1:pos + 1], d["v"])
    want = oracle.attn_f32kv(oq, np.concatenate([old_k, ok]), np.concatenate([old_v, d["v"]]), pos - 1, nh, nkv)
    err = np.abs(got - want).max()
    print(f"mtp head pass max_abs={err:.3g}")
    assert err <= TOL
    assert_argmax_agrees(got, want)


def _f32kv_raw(q, kd, vd, pos0, nt, nh, nkv, scratch, nbytes):
    from irontimber_amd._lib import call
    out = torch.empty(nt, nh * 256, device=kd.device)
    call("it_attn_f32kv", q.data_ptr(), nh * 512, kd.data_ptr(), vd.data_ptr(), nkv * 256, pos0, 256, nh, nkv, nt,
         1 / 16, out.data_ptr(), nh * 256, scratch.data_ptr() if scratch is not None else None, nbytes,
         torch.cuda.current_stream().cuda_stream)
    return host(out)


def _f32kv_plan(pos0, nt, nh, nkv, budget):
    import ctypes
    from irontimber_amd._lib import lib
    c, b = ctypes.c_int(), ctypes.c_size_t()
    assert lib().it_attn_f32kv_plan(pos0, nt, 256, nh, nkv, budget, ctypes.byref(c), ctypes.byref(b)) == 0
    return c.value, b.value


@pytest.mark.parametrize("pos0,nt", [(1921, 64), (4096, 64), (8128, 64), (8049, 16), (8191, 1)])
def test_f32kv_reference_room_is_enough(dev, pos0, nt):
    """The MTP head's attention given exactly the reference arena's room at capacity 8192
    (attention_dispatch_room, src/vk/mod.rs:148-150; the f32 branch's C doubling, 730-733), with a
    guard band behind it: the split grows until the records fit, nothing past the room is written,
    and the result matches the restatement of mtp.rs:122-130. nt = 64 from slot 1921 on is the MTP
    prefill catch-up (vk/mod.rs:1002 -> 942), which 64-key splits overflow."""
    from irontimber_amd._lib import lib
    nh, nkv = 16, 2
    room = lib().it_attention_dispatch_room(8192, nh, nt) * 4
    pref = lib().it_attn_f32kv_scratch_bytes(pos0, nt, 256, nh, nkv)
    chunk, nbytes = _f32kv_plan(pos0, nt, nh, nkv, room)
    announce(f"f32kv room pos0={pos0} nt={nt} room={room} preferred={pref} chunk={chunk}")
    assert chunk > 0 and nbytes <= room
    q, k, v = f32kv_inputs(pos0 + 3 * nt, pos0 + nt, nt, nh, nkv)
    guard = 1 << 16
    buf = torch.full((room + guard,), 0x5A, dtype=torch.uint8, device=dev)
    qd, kd, vd = dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev)
    got = _f32kv_raw(qd, kd, vd, pos0, nt, nh, nkv, buf, room)
    assert bool((buf[room:] == 0x5A).all()), "scratch written past the room"
    want = oracle.attn_f32kv(q, k, v, pos0, nh, nkv)
    err = np.abs(got - want).max()
    print(f"f32kv room max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= 2e-5
    assert assert_argmax_agrees(got, want) == 0


@pytest.mark.parametrize("rows,nt,nh,nkv", [(8192, 1, 16, 2), (4096 + 64, 64, 16, 2), (100, 3, 16, 2),
                                            (129, 7, 4, 1), (90, 5, 3, 1), (777, 33, 24, 4)])
def test_f32kv_one_pass_without_scratch(dev, rows, nt, nh, nkv):
    """No scratch at all (and a scratch one byte short of a record per row): the one-pass form,
    which writes the gated output directly like the reference's whole-context `attn` kernel
    (kernels/src/lib.rs:83-116, the fallback of src/vk/mod.rs:740), against the oracle."""
    announce(f"f32kv one pass rows={rows} nt={nt} nh={nh} nkv={nkv}")
    q, k, v = f32kv_inputs(rows + 2 * nt, rows, nt, nh, nkv)
    pos0 = rows - nt
    qd, kd, vd = dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev)
    want = oracle.attn_f32kv(q, k, v, pos0, nh, nkv)
    short = nt * nh * 1040 - 1
    assert _f32kv_plan(pos0, nt, nh, nkv, short) == (0, 0)
    buf = torch.full((short + 4096,), 0x5A, dtype=torch.uint8, device=dev)
    for scratch, nbytes in ((None, 0), (buf, short)):
        got = _f32kv_raw(qd, kd, vd, pos0, nt, nh, nkv, scratch, nbytes)
        err = np.abs(got - want).max()
        print(f"f32kv one pass max_abs={err:.3g}")
        assert np.isfinite(got).all() and err <= 2e-5
        assert assert_argmax_agrees(got, want) == 0
    assert bool((buf == 0x5A).all()), "the one-pass form wrote to the scratch"


def test_f32kv_forced_long_splits_equal_short(dev):
    """Splits of several 64-key tiles (a small scratch) against the preferred 64-key splits: the same
    softmax, so within f32 reassociation of the merge."""
    rows, nt, nh, nkv = 3000, 4, 16, 2
    q, k, v = f32kv_inputs(11, rows, nt, nh, nkv)
    pos0 = rows - nt
    qd, kd, vd = dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev)
    base = host(ops.attn_f32kv(qd, kd, vd, pos0, nh, nkv))
    for splits in (2, 3, 7):
        budget = nt * nh * splits * 1040
        chunk, nbytes = _f32kv_plan(pos0, nt, nh, nkv, budget)
        assert chunk % 64 == 0 and chunk > 64 and nbytes <= budget
        buf = torch.empty(budget, dtype=torch.uint8, device=dev)
        got = _f32kv_raw(qd, kd, vd, pos0, nt, nh, nkv, buf, budget)
        np.testing.assert_allclose(got, base, atol=2e-6)
