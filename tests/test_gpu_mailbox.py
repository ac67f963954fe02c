"""Decode attention in one launch through a mailbox (it_attn_f16_mailbox): bit-equal to the
two-launch split-K path (same partials, same merge order) wherever the wave merge is used, within
the attention tolerance of the oracle, the mailbox left clean (every piece word back to the empty
pattern, poison flag clear) after any sequence of calls, fallbacks for geometries that do not
qualify, and replays of a captured graph."""
import numpy as np
import pytest
import torch

import oracle
from irontimber_amd import ops
from irontimber_amd.synth import attn_inputs
from tests.gpu_util import announce, assert_argmax_agrees, dev_f16bits, dev_f32, host

pytestmark = pytest.mark.gpu
TOL = 2e-3
EMPTY = np.uint32(0xFFFFFFFF)


def _inputs(dev, seed, ctx, nt, nh, nkv):
    q, kb, vb = attn_inputs(seed, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    return q, kb, vb, dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)


MAGIC = np.uint32(0x4D424F58)


def _clean(mb):
    words = host(mb).view(np.uint32)
    # words 2-3: the device address of the mailbox's host-visible report word
    return (words[0] == 0 and words[1] == MAGIC and (words[2:4] != 0).any() and (words[4:64] == 0).all()
            and (words[64:] == EMPTY).all())


# (ctx, nt, nh, nkv, one launch expected): decode at the BASELINE geometry (ctx 8192), 256 splits
# (ctx 16384), a one-key last split (ctx 2049), other GQA groups, verify rows whose last split is
# invisible to the first token (pos0 % 64 == 63) with 8 rows per KV head; and geometries that take
# the two-launch path: short contexts with fewer waves than merge units (ctx
# 512, among them), more rows per KV head, or a grid larger than the device holds at once (8 KV
# heads x 128 splits)
SHAPES = [(8192, 1, 16, 2, True), (16384, 1, 16, 2, True), (2049, 1, 16, 2, True), (2000, 1, 32, 4, True),
          (64 * 20 + 63 + 4, 4, 8, 8, True), (4096 + 1, 2, 8, 8, True), (8192 + 3, 3, 4, 2, True),
          (512, 1, 16, 2, False), (1, 1, 16, 2, False), (65, 1, 16, 2, False), (64, 1, 24, 4, False),
          (300, 5, 8, 8, False), (129, 2, 4, 1, False), (8192, 8, 8, 8, False), (8192, 4, 16, 2, False),
          (100, 3, 16, 2, False)]


@pytest.mark.parametrize("ctx,nt,nh,nkv,one", SHAPES)
def test_mailbox_equals_two_launches(dev, ctx, nt, nh, nkv, one):
    announce(f"mailbox ctx={ctx} nt={nt} nh={nh} nkv={nkv}")
    pos0 = ctx - nt
    q, kb, vb, qd, kc, vc = _inputs(dev, 31 + ctx, ctx, nt, nh, nkv)
    mb = ops.attn_mailbox(ctx, nt, nh, dev)
    assert ops.attn_mailbox_would_launch(pos0, nt, nh, nkv, mb) == one
    got = host(ops.attn_f16_mailbox(qd, kc, vc, pos0, nh, nkv, mb))
    ref = host(ops.attn_f16(qd, kc, vc, pos0, nh, nkv))
    want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, nh, nkv)
    err = np.abs(got - want).max()
    print(f"mailbox vs oracle {err:.3g}, vs two launches {np.abs(got - ref).max():.3g}")
    np.testing.assert_array_equal(got, ref)
    assert err <= TOL
    assert not ops.attn_mailbox_poisoned(mb)
    assert _clean(mb)


def test_mailbox_sequence_and_baseline_argmax(dev):
    """One mailbox over a run of calls of different geometries (as an engine's layers and steps
    would use it): every result equals the two-launch path and the mailbox stays clean."""
    nh, nkv = 16, 2
    mb = ops.attn_mailbox(8192, 4, nh, dev)
    for i, (ctx, nt) in enumerate([(8192, 1), (8192, 4), (37, 1), (8192, 1), (5000, 1), (8192, 4), (3000, 1)]):
        announce(f"mailbox sequence step {i} ctx={ctx} nt={nt}")
        q, kb, vb, qd, kc, vc = _inputs(dev, 100 + i, ctx, nt, nh, nkv)
        got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - nt, nh, nkv, mb))
        np.testing.assert_array_equal(got, host(ops.attn_f16(qd, kc, vc, ctx - nt, nh, nkv)))
        if ctx == 8192:
            want = oracle.attn(q.reshape(nt, -1), kb, vb, ctx - nt, nh, nkv)
            assert np.abs(got - want).max() <= TOL and assert_argmax_agrees(got, want) == 0
    assert not ops.attn_mailbox_poisoned(mb)
    assert _clean(mb)


@pytest.mark.parametrize("ctx,nt,small", [(8192, 64, False), (16384 + 64, 1, False), (8192, 1, True)])
def test_mailbox_fallbacks(dev, ctx, nt, small):
    """Geometries the one-launch form does not take (a prefill chunk, more than 256 splits, a
    mailbox too small for the call) run the two-launch path with the caller's scratch."""
    nh, nkv = 16, 2
    pos0 = ctx - nt
    announce(f"mailbox fallback ctx={ctx} nt={nt} small={small}")
    q, kb, vb, qd, kc, vc = _inputs(dev, 7, ctx, nt, nh, nkv)
    mb = ops.attn_mailbox(512 if small else ctx, nt, nh, dev)
    assert not ops.attn_mailbox_would_launch(pos0, nt, nh, nkv, mb)
    got = host(ops.attn_f16_mailbox(qd, kc, vc, pos0, nh, nkv, mb))
    np.testing.assert_array_equal(got, host(ops.attn_f16(qd, kc, vc, pos0, nh, nkv)))
    assert _clean(mb)


def test_mailbox_graph_replays(dev):
    """A captured graph of ten one-launch decode calls replayed several times, with eager work and
    synchronisation between the replays: every replay equals the eager result."""
    nh, nkv, ctx = 16, 2, 8192
    q, kb, vb, qd, kc, vc = _inputs(dev, 5, ctx, 1, nh, nkv)
    mb = ops.attn_mailbox(ctx, 1, nh, dev)
    out = torch.empty(1, nh * 256, device=dev, dtype=torch.float32)
    eager = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(10):
                ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(out), eager)
        ops.attn_f16(qd, kc, vc, ctx - 1, nh, nkv)   # eager work between replays
        torch.cuda.synchronize()
    assert not ops.attn_mailbox_poisoned(mb)
    assert _clean(mb)


def test_poisoned_mailbox_fails_loudly(dev):
    """A mailbox whose poison flag is set (as a merge that ran out of time leaves it) gives NaN
    outputs at once, without waiting, until it is initialised again; the flag is forced from the
    host here, so no kernel waits or times out."""
    nh, nkv, ctx = 16, 2, 8192
    q, kb, vb, qd, kc, vc = _inputs(dev, 9, ctx, 1, nh, nkv)
    mb = ops.attn_mailbox(ctx, 1, nh, dev)
    mb[:4] = 1
    got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb))
    assert np.isnan(got).all()
    assert ops.attn_mailbox_poisoned(mb)
    # that call has completed: the next one fails before any device work
    from irontimber_amd._lib import ItError, call
    with pytest.raises(ItError, match="poisoned"):
        ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb)
    call("it_attn_mailbox_init", mb.data_ptr(), mb.numel(), torch.cuda.current_stream().cuda_stream)
    got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb))
    np.testing.assert_array_equal(got, host(ops.attn_f16(qd, kc, vc, ctx - 1, nh, nkv)))
    assert _clean(mb)


def test_uninitialised_mailbox_fails_loudly(dev):
    """A mailbox that it_attn_mailbox_init never filled (here zeroed device memory, whose words
    would otherwise pass for records) is treated as poisoned: NaN outputs, the flag reported."""
    nh, nkv, ctx = 16, 2, 8192
    q, kb, vb, qd, kc, vc = _inputs(dev, 11, ctx, 1, nh, nkv)
    mb = torch.zeros(ops.lib().it_attn_mailbox_bytes(ctx, 1, nh), device=dev, dtype=torch.uint8)
    assert ops.attn_mailbox_poisoned(mb)
    got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb))
    assert np.isnan(got).all()


@pytest.mark.parametrize("bits", [0xFFFF, 0x7E01, 0xFC00])
def test_nonfinite_value_does_not_poison_the_mailbox(dev, bits):
    """A NaN or infinite value in V (f16 0xFFFF: a NaN with every payload bit set; 0x7E01; -inf)
    reaches the outputs of that call as it does on the two-launch path, and leaves the mailbox
    clean: record words are stored with NaN canonicalised, so no stored word equals the empty
    pattern and no merge waits on a piece that looks unwritten. The next call is exact again."""
    nh, nkv, ctx = 16, 2, 8192
    q, kb, vb, qd, kc, vc = _inputs(dev, 13, ctx, 1, nh, nkv)
    mb = ops.attn_mailbox(ctx, 1, nh, dev)
    bad = vb.copy()
    bad[4000, 3] = bits                      # key 4000, KV head 0, dim 3
    vbad = dev_f16bits(bad, dev)
    got = host(ops.attn_f16_mailbox(qd, kc, vbad, ctx - 1, nh, nkv, mb))
    ref = host(ops.attn_f16(qd, kc, vbad, ctx - 1, nh, nkv))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))
    assert not np.isfinite(got[0, 3])        # head 0 sees the key: dim 3 is not finite
    assert not ops.attn_mailbox_poisoned(mb) and _clean(mb)
    got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, nh, nkv, mb))
    np.testing.assert_array_equal(got, host(ops.attn_f16(qd, kc, vc, ctx - 1, nh, nkv)))
