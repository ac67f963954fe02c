"""Guard bands around every caller-owned scratch the compiled kernels write: each buffer is given
exactly the bytes its size function returns (it_attn_scratch_bytes_ex, it_attn_f32kv_scratch_bytes,
it_attn_mailbox_bytes, it_gdn_chunked_scratch_bytes, it_gdn_prefill_scratch_bytes), with 64 KiB of a
sentinel byte before and after it. After the call both bands must be untouched, so an index
formula in a kernel that drifts past its records (or before them) fails here, on the kernels
themselves; the results are checked against the oracle as well."""
import numpy as np
import pytest
import torch

import oracle
from irontimber_amd import ops
from irontimber_amd._lib import lib
from irontimber_amd.synth import attn_inputs, gdn_inputs
from tests.gpu_util import announce, dev_f16bits, dev_f32, host

pytestmark = pytest.mark.gpu
GUARD = 1 << 16
SENT = 0xA5


def banded(n, dev):
    """(whole buffer, view of exactly n bytes between two sentinel bands)."""
    buf = torch.full((GUARD + n + GUARD,), SENT, dtype=torch.uint8, device=dev)
    return buf, buf[GUARD:GUARD + n]


def assert_bands(buf, n):
    torch.cuda.synchronize()
    assert bool((buf[:GUARD] == SENT).all()), "written before the scratch"
    assert bool((buf[GUARD + n:] == SENT).all()), "written past the scratch"


@pytest.mark.parametrize("ctx,nt,nh,nkv,kernel,chunk", [
    (8192, 1, 16, 2, ops.KERNEL_SPLITK, 64), (8192, 4, 16, 2, ops.KERNEL_SPLITK, 64),
    (8192, 1, 16, 2, ops.KERNEL_SPLITK, 192), (777, 33, 16, 2, ops.KERNEL_SPLITK, 64),
    (100, 3, 16, 2, ops.KERNEL_SPLITK, 128), (65, 1, 24, 4, ops.KERNEL_SPLITK, 64), (300, 5, 8, 8, ops.KERNEL_SPLITK, 64),
    (4096 + 64, 64, 16, 2, ops.KERNEL_FLASH, 0), (4096 + 64, 64, 16, 2, ops.KERNEL_FLASH, 64),
    (4096 + 64, 64, 16, 2, ops.KERNEL_FLASH, 640), (333, 129, 24, 4, ops.KERNEL_FLASH, 64),
    (1000, 64, 4, 1, ops.KERNEL_FLASH, 128), (4096 + 64, 64, 16, 2, ops.KERNEL_FLASH_F32, 0),
    (333, 129, 24, 4, ops.KERNEL_FLASH_F32, 64), (8192, 64, 16, 2, ops.KERNEL_FLASH, 0),
])
def test_attention_scratch_bands(dev, ctx, nt, nh, nkv, kernel, chunk):
    pos0 = ctx - nt
    n = ops.attn_scratch_bytes(pos0, nt, nh, nkv, 256, kernel, chunk)
    announce(f"bands attn ctx={ctx} nt={nt} nh={nh}/{nkv} kernel={kernel} chunk={chunk} bytes={n}")
    assert n > 0
    q, kb, vb = attn_inputs(41, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    buf, scr = banded(n, dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    got = host(ops.attn_f16(dev_f32(q.reshape(nt, -1), dev), kc, vc, pos0, nh, nkv, scratch=scr, kernel=kernel,
                            chunk=chunk))
    assert_bands(buf, n)
    want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, nh, nkv)
    assert np.abs(got - want).max() <= 2e-3


@pytest.mark.parametrize("rows,nt,nh,nkv,splits", [(8192, 1, 16, 2, 0), (8192, 2, 16, 2, 0), (4096 + 64, 64, 16, 2, 0),
                                                   (4096 + 64, 64, 16, 2, 3), (129, 7, 4, 1, 0), (777, 33, 24, 4, 2)])
def test_f32kv_scratch_bands(dev, rows, nt, nh, nkv, splits):
    """The preferred scratch (splits 0), or room for `splits` records per row (longer splits)."""
    pos0 = rows - nt
    n = lib().it_attn_f32kv_scratch_bytes(pos0, nt, 256, nh, nkv) if not splits else nt * nh * splits * 1040
    announce(f"bands f32kv rows={rows} nt={nt} nh={nh}/{nkv} bytes={n}")
    rng = np.random.default_rng(rows + nt)
    q = rng.standard_normal((nt, nh * 512)).astype(np.float32)
    k = rng.standard_normal((rows, nkv * 256)).astype(np.float32)
    v = rng.standard_normal((rows, nkv * 256)).astype(np.float32)
    buf, scr = banded(n, dev)
    got = host(ops.attn_f32kv(dev_f32(q, dev), dev_f32(k, dev), dev_f32(v, dev), pos0, nh, nkv, scratch=scr))
    assert_bands(buf, n)
    assert np.abs(got - oracle.attn_f32kv(q, k, v, pos0, nh, nkv)).max() <= 2e-5


@pytest.mark.parametrize("ctx", [8192, 2048])
def test_mailbox_bands(dev, ctx):
    """The one-launch decode's mailbox of exactly it_attn_mailbox_bytes: two calls in a row (the
    second finds the pieces the first cleared), nothing written outside it."""
    n = lib().it_attn_mailbox_bytes(ctx, 1, 16)
    announce(f"bands mailbox ctx={ctx} bytes={n}")
    buf, mb = banded(n, dev)
    from irontimber_amd._lib import call
    call("it_attn_mailbox_init", mb.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    assert ops.attn_mailbox_would_launch(ctx - 1, 1, 16, 2, mb)
    q, kb, vb = attn_inputs(43, ctx=ctx, nt=1)
    qd, kc, vc = dev_f32(q.reshape(1, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    want = oracle.attn(q.reshape(1, -1), kb, vb, ctx - 1, 16, 2)
    for _ in range(2):
        got = host(ops.attn_f16_mailbox(qd, kc, vc, ctx - 1, 16, 2, mb))
        assert np.abs(got - want).max() <= 2e-3
    assert_bands(buf, n)
    assert not ops.attn_mailbox_poisoned(mb)


@pytest.mark.parametrize("nt", [64, 200, 1000])
def test_gdn_scratch_bands(dev, nt):
    """The chunked GDN scan's records and the one-call prefill's f16 conv output + records."""
    d = gdn_inputs(47, nt=nt)
    t = lambda a: dev_f32(a, dev)
    n = lib().it_gdn_prefill_scratch_bytes(nt, 32, 16, 128)
    announce(f"bands gdn prefill nt={nt} bytes={n}")
    buf, scr = banded(n, dev)
    st = t(d["state"])
    cs = t(d["conv_state"])
    out = host(ops.gdn_prefill(t(d["x"]), t(d["w"]), cs, t(d["beta_raw"]), t(d["alpha_raw"]), t(d["dt"]), t(d["a"]),
                               st, 32, 16, scratch=scr))
    assert_bands(buf, n)
    assert np.isfinite(out).all()
    # the chunked scan alone over the f32 conv output
    co = np.zeros((nt, d["cd"]), np.float32)
    cs2, ss2 = d["conv_state"].copy(), d["state"].copy()
    gref = np.zeros((nt, 32 * 128), np.float32)
    P = lambda a_: a_.ctypes.data
    oracle.lib().it_ref_gdn_layer(P(d["x"]), d["cd"], P(d["w"]), P(cs2), 4, P(d["beta_raw"]), P(d["alpha_raw"]), 32,
                                  P(d["dt"]), P(d["a"]), P(ss2), P(gref), 32 * 128, P(co), nt, 32, 16, 128, 1e-6,
                                  oracle.hardware_threads())
    assert np.abs(out - gref).max() <= 2e-3
    n2 = lib().it_gdn_chunked_scratch_bytes(nt, 32, 128)
    buf2, scr2 = banded(n2, dev)
    st2 = t(d["state"])
    out2 = host(ops.gdn_step(t(co), t(d["beta_raw"]), t(d["alpha_raw"]), t(d["dt"]), t(d["a"]), st2, 32, 16,
                             chunked=True, scratch=scr2))
    assert_bands(buf2, n2)
    assert np.abs(out2 - gref).max() <= 2e-3
