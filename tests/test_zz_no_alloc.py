"""it_attn_f16_noalloc (partial records in the library's device array, no allocation) against
it_attn_f16 with a caller buffer and the same split, through the C ABI: bit-identical outputs on
two calls in a row, the second with a smaller input, and the oracle's tolerance on both."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from irontimber_amd import _lib
from irontimber_amd.synth import attn_inputs
from tests.gpu_util import announce, dev_f16bits, dev_f32, host

TOL = 2e-3
NOALLOC_BYTES = 16 << 20


def test_noalloc_rejects_oversized_geometry_before_device_work():
    """A split-K geometry whose minimum record set (nt*nh*1040 bytes) exceeds the 16 MiB array is
    refused with a message, before any device access (the pointers are never dereferenced)."""
    fake = ctypes.c_void_p(1 << 20)
    nt, nh = 15, 1200
    rc = _lib.lib().it_attn_f16_noalloc(fake, nh * 512, fake, fake, 256, 0, 256, nh, 1, nt, 0.0625, fake, nh * 256,
                                        None)
    assert rc != 0 and "device scratch" in _lib.last_error()


def plan(pos0, nt, budget):
    k, c, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    assert _lib.lib().it_attn_plan(pos0, nt, 256, 16, 2, budget, ctypes.byref(k), ctypes.byref(c), ctypes.byref(b)) == 0
    return k.value, c.value, b.value


@pytest.mark.gpu
def test_noalloc_matches_caller_scratch(dev):
    calls = [(2, 4096, 64), (1, 1000, 1)]    # config 3(i) chunk, then a smaller decode call
    for seed, pos0, nt in calls:
        announce(f"noalloc seed={seed} pos0={pos0} nt={nt}")
        q, kb, vb = attn_inputs(seed, ctx=pos0 + nt, nt=nt)
        qd, kc, vc = dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)
        out_a = torch.full((nt, 16 * 256), float("nan"), device=dev)
        out_b = torch.full((nt, 16 * 256), float("nan"), device=dev)
        st = torch.cuda.current_stream().cuda_stream
        _lib.call("it_attn_f16_noalloc", qd.data_ptr(), 16 * 512, kc.data_ptr(), vc.data_ptr(), 512, pos0, 256, 16, 2,
                  nt, 1.0 / 16, out_a.data_ptr(), 16 * 256, st)
        kernel, chunk, nbytes = plan(pos0, nt, NOALLOC_BYTES)
        assert nbytes <= NOALLOC_BYTES
        scr = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        _lib.call("it_attn_f16_ex", qd.data_ptr(), 16 * 512, kc.data_ptr(), vc.data_ptr(), 512, pos0, 256, 16, 2, nt,
                  1.0 / 16, out_b.data_ptr(), 16 * 256, scr.data_ptr(), scr.numel(), kernel,
                  chunk if chunk else (1 << 30), st)
        a, b = host(out_a), host(out_b)
        assert np.array_equal(a, b), f"noalloc differs from the caller-scratch call (kernel {kernel}, chunk {chunk})"
        want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, 16, 2)
        assert np.abs(a - want).max() <= TOL
