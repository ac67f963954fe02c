"""The matrix-core rate probe (it_calib_mfma_f16) that bench.py quotes the prefill roofline
against: it must run exactly the MFMA chains it is asked for."""
import pytest
import torch

from irontimber_amd._lib import ItError, call
from tests.gpu_util import announce


@pytest.mark.gpu
def test_probe_counts_its_ops(dev):
    """Every accumulator gets iters identical products, all exact in f32 (operands are multiples
    of 1/8 and 1/16 below 1, so each thread's sum is a multiple of 1/128 far below 2^24 / 128):
    the output at iters = 8 is exactly 8 times the output at iters = 1."""
    announce("mfma probe")
    st = torch.cuda.current_stream().cuda_stream
    o1 = torch.empty(4 * 256, device=dev)
    o8 = torch.empty(4 * 256, device=dev)
    call("it_calib_mfma_f16", 4, 1, o1.data_ptr(), st)
    call("it_calib_mfma_f16", 4, 8, o8.data_ptr(), st)
    torch.cuda.synchronize()
    assert bool((o1 > 0).all())
    assert torch.equal(o8, o1 * 8)


def test_probe_rejects_bad_arguments():
    with pytest.raises(ItError):
        call("it_calib_mfma_f16", 0, 1, 1 << 20, None)
