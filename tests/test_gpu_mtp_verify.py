"""MTP verify checkpoint and rollback of the GDN recurrent state (src/vk/mod.rs:790-801 checkpoint
after token 0, 1018-1025 rollback; CPU semantics mtp.rs:227-234), through the C ABI."""
import numpy as np
import pytest
import torch

import oracle
from irontimber_amd import ops
from irontimber_amd._lib import ItError
from irontimber_amd.synth import gdn_inputs, gdn_step_inputs
from tests.gpu_util import announce, assert_argmax_agrees, dev_f32, host

pytestmark = pytest.mark.gpu
STATE_TOL, OUT_TOL = 5e-3, 2e-3


def _step_args(d, dev):
    return [dev_f32(d[k], dev) for k in ("co", "beta_raw", "alpha_raw", "dt", "a")]


@pytest.mark.parametrize("nt,ck_after,nv,nk", [(2, 0, 32, 16), (4, 2, 32, 16), (3, 2, 8, 4), (17, 5, 4, 2)])
def test_step_checkpoint_is_the_prefix_state(dev, nt, ck_after, nv, nk):
    """The checkpoint equals the state after running only tokens 0..ck_after (bit for bit: the same
    arithmetic in the same order), and the checkpointing call's outputs and final state equal the
    plain call's."""
    announce(f"gdn_step ckpt nt={nt} after={ck_after} nv={nv}")
    d = gdn_step_inputs(21, nt, nv=nv, nk=nk)
    co, br, ar, dt, a = _step_args(d, dev)
    st, ck = dev_f32(d["state"], dev), torch.full_like(dev_f32(d["state"], dev), float("nan"))
    out = host(ops.gdn_step(co, br, ar, dt, a, st, nv, nk, ckpt=ck, ckpt_after=ck_after))
    st_plain = dev_f32(d["state"], dev)
    out_plain = host(ops.gdn_step(co, br, ar, dt, a, st_plain, nv, nk))
    np.testing.assert_array_equal(out, out_plain)
    np.testing.assert_array_equal(host(st), host(st_plain))
    st_pre = dev_f32(d["state"], dev)
    n = ck_after + 1
    ops.gdn_step(co[:n].contiguous(), br[:n].contiguous(), ar[:n].contiguous(), dt, a, st_pre, nv, nk)
    np.testing.assert_array_equal(host(ck), host(st_pre))


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("nt,ck_after,K", [(2, 0, 4), (4, 3, 4), (3, 1, 3), (40, 17, 4), (40, 0, 2)])
def test_conv_checkpoint_is_the_prefix_state(dev, fused, nt, ck_after, K):
    """Conv state checkpoint after token ck_after, for one token run (written from the window) and
    for several runs (nt > 16: written by the state kernel before the conv)."""
    announce(f"conv ckpt fused={fused} nt={nt} after={ck_after} K={K}")
    d = gdn_inputs(22, nt=nt, nv=8, nk=4)
    x, w = dev_f32(d["x"], dev), dev_f32(d["w"][:, :K], dev)
    st0 = d["conv_state"][:K - 1]
    run = (lambda x_, st_, **kw: ops.gdn_conv_l2norm(x_, w, st_, 8, **kw)) if fused else \
          (lambda x_, st_, **kw: ops.gdn_conv(x_, w, st_, **kw))
    st, ck = dev_f32(st0, dev), torch.full_like(dev_f32(st0, dev), float("nan"))
    out = host(run(x, st, ckpt=ck, ckpt_after=ck_after))
    st_plain = dev_f32(st0, dev)
    np.testing.assert_array_equal(out, host(run(x, st_plain)))
    np.testing.assert_array_equal(host(st), host(st_plain))
    st_pre = dev_f32(st0, dev)
    run(x[:ck_after + 1].contiguous(), st_pre)
    np.testing.assert_array_equal(host(ck), host(st_pre))
    _, want_ck = oracle.gdn_conv(d["x"][:ck_after + 1], d["w"][:, :K], st0)
    np.testing.assert_array_equal(host(ck), want_ck)


def _oracle_layer(d, toks, nv, nk, S=128):
    """cpu.rs:194-232 over the given token rows, sequentially, from d's initial states."""
    x = np.ascontiguousarray(d["x"][toks])
    br = np.ascontiguousarray(d["beta_raw"][toks]); ar = np.ascontiguousarray(d["alpha_raw"][toks])
    nt = len(toks)
    cst, sst = d["conv_state"].copy(), d["state"].copy()
    out = np.zeros((nt, nv * S), np.float32); co = np.zeros((nt, d["cd"]), np.float32)
    P = lambda a: a.ctypes.data
    oracle.lib().it_ref_gdn_layer(P(x), d["cd"], P(d["w"]), P(cst), 4, P(br), P(ar), nv, P(d["dt"]), P(d["a"]),
                                  P(sst), P(out), nv * S, P(co), nt, nv, nk, S, 1e-6, oracle.hardware_threads())
    return out, cst, sst


@pytest.mark.parametrize("accept", [True, False])
def test_verify_accept_or_reject_cycle(dev, accept):
    """One GDN layer at the BASELINE geometry (32 V / 16 QK heads, K = 4). Verify the pair
    [x, draft] in one nt = 2 call with checkpoints after token 0. Accept: the state is the oracle's
    after [x, draft]. Reject: roll back, run the corrected token c; the state and output are the
    oracle's after [x, c] (the CPU backend's mtp_reject + next step, mtp.rs:227-234)."""
    nv, nk, S = 32, 16, 128
    d = gdn_inputs(23, nt=3, nv=nv, nk=nk)       # rows: 0 = x, 1 = draft, 2 = correction
    announce(f"mtp verify cycle accept={accept}")
    t = lambda a: dev_f32(a, dev)
    w, dtv, av = t(d["w"]), t(d["dt"]), t(d["a"])
    cst, sst = t(d["conv_state"]), t(d["state"])
    ck_conv, ck_ssm = torch.empty_like(cst), torch.empty_like(sst)
    co = ops.gdn_conv_l2norm(t(d["x"][0:2]), w, cst, 2 * nk, ckpt=ck_conv, ckpt_after=0)
    o2 = host(ops.gdn_step(co, t(d["beta_raw"][0:2]), t(d["alpha_raw"][0:2]), dtv, av, sst, nv, nk, ckpt=ck_ssm,
                           ckpt_after=0))
    want2, wc2, ws2 = _oracle_layer(d, [0, 1], nv, nk)
    assert np.abs(o2 - want2).max() <= OUT_TOL
    assert_argmax_agrees(o2, want2)
    if accept:
        assert np.abs(host(sst) - ws2).max() <= STATE_TOL
        np.testing.assert_array_equal(host(cst), wc2)
        return
    ops.gdn_rollback(ck_conv, cst, ck_ssm, sst)
    co = ops.gdn_conv_l2norm(t(d["x"][2:3]), w, cst, 2 * nk)
    o1 = host(ops.gdn_step(co, t(d["beta_raw"][2:3]), t(d["alpha_raw"][2:3]), dtv, av, sst, nv, nk))
    want, wc, ws = _oracle_layer(d, [0, 2], nv, nk)
    e_out, e_st = np.abs(o1 - want[1:]).max(), np.abs(host(sst) - ws).max()
    print(f"reject path: out {e_out:.3g} state {e_st:.3g}")
    assert e_out <= OUT_TOL and e_st <= STATE_TOL
    np.testing.assert_array_equal(host(cst), wc)
    assert_argmax_agrees(o1, want[1:])


def test_checkpoint_validation(dev):
    d = gdn_step_inputs(24, 2, nv=4, nk=2)
    co, br, ar, dt, a = _step_args(d, dev)
    st = dev_f32(d["state"], dev)
    with pytest.raises(ItError, match="outside"):
        ops.gdn_step(co, br, ar, dt, a, st, 4, 2, ckpt=torch.empty_like(st), ckpt_after=2)
    with pytest.raises(ItError, match="overlaps"):
        ops.gdn_step(co, br, ar, dt, a, st, 4, 2, ckpt=st, ckpt_after=0)


@pytest.mark.gpu
@pytest.mark.parametrize("nc,ns,offs", [(24576, 524288, 0), (3 * 8192, 0, 0), (0, 4096, 0), (1001, 777, 1), (5, 4099, 0)])
def test_rollback_copies(dev, nc, ns, offs):
    """it_gdn_rollback's one copy kernel: both ranges restored exactly and nothing past them touched,
    with whole-f4 moves (aligned, multiples of 4) and the float path (odd counts, unaligned)."""
    announce(f"rollback nc={nc} ns={ns} offs={offs}")
    g = torch.Generator().manual_seed(nc * 7 + ns)
    ckc = torch.randn(nc + offs + 8, generator=g).to(dev)
    cks = torch.randn(ns + offs + 8, generator=g).to(dev)
    cst = torch.full((nc + offs + 8,), 7.0, device=dev)
    sst = torch.full((ns + offs + 8,), 7.0, device=dev)
    ops.gdn_rollback(ckc[offs:offs + nc], cst[offs:offs + nc], cks[offs:offs + ns], sst[offs:offs + ns])
    torch.cuda.synchronize()
    assert torch.equal(cst[offs:offs + nc], ckc[offs:offs + nc]) and torch.equal(sst[offs:offs + ns], cks[offs:offs + ns])
    assert bool((cst[:offs] == 7).all()) and bool((cst[offs + nc:] == 7).all())
    assert bool((sst[:offs] == 7).all()) and bool((sst[offs + ns:] == 7).all())
