"""The reference's kernel-parity harness cases for this path (src/vk/kparity.rs:31-36) on its own
xorshift arena and params (kparity.rs:13, 59-63), through the C ABI, against the oracle and float64.
The harness compares two GPU kernel sets with max |a - b| / max(1, |b|) <= 1e-4 over the arena
(kparity.rs:2-3); the same relative measure is used here against the oracle."""
import numpy as np
import pytest
import torch

import oracle
from oracle.ref_np import gdn_seq_f64
from irontimber_amd import ops
from tests.gpu_util import announce, dev_f32, host

pytestmark = pytest.mark.gpu
MB = 1 << 20


def draws():
    a, p = oracle.kparity_draws(5 << 20, 1 << 16)
    p = p.copy()
    p[16:20] = -np.abs(p[16:20]) - 0.1      # gdn decay a < 0, like the model (kparity.rs:63)
    return a, p


def rel_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(1.0, np.abs(want))))


def test_kparity_attn_f32_cache(dev):
    """"attn" (kparity.rs:34): q at arena 0 (token stride 2048 = 4 heads x [q | gate]), f32 K/V
    caches at arena 1M / 2M (kvd 512 = 2 KV heads x 256), pos0 5, 3 tokens, scale 1/16."""
    a, _ = draws()
    nt, pos0, nh, nkv = 3, 5, 4, 2
    q = a[:nt * 2048].reshape(nt, 2048)
    kc = a[MB:MB + (pos0 + nt) * 512].reshape(pos0 + nt, 512)
    vc = a[2 * MB:2 * MB + (pos0 + nt) * 512].reshape(pos0 + nt, 512)
    announce("kparity attn f32 cache")
    got = host(ops.attn_f32kv(dev_f32(q, dev), dev_f32(kc, dev), dev_f32(vc, dev), pos0, nh, nkv, scale=1.0 / 16))
    want = oracle.attn_f32kv(q, kc, vc, pos0, nh, nkv, scale=1.0 / 16)
    # float64 statement of cpu.rs:260-272 (also mtp.rs:122-130) for the same rows
    ref = np.zeros((nt, nh * 256))
    for t in range(nt):
        n = pos0 + t + 1
        for h in range(nh):
            kh = h // (nh // nkv)
            qv = q[t, h * 512:h * 512 + 256].astype(np.float64)
            gate = q[t, h * 512 + 256:h * 512 + 512].astype(np.float64)
            s = kc[:n, kh * 256:(kh + 1) * 256].astype(np.float64) @ qv / 16.0
            e = np.exp(s - s.max())
            ref[t, h * 256:(h + 1) * 256] = (e / e.sum()) @ vc[:n, kh * 256:(kh + 1) * 256].astype(np.float64) / (1 + np.exp(-gate))
    print(f"kparity attn: gpu-f64 {rel_err(got, ref):.3g} oracle-f64 {rel_err(want, ref):.3g}")
    assert rel_err(got, ref) <= 2e-6 and rel_err(want, ref) <= 2e-6


def gdn_case():
    """"gdn" / "gdn_p" (kparity.rs:35-36): 6 tokens, co at arena 0 (stride 1024: 2 QK heads of q,
    2 of k, 4 V heads), beta at arena 1M + 4t + h, alpha at 1M + 64 + 4t + h, dt at params 0,
    a at params 16, state [4][128][128] at arena 2M; q/k are the raw draws (no L2 norm)."""
    a, p = draws()
    nt, nv, nk = 6, 4, 2
    co = a[:nt * 1024].reshape(nt, 1024)
    br = a[MB:MB + nt * 4].reshape(nt, 4)
    ar = a[MB + 64:MB + 64 + nt * 4].reshape(nt, 4)
    dt, av = p[0:4].copy(), p[16:20].copy()
    st = a[2 * MB:2 * MB + nv * 128 * 128].reshape(nv, 128, 128)
    return co, br, ar, dt, av, st, nv, nk


def test_kparity_gdn_token_sequential(dev):
    """The recurrence kernels (gdn: one token a launch; gdn_p: the 6-token run) against the oracle and
    the float64 recurrence. With unnormalised k (|k|^2 ~ 43) the delta rule amplifies rounding by
    ~|1 - beta |k|^2| per token, so the bound is relative, as in the harness."""
    co, br, ar, dt, av, st, nv, nk = gdn_case()
    o64, s64 = gdn_seq_f64(co, br, ar, dt, av, st, nv, nk)
    wo, ws = oracle.gdn_step(co, br, ar, dt, av, st, nv, nk)
    announce("kparity gdn 6 tokens, one call")
    sd = dev_f32(st, dev)
    got = host(ops.gdn_step(dev_f32(co, dev), dev_f32(br, dev), dev_f32(ar, dev), dev_f32(dt, dev), dev_f32(av, dev),
                            sd, nv, nk))
    gst = host(sd)
    # the decode form: one token per call, the state carried in place
    sd1 = dev_f32(st, dev)
    got1 = np.concatenate([host(ops.gdn_step(dev_f32(co[t:t + 1], dev), dev_f32(br[t:t + 1], dev),
                                             dev_f32(ar[t:t + 1], dev), dev_f32(dt, dev), dev_f32(av, dev), sd1, nv, nk))
                           for t in range(6)])
    scale = max(1.0, float(np.abs(o64).max()))
    print(f"kparity gdn: |out| max {np.abs(o64).max():.3g}; rel gpu {rel_err(got, o64):.3g} one-token "
          f"{rel_err(got1, o64):.3g} oracle {rel_err(wo, o64):.3g}; state rel {rel_err(gst, s64):.3g}")
    for x in (got, got1, wo):
        assert rel_err(x, o64) <= 1e-4
    for s_ in (gst, host(sd1), ws):
        assert rel_err(s_, s64) <= 1e-4
    del scale


def test_kparity_gdn_chunked_normalised(dev):
    """The chunk-64 scan on the same draws with q and k L2-normalised per head, as the layer's
    rmsnorm mode 2 guarantees before the recurrence (cpu.rs:214): within the north-star bounds of
    the float64 recurrence. (Its f16 operand records assume |k| <= 1.)"""
    co, br, ar, dt, av, st, nv, nk = gdn_case()
    co = co.copy()
    qk = co[:, :2 * nk * 128].reshape(6, 2 * nk, 128).astype(np.float64)
    co[:, :2 * nk * 128] = (qk / np.maximum(np.linalg.norm(qk, axis=-1, keepdims=True), 1e-6)).reshape(6, -1)
    st = (st * 0.02).astype(np.float32)
    o64, s64 = gdn_seq_f64(co, br, ar, dt, av, st, nv, nk)
    sd = dev_f32(st, dev)
    got = host(ops.gdn_step(dev_f32(co, dev), dev_f32(br, dev), dev_f32(ar, dev), dev_f32(dt, dev), dev_f32(av, dev),
                            sd, nv, nk, chunked=True))
    assert np.abs(got - o64).max() <= 2e-3 and np.abs(host(sd) - s64).max() <= 5e-3
