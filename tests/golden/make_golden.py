"""Writes the committed golden fixtures of this directory (run from the repository root:
python3 tests/golden/make_golden.py). Nothing here runs the reference (Rust, not buildable in this
image): the inputs are the reference's own known-answer inputs, and the expected outputs come from
float64 statements of the arithmetic, independent of the HIP kernels and of the C++ oracle's f32
arithmetic.

- r012_baseline.npz: the closed-form attention arena of src/vk/r012_parity.rs:6-28 at the BASELINE
  geometry (16 q / 2 KV heads, hd 256), RTZ f16 K/V, scale 1/16; float64 softmax + sigmoid gate,
  stored as float32. Every token of the short cases and the last token of the 64-token case.
- kparity.npz: the kernel-parity harness inputs of src/vk/kparity.rs:13, 31-36, 59-63 (xorshift64
  arena and params) for its attn (f32 cache), conv (cd 1000, 5 tokens, K 4) and gdn / gdn_p cases
  (6 tokens, 4 V / 2 QK heads, unnormalised q/k), with float64 expected outputs (the final GDN
  state as float32)."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402  (the xorshift draws of kparity.rs:13, restated in oracle/cpu_ref.cpp)
from irontimber_amd.synth import f16_bits_rtz  # noqa: E402
from oracle.ref_np import attn_f64, f16_to_f64, gdn_seq_f64  # noqa: E402
from tests.r012 import CASES, arena  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
MB = 1 << 20


def r012():
    nh, nkv, hd = 16, 2, 256
    out = {}
    for pos0, nt in CASES:
        q, k, v = arena(pos0, nt, nh, nkv, hd)
        want = attn_f64(q, f16_to_f64(f16_bits_rtz(k)), f16_to_f64(f16_bits_rtz(v)), pos0, nh, nkv, hd, 1.0 / 16)
        rows = list(range(nt)) if nt <= 2 else [nt - 1]
        out[f"out_{pos0}_{nt}"] = want[rows].astype(np.float32)
        out[f"rows_{pos0}_{nt}"] = np.array(rows, np.int32)
        out[f"qsum_{pos0}_{nt}"] = np.array([q.astype(np.float64).sum(), k.astype(np.float64).sum()])
    np.savez(os.path.join(HERE, "r012_baseline.npz"), cases=np.array(CASES, np.int32), **out)


def conv_f64(x, w, st0):
    K = w.shape[1]
    xx = np.concatenate([st0, x]).astype(np.float64)
    out = np.zeros(x.shape)
    for t in range(x.shape[0]):
        s = (xx[t:t + K].T * w.astype(np.float64)).sum(axis=1)
        out[t] = s / (1.0 + np.exp(-s))
    return out


def kparity():
    a, p = oracle.kparity_draws(5 << 20, 1 << 16)
    p = p.copy()
    p[16:20] = -np.abs(p[16:20]) - 0.1      # gdn decay a < 0, set before every case (kparity.rs:63)
    d = {}
    # attn (kparity.rs:34): 4 heads / 2 KV heads, pos0 5, 3 tokens, f32 cache, scale 1/16
    nt, pos0, nh, nkv = 3, 5, 4, 2
    q = a[:nt * 2048].reshape(nt, 2048)
    kc = a[MB:MB + (pos0 + nt) * 512].reshape(pos0 + nt, 512)
    vc = a[2 * MB:2 * MB + (pos0 + nt) * 512].reshape(pos0 + nt, 512)
    d.update(attn_q=q, attn_k=kc, attn_v=vc,
             attn_out=attn_f64(q, kc.astype(np.float64), vc.astype(np.float64), pos0, nh, nkv, 256, 1.0 / 16))
    # conv (kparity.rs:32): cd 1000, 5 tokens, K 4
    cd, nc, K = 1000, 5, 4
    x = a[:nc * cd].reshape(nc, cd)
    w = p[:cd * K].reshape(cd, K)
    st0 = a[2 * MB:2 * MB + (K - 1) * cd].reshape(K - 1, cd)
    d.update(conv_x=x, conv_w=w, conv_state=st0, conv_out=conv_f64(x, w, st0))
    # gdn / gdn_p (kparity.rs:35-36): 6 tokens, 4 V / 2 QK heads, S 128
    co = a[:6 * 1024].reshape(6, 1024)
    br, ar = a[MB:MB + 24].reshape(6, 4), a[MB + 64:MB + 88].reshape(6, 4)
    st = a[2 * MB:2 * MB + 4 * 128 * 128].reshape(4, 128, 128)
    o64, s64 = gdn_seq_f64(co, br, ar, p[0:4], p[16:20], st, 4, 2)
    d.update(gdn_co=co, gdn_beta=br, gdn_alpha=ar, gdn_dt=p[0:4], gdn_a=p[16:20], gdn_state=st, gdn_out=o64,
             gdn_state_out=s64.astype(np.float32))
    np.savez(os.path.join(HERE, "kparity.npz"), **d)


if __name__ == "__main__":
    r012()
    kparity()
    for f in ("r012_baseline.npz", "kparity.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
