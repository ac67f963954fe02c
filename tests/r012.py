"""The reference's known-answer attention fixture (src/vk/r012_parity.rs:5-9), rebuilt from its
closed-form inputs: every arena word i holds ((17 i mod 1009) - 504) / 503, the q rows come first
(token stride 2*nh*hd), then the f32 K rows, then the f32 V rows (row stride kvd)."""
import numpy as np

CASES = [(0, 1), (0, 64), (63, 2), (64, 2), (65, 1), (2047, 2), (4095, 2), (8190, 2)]   # r012_parity.rs:6
GEOMS = [(24, 4, 256), (16, 2, 256)]   # the reference's geometry, then the BASELINE one


def arena(pos0: int, nt: int, nh: int, nkv: int, hd: int):
    kvd = nkv * hd
    qts = nh * hd * 2
    total = pos0 + nt
    kf = nt * qts
    vf = kf + total * kvd
    n = vf + total * kvd
    i = np.arange(n, dtype=np.int64)
    a = (((i * 17) % 1009).astype(np.float32) - np.float32(504.0)) / np.float32(503.0)
    q = a[:kf].reshape(nt, qts)
    k = a[kf:vf].reshape(total, kvd)
    v = a[vf:n].reshape(total, kvd)
    return q, k, v
