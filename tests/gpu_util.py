"""Helpers for the GPU parity tests: numpy <-> device tensors, named progress lines."""
import sys

import numpy as np
import torch


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def dev_f16bits(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _projection(dim: int, n_cls: int = 997, seed: int = 1234) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((dim, n_cls)).astype(np.float64)


def argmax_projection(out: np.ndarray, n_cls: int = 997, seed: int = 1234) -> np.ndarray:
    """Fixed random projection of every output row, then argmax: the downstream-argmax check."""
    return (out.astype(np.float64) @ _projection(out.shape[-1], n_cls, seed)).argmax(axis=-1)


def assert_argmax_agrees(got: np.ndarray, want: np.ndarray, n_cls: int = 997, seed: int = 1234, sigmas: float = 4.0):
    """The downstream-argmax check: the argmax of a fixed random projection of every output row is
    identical, except on rows where the oracle's own top-2 margin is inside the noise of the
    measured error. For an error row e independent of the N(0,1) projection W, the change of the
    difference of two logits is e.(W_a - W_b) ~ N(0, 2|e|^2); a row may flip only if its oracle
    margin is below `sigmas` standard deviations of that (a near tie no finite-precision kernel
    can decide). Returns the number of such near-tie flips."""
    W = _projection(got.shape[-1], n_cls, seed)
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    w = want.reshape(-1, want.shape[-1]).astype(np.float64)
    lg, lw = g @ W, w @ W
    ag, aw = lg.argmax(-1), lw.argmax(-1)
    rows = np.nonzero(ag != aw)[0]
    if rows.size == 0:
        print(f"argmax: identical on all {g.shape[0]} rows")
        return 0
    margin = lw[rows, aw[rows]] - lw[rows, ag[rows]]
    noise = np.sqrt(2.0) * np.linalg.norm(g[rows] - w[rows], axis=-1)
    bad = rows[margin > sigmas * noise]
    assert bad.size == 0, f"argmax differs on {bad.size} rows with margins above {sigmas} sigma: {bad[:8]}"
    print(f"argmax: {rows.size} near-tie rows of {g.shape[0]} (margins {margin.max():.2e} <= {sigmas} sigma)")
    return int(rows.size)
