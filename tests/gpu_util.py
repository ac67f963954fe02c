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


def argmax_projection(out: np.ndarray, n_cls: int = 997, seed: int = 1234) -> np.ndarray:
    """Fixed random projection of every output row, then argmax: the downstream-argmax check."""
    W = np.random.default_rng(seed).standard_normal((out.shape[-1], n_cls)).astype(np.float64)
    return (out.astype(np.float64) @ W).argmax(axis=-1)
