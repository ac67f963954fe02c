"""Seeded synthetic inputs for the attention / Gated-DeltaNet workloads.

The stream is the reference's splitmix64 generator (src/sampling.rs:40-45): the i-th draw
(i = 1, 2, ...) is mix(seed + i * 0x9e3779b97f4a7c15), uniform = (draw >> 11) / 2**53.
Normals use Box-Muller on two consecutive uniforms (cos branch only). Everything is vectorised
with numpy so the 8192-position workloads generate in well under a second. Tensors are drawn in
the order each builder documents, so a (config, seed) pair always yields the same bytes.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


class Rng:
    """Counter-form splitmix64 (same outputs as sampling.rs Rng::next_u64, in order)."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        self.count = 0

    def u64(self, n: int) -> np.ndarray:
        idx = np.arange(self.count + 1, self.count + n + 1, dtype=np.uint64)
        self.count += n
        with np.errstate(over="ignore"):
            z = self.state + idx * _GAMMA
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))

    def uniform(self, n: int) -> np.ndarray:
        """float64 in [0, 1)."""
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))

    def normal(self, n: int, std: float = 1.0) -> np.ndarray:
        """float32 N(0, std^2) via Box-Muller on consecutive uniform pairs."""
        u = self.uniform(2 * n).reshape(n, 2)
        r = np.sqrt(-2.0 * np.log(1.0 - u[:, 0]))
        return (r * np.cos(2.0 * np.pi * u[:, 1]) * std).astype(np.float32)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> f16 round-to-nearest-even (the half crate's f16::from_f32), returned as uint16 bits."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_rtz(x: np.ndarray) -> np.ndarray:
    """f32 -> f16 rounding toward zero (packHalf2x16 on the reference's GPU), as uint16 bits."""
    x = np.asarray(x, dtype=np.float32)
    h = x.astype(np.float16)
    back = h.astype(np.float32)
    bits = h.view(np.uint16).copy()
    over = np.abs(back) > np.abs(x)
    bits[over] -= 1
    return bits


def rmsnorm_rows(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Unit-weight RMS norm over the last axis (cpu.rs:14-18), float32."""
    x = x.astype(np.float32)
    ss = (x * x).mean(axis=-1, keepdims=True, dtype=np.float32)
    return (x / np.sqrt(ss + np.float32(eps))).astype(np.float32)


def attn_inputs(seed: int, ctx: int, nt: int, nh: int = 16, nkv: int = 2, hd: int = 256):
    """Attention workload: returns (q [nt, nh, 2*hd] f32, kc/vc [ctx, nkv*hd] f16 bits).

    Draw order: K (ctx*nkv*hd), V (same), q+gate (nt*nh*2*hd). K is RMS-normalised per head with
    unit weight and eps 1e-6 before the f16 cast; RoPE counts as already applied. The cache holds
    `ctx` rows; a call with pos0 = ctx - nt attends over all of them.
    """
    r = Rng(seed)
    k = r.normal(ctx * nkv * hd).reshape(ctx, nkv, hd)
    v = r.normal(ctx * nkv * hd).reshape(ctx, nkv * hd)
    q = r.normal(nt * nh * 2 * hd).reshape(nt, nh, 2 * hd)
    k = rmsnorm_rows(k).reshape(ctx, nkv * hd)
    return q, f16_bits(k), f16_bits(v)


def gdn_inputs(seed: int, nt: int, nv: int = 32, nk: int = 16, S: int = 128, K: int = 4):
    """Gated-DeltaNet workload (conv input side). Draw order:
    state [nv,S,S] ~ N(0, 0.02^2); conv weight [cd,K] ~ N(0,1)/2; conv state [K-1,cd] ~ N(0,1);
    x [nt,cd] ~ N(0,1); beta_raw [nt,nv] ~ N(0,1); alpha_raw [nt,nv] ~ N(0,1);
    A_log [nv] ~ U(-1,1) -> a = -exp(A_log); dt = 0.
    """
    r = Rng(seed)
    cd = 2 * nk * S + nv * S
    state = r.normal(nv * S * S, std=0.02).reshape(nv, S, S)
    w = (r.normal(cd * K) * np.float32(0.5)).reshape(cd, K)
    conv_state = r.normal((K - 1) * cd).reshape(K - 1, cd)
    x = r.normal(nt * cd).reshape(nt, cd)
    beta_raw = r.normal(nt * nv).reshape(nt, nv)
    alpha_raw = r.normal(nt * nv).reshape(nt, nv)
    a_log = (r.uniform(nv) * 2.0 - 1.0).astype(np.float32)
    a = (-np.exp(a_log)).astype(np.float32)
    dt = np.zeros(nv, np.float32)
    return dict(state=state, w=w, conv_state=conv_state, x=x, beta_raw=beta_raw, alpha_raw=alpha_raw,
                a=a, dt=dt, cd=cd)


def gdn_step_inputs(seed: int, nt: int, nv: int = 32, nk: int = 16, S: int = 128):
    """Recurrence-only inputs (conv already applied): state, co [nt, (2nk+nv)S] with q/k rows
    L2-normalised per head, beta_raw, alpha_raw, dt, a. Same distributions as gdn_inputs."""
    r = Rng(seed)
    state = r.normal(nv * S * S, std=0.02).reshape(nv, S, S)
    co = r.normal(nt * (2 * nk + nv) * S).reshape(nt, 2 * nk + nv, S)
    qk = co[:, : 2 * nk, :].astype(np.float64)
    co[:, : 2 * nk, :] = (qk / np.maximum(np.linalg.norm(qk, axis=-1, keepdims=True), 1e-6)).astype(np.float32)
    beta_raw = r.normal(nt * nv).reshape(nt, nv)
    alpha_raw = r.normal(nt * nv).reshape(nt, nv)
    a_log = (r.uniform(nv) * 2.0 - 1.0).astype(np.float32)
    a = (-np.exp(a_log)).astype(np.float32)
    dt = np.zeros(nv, np.float32)
    return dict(state=state, co=co.reshape(nt, -1), beta_raw=beta_raw, alpha_raw=alpha_raw, a=a, dt=dt)


# Qwen3.5 rope geometry (the reference's kparity push constants, src/vk/kparity.rs:33): 64 rotated
# dims per head, base 1e7, sections [11, 11, 10, 0].
ROPE_N_ROT, ROPE_BASE, ROPE_SECTIONS = 64, 1e7, (11, 11, 10, 0)


def rope_theta_scale(base: float, n_rot: int) -> float:
    """base^(-2/n_rot) rounded to f32 (the theta_scale the reference computes and pushes)."""
    return float(np.float32(np.float32(base) ** np.float32(-2.0 / n_rot)))


def prep_inputs(seed: int, nt: int, nh: int = 16, nkv: int = 2, hd: int = 256):
    """Attention pre-pass inputs (the q/k/v projections before norm and rope). Draw order:
    q+gate [nt, nh*2*hd] ~ N(0, 2^2); k [nt, nkv*hd] ~ N(0, 2^2); v [nt, nkv*hd] ~ N(0,1);
    q_norm, k_norm [hd] ~ 1 + N(0, 0.1^2)."""
    r = Rng(seed)
    q = r.normal(nt * nh * 2 * hd, std=2.0).reshape(nt, nh * 2 * hd)
    k = r.normal(nt * nkv * hd, std=2.0).reshape(nt, nkv * hd)
    v = r.normal(nt * nkv * hd).reshape(nt, nkv * hd)
    q_norm = (1.0 + r.normal(hd, std=0.1)).astype(np.float32)
    k_norm = (1.0 + r.normal(hd, std=0.1)).astype(np.float32)
    return dict(q=q, k=k, v=v, q_norm=q_norm, k_norm=k_norm)
