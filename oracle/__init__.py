"""TEST INFRASTRUCTURE ONLY: the CPU oracle of the attention / Gated-DeltaNet hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker (or the timed CPU baseline). The product path never routes through it.

- `cpu_ref.cpp` (built to liboracle.so by oracle/Makefile): restatement of the reference's CPU
  forward pass, src/cpu.rs:14-22, 145-164, 194-274, in f32 with the reference's loop order.
- `ref_np.py`: float64 references used to pin that restatement (the r012 known-answer softmax of
  src/vk/r012_parity.rs:22-28, a brute-force float64 gated-delta recurrence) and the numpy
  statement of the chunk-64 WY/UT scan (a new algorithm, pinned only by equality with the
  sequential recurrence).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_P = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_SIG = {
    "it_ref_hardware_threads": (_i, []),
    "it_ref_xorshift_fill": (None, [_P, ctypes.c_size_t, _P]),
    "it_ref_f32_to_f16_rne": (ctypes.c_uint16, [_f]),
    "it_ref_f16_to_f32": (_f, [ctypes.c_uint16]),
    "it_ref_rmsnorm": (None, [_P, _P, _i, _f, _P]),
    "it_ref_l2norm": (None, [_P, _i, _f]),
    "it_ref_gdn_gated_norm": (None, [_P, _P, _P, _i, _i, _i, _i, _f, _P]),
    "it_ref_rope_theta_scale": (_f, [_f, _i]),
    "it_ref_rope": (None, [_P, _i, _i, _i, _i, _f, _P]),
    "it_ref_attn_prep": (None, [_P, _i, _P, _i, _P, _P, _f, _P, _i, _i, _i, _i, _i, _i, _f, _P]),
    "it_ref_attn": (None, [_P, _i, _P, _P, _i, _i, _i, _i, _i, _i, _f, _P, _i, _i]),
    "it_ref_attn_f32kv": (None, [_P, _i, _P, _P, _i, _i, _i, _i, _i, _i, _f, _P, _i, _i]),
    "it_ref_gdn_conv": (None, [_P, _i, _P, _P, _P, _i, _i, _i, _i]),
    "it_ref_gdn_step": (None, [_P, _i, _P, _P, _i, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i]),
    "it_ref_gdn_layer": (None, [_P, _i, _P, _P, _i, _P, _P, _i, _P, _P, _P, _P, _i, _P, _i, _i, _i, _i, _f, _i]),
}
_lib = None


def build() -> None:
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIG.items():
            fn = getattr(h, n)
            fn.restype, fn.argtypes = r, a
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def kparity_draws(n_arena: int, n_params: int, seed: int = 0x9E3779B97F4A7C15):
    """The arena and params floats of the reference's kernel-parity harness (src/vk/kparity.rs:13,
    59-62): n_arena then n_params uniform [-1, 1) draws from one xorshift64 stream."""
    st = np.array([seed], np.uint64)
    a = np.empty(n_arena, np.float32)
    p = np.empty(n_params, np.float32)
    lib().it_ref_xorshift_fill(_p(st), n_arena, _p(a))
    lib().it_ref_xorshift_fill(_p(st), n_params, _p(p))
    return a, p


def hardware_threads() -> int:
    return lib().it_ref_hardware_threads()


def attn(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos0: int, nh: int, nkv: int, hd: int = 256,
         scale: float | None = None, threads: int = 0) -> np.ndarray:
    """cpu.rs:260-272 attention. q [nt, nh*2*hd] f32; kc/vc [>=pos0+nt, nkv*hd] uint16 f16 bits."""
    q = np.ascontiguousarray(q, np.float32).reshape(q.shape[0], -1)
    kc = np.ascontiguousarray(kc, np.uint16); vc = np.ascontiguousarray(vc, np.uint16)
    nt = q.shape[0]
    out = np.zeros((nt, nh * hd), np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    lib().it_ref_attn(_p(q), q.shape[1], _p(kc), _p(vc), nkv * hd, pos0, hd, nh, nkv, nt, scale, _p(out), nh * hd,
                      threads or hardware_threads())
    return out


def attn_f32kv(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos0: int, nh: int, nkv: int, hd: int = 256,
               scale: float | None = None, threads: int = 0) -> np.ndarray:
    """src/mtp.rs:122-130 attention over an f32 cache. q [nt, nh*2*hd]; kc/vc [>=pos0+nt, nkv*hd] f32."""
    q = np.ascontiguousarray(q, np.float32).reshape(q.shape[0], -1)
    kc = np.ascontiguousarray(kc, np.float32); vc = np.ascontiguousarray(vc, np.float32)
    nt = q.shape[0]
    out = np.zeros((nt, nh * hd), np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    lib().it_ref_attn_f32kv(_p(q), q.shape[1], _p(kc), _p(vc), nkv * hd, pos0, hd, nh, nkv, nt, scale, _p(out),
                            nh * hd, threads or hardware_threads())
    return out


def gdn_conv(x: np.ndarray, w: np.ndarray, state: np.ndarray):
    """cpu.rs:201-212 per token. Returns (out [nt, cd], new_state [K-1, cd])."""
    x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
    st = np.ascontiguousarray(state, np.float32).copy()
    nt, cd = x.shape
    out = np.zeros_like(x)
    lib().it_ref_gdn_conv(_p(x), cd, _p(w), _p(st), _p(out), cd, cd, nt, w.shape[1])
    return out, st


def l2norm_heads(x: np.ndarray, nheads: int, d: int, eps: float = 1e-6) -> np.ndarray:
    """cpu.rs:164/214 on the first nheads rows of d floats of every token row; returns a copy."""
    x = np.ascontiguousarray(x, np.float32).copy()
    for t in range(x.shape[0]):
        for h in range(nheads):
            row = np.ascontiguousarray(x[t, h * d:(h + 1) * d])
            lib().it_ref_l2norm(_p(row), d, eps)
            x[t, h * d:(h + 1) * d] = row
    return x


def gdn_step(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, threads: int = 0):
    """cpu.rs:216-232 token by token. state [nv,S,S] in the [h][i][j] layout. Returns (out, new_state)."""
    co = np.ascontiguousarray(co, np.float32)
    br = np.ascontiguousarray(beta_raw, np.float32); ar = np.ascontiguousarray(alpha_raw, np.float32)
    dt = np.ascontiguousarray(dt, np.float32); a = np.ascontiguousarray(a, np.float32)
    st = np.ascontiguousarray(state, np.float32).copy()
    nt = co.shape[0]; S = st.shape[-1]
    out = np.zeros((nt, nv * S), np.float32)
    lib().it_ref_gdn_step(_p(co), co.shape[1], _p(br), _p(ar), br.shape[1], _p(dt), _p(a), _p(st), _p(out), nv * S,
                          nt, nv, nk, S, threads or hardware_threads())
    return out, st


def _sections(sections) -> np.ndarray:
    s = np.zeros(4, np.int32)
    s[:len(sections)] = sections
    return s


def rope_theta_scale(base: float, n_rot: int) -> float:
    """cpu.rs:147: base^(-2/n_rot) in f32."""
    return float(lib().it_ref_rope_theta_scale(base, n_rot))


def rope(x: np.ndarray, pos: int, n_rot: int, base: float, sections=(0, 0, 0, 0)) -> np.ndarray:
    """cpu.rs:145-162 on every row of x [..., head_dim]; returns a copy."""
    y = np.ascontiguousarray(x, np.float32).copy()
    hd = y.shape[-1]
    lib().it_ref_rope(_p(y), y.size // hd, hd, n_rot, pos, base, _p(_sections(sections)))
    return y


def attn_prep(q: np.ndarray, k: np.ndarray, q_norm, k_norm, eps: float, pos0: int, nh: int, nkv: int, hd: int,
              n_rot: int, base: float, sections=(0, 0, 0, 0)):
    """cpu.rs:249-257 for nt tokens. q [nt, nh*2*hd], k [nt, nkv*hd] f32; q_norm/k_norm [hd] or None.
    Returns (q with its query halves normed and roped, k normed and roped), both f32."""
    q = np.ascontiguousarray(q, np.float32).reshape(q.shape[0], -1).copy()
    k = np.ascontiguousarray(k, np.float32).reshape(k.shape[0], -1)
    nt = q.shape[0]
    ko = np.zeros((nt, nkv * hd), np.float32)
    qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
    kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
    lib().it_ref_attn_prep(_p(q), q.shape[1], _p(k), k.shape[1], None if qn is None else _p(qn),
                           None if kn is None else _p(kn), eps, _p(ko), pos0, hd, nh, nkv, nt, n_rot, base,
                           _p(_sections(sections)))
    return q, ko


def gdn_gated_norm(o: np.ndarray, z: np.ndarray, w: np.ndarray, nv: int, eps: float = 1e-6) -> np.ndarray:
    """cpu.rs:234-238: per hv-wide head row, rmsnorm(o) * w * silu(z). o, z [nt, nv*hv]."""
    o = np.ascontiguousarray(o, np.float32); z = np.ascontiguousarray(z, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    nt = o.shape[0]; hv = w.shape[0]
    out = np.zeros_like(o)
    lib().it_ref_gdn_gated_norm(_p(o), _p(z), _p(w), nv, hv, nt, o.shape[1], eps, _p(out))
    return out
