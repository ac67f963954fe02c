"""TEST INFRASTRUCTURE ONLY: float64 references that pin the oracle (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np


def f16_to_f64(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def attn_f64(q: np.ndarray, kf: np.ndarray, vf: np.ndarray, pos0: int, nh: int, nkv: int, hd: int,
             scale: float) -> np.ndarray:
    """Softmax attention with sigmoid gate in float64, the known-answer oracle of
    src/vk/r012_parity.rs:22-27. q [nt, nh*2*hd]; kf/vf [>= pos0+nt, nkv*hd] float64 key/value
    values (already f16-rounded as the cache holds them). Token t sees n = pos0+t+1 keys."""
    nt = q.shape[0]
    q = q.reshape(nt, nh, 2 * hd).astype(np.float64)
    g = nh // nkv
    out = np.zeros((nt, nh, hd))
    for t in range(nt):
        n = pos0 + t + 1
        for kh in range(nkv):
            K = kf[:n, kh * hd:(kh + 1) * hd]
            V = vf[:n, kh * hd:(kh + 1) * hd]
            qs = q[t, kh * g:(kh + 1) * g, :hd]
            s = qs @ K.T * scale
            s -= s.max(axis=1, keepdims=True)
            e = np.exp(s)
            o = (e @ V) / e.sum(axis=1, keepdims=True)
            gate = q[t, kh * g:(kh + 1) * g, hd:]
            out[t, kh * g:(kh + 1) * g] = o / (1.0 + np.exp(-gate))
    return out.reshape(nt, nh * hd)


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gdn_decay_beta(beta_raw, alpha_raw, dt, a):
    """beta = sigmoid(b), g = softplus(alpha + dt) * a (cpu.rs:222), float64 [nt, nv]."""
    beta = 1.0 / (1.0 + np.exp(-np.asarray(beta_raw, np.float64)))
    g = _softplus(np.asarray(alpha_raw, np.float64) + np.asarray(dt, np.float64)) * np.asarray(a, np.float64)
    return beta, g


def gdn_seq_f64(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int):
    """Brute-force float64 gated-delta recurrence, written from the update rule itself:
    S <- e^g S;  S <- S + beta k (v - S^T k)^T;  o = S^T q / sqrt(S).
    state [nv, S, S] indexed [h][i = key][j = value]. Returns (out [nt, nv*S], state)."""
    co = np.asarray(co, np.float64)
    st = np.asarray(state, np.float64).copy()
    nt = co.shape[0]
    S = st.shape[-1]
    qk = nk * S
    beta, g = gdn_decay_beta(beta_raw, alpha_raw, dt, a)
    out = np.zeros((nt, nv, S))
    for t in range(nt):
        for h in range(nv):
            kh = h % nk
            q = co[t, kh * S:(kh + 1) * S]
            k = co[t, qk + kh * S:qk + (kh + 1) * S]
            v = co[t, 2 * qk + h * S:2 * qk + (h + 1) * S]
            M = st[h] * np.exp(g[t, h])
            M = M + beta[t, h] * np.outer(k, v - M.T @ k)
            st[h] = M
            out[t, h] = M.T @ q / np.sqrt(S)
    return out.reshape(nt, nv * S), st


def gdn_chunked_f64(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, C: int = 64):
    """Chunked (WY/UT) form of the same recurrence in float64. Per chunk of L <= C tokens with
    in-chunk cumulative log-decay G (inclusive), D[t,s] = exp(G_t - G_s):
        A  = strict_lower(D * K K^T)             T = (I + diag(beta) A)^-1 diag(beta)
        W  = T diag(e^G) K                       U = T V - W S0
        O  = (diag(e^G) Q S0 + lower_incl(D * Q K^T) U) / sqrt(S)
        S1 = e^{G_L} S0 + (diag(e^{G_L - G}) K)^T U
    Only decay differences G_t - G_s <= 0 (t >= s) are exponentiated, so nothing overflows."""
    co = np.asarray(co, np.float64)
    st = np.asarray(state, np.float64).copy()
    nt = co.shape[0]
    S = st.shape[-1]
    qk = nk * S
    beta, g = gdn_decay_beta(beta_raw, alpha_raw, dt, a)
    out = np.zeros((nt, nv, S))
    for h in range(nv):
        kh = h % nk
        Qa = co[:, kh * S:(kh + 1) * S]
        Ka = co[:, qk + kh * S:qk + (kh + 1) * S]
        Va = co[:, 2 * qk + h * S:2 * qk + (h + 1) * S]
        S0 = st[h]
        for c0 in range(0, nt, C):
            c1 = min(nt, c0 + C)
            Q, K, V = Qa[c0:c1], Ka[c0:c1], Va[c0:c1]
            b = beta[c0:c1, h]
            G = np.cumsum(g[c0:c1, h])
            D = np.exp(np.minimum(G[:, None] - G[None, :], 0.0))
            L = c1 - c0
            A = np.tril(D * (K @ K.T), -1)
            Minv = np.linalg.inv(np.eye(L) + b[:, None] * A)
            T = Minv * b[None, :]
            W = T @ (np.exp(G)[:, None] * K)
            U = T @ V - W @ S0
            O = np.exp(G)[:, None] * (Q @ S0) + np.tril(D * (Q @ K.T)) @ U
            out[c0:c1, h] = O / np.sqrt(S)
            S0 = np.exp(G[-1]) * S0 + (np.exp(G[-1] - G)[:, None] * K).T @ U
        st[h] = S0
    return out.reshape(nt, nv * S), st



def gdn_chunked_folded_f64(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, C: int = 64):
    """The regrouping the GPU chunk kernels compute (no reference counterpart), in float64 and
    chunk length C (a multiple of 16), the chunk padded with beta = 0, g = 0. With
    M = (I + diag(beta) A)^-1 diag(beta) (A as in gdn_chunked_f64):
        Y  = V - diag(e^G) K S0                      (so U above = M Y)
        Kh = M^T diag(e^{G_L - G}) K                 P = lower_incl(D * Q K^T) M
        O  = (diag(e^G) Q S0 + P Y) / sqrt(S)        S1 = e^{G_L} S0 + Kh^T Y
    Kh and P^T come from one backward substitution (I + diag(beta) A)^T Z = [diag(e^{G_L - G}) K |
    lower_incl(D * Q K^T)^T] blocked by 16 rows (the last block first), rows then scaled by beta:
    the steps of the GPU chunk prep."""
    co = np.asarray(co, np.float64)
    st = np.asarray(state, np.float64).copy()
    nt = co.shape[0]
    S = st.shape[-1]
    qk = nk * S
    beta, g = gdn_decay_beta(beta_raw, alpha_raw, dt, a)
    out = np.zeros((nt, nv, S))
    nb = C // 16
    for h in range(nv):
        kh = h % nk
        S0 = st[h]
        for c0 in range(0, nt, C):
            L = min(nt, c0 + C) - c0
            pad = lambda m: np.pad(m, ((0, C - L),) + ((0, 0),) * (m.ndim - 1))
            Q = pad(co[c0:c0 + L, kh * S:(kh + 1) * S])
            K = pad(co[c0:c0 + L, qk + kh * S:qk + (kh + 1) * S])
            V = pad(co[c0:c0 + L, 2 * qk + h * S:2 * qk + (h + 1) * S])
            b = pad(beta[c0:c0 + L, h])
            G = np.cumsum(pad(g[c0:c0 + L, h]))
            D = np.exp(np.minimum(G[:, None] - G[None, :], 0.0))
            Ap = np.tril(b[:, None] * (D * (K @ K.T)), -1)
            Aqk = np.tril(D * (Q @ K.T))
            R = np.concatenate([np.exp(G[-1] - G)[:, None] * K, Aqk.T], axis=1)
            Z = np.zeros_like(R)
            for i in range(nb - 1, -1, -1):
                bi = slice(16 * i, 16 * i + 16)
                acc = R[bi].copy()
                for k in range(i + 1, nb):
                    bk = slice(16 * k, 16 * k + 16)
                    acc -= Ap[bk, bi].T @ Z[bk]
                Ti = np.linalg.inv(np.eye(16) + Ap[bi, bi])
                Z[bi] = Ti.T @ acc
            Kh = b[:, None] * Z[:, :S]
            P = (b[:, None] * Z[:, S:]).T
            Y = V - np.exp(G)[:, None] * (K @ S0)
            O = np.exp(G)[:, None] * (Q @ S0) + P @ Y
            out[c0:c0 + L, h] = O[:L] / np.sqrt(S)
            S0 = np.exp(G[-1]) * S0 + Kh.T @ Y
        st[h] = S0
    return out.reshape(nt, nv * S), st

def rope_f64(x: np.ndarray, pos: int, n_rot: int, theta_scale: float, sections=(0, 0, 0, 0)) -> np.ndarray:
    """Neox-style (I)MRoPE in float64 with exact angles pos * theta_scale**i (theta_scale the f32
    value, cpu.rs:147), the sector rule of cpu.rs:152-155; x [..., head_dim] -> float64 copy.
    Differs from cpu.rs:145-162 only by that function's f32 angle recurrence."""
    y = np.array(x, np.float64)
    half = n_rot // 2
    s0, s1, s2, s3 = (list(sections) + [0, 0, 0, 0])[:4]
    sect = s0 + s1 + s2 + s3
    i = np.arange(half)
    sector = i % sect if sect > 0 else np.zeros_like(i)
    keep = ((sector % 3 == 1) & (sector < 3 * s1)) | ((sector % 3 == 2) & (sector < 3 * s2)) | \
           ((sector % 3 == 0) & (sector < 3 * s0))
    use_e = (sect > 0) & ~keep
    th = np.where(use_e, 0.0, float(pos) * np.float64(theta_scale) ** i)
    c, s = np.cos(th), np.sin(th)
    x0, x1 = y[..., :half].copy(), y[..., half:n_rot].copy()
    y[..., :half] = x0 * c - x1 * s
    y[..., half:n_rot] = x0 * s + x1 * c
    return y


def rmsnorm_f64(x: np.ndarray, w=None, eps: float = 1e-6) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * w over the last axis, float64 (cpu.rs:14-18)."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return y if w is None else y * np.asarray(w, np.float64)
