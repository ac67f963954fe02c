"""Pins the GDN oracle (oracle/cpu_ref.cpp it_ref_gdn_*, restating src/cpu.rs:201-232) and the
float64 chunked WY/UT statement (oracle/ref_np.py), which has no reference counterpart."""
import numpy as np
import pytest

import oracle
from oracle.ref_np import gdn_chunked_f64, gdn_chunked_folded_f64, gdn_seq_f64
from irontimber_amd.synth import gdn_inputs, gdn_step_inputs


def small(seed=5, nt=6, nv=4, nk=2):
    return gdn_step_inputs(seed, nt, nv=nv, nk=nk)


def test_step_matches_float64_recurrence():
    d = small()
    out, st = oracle.gdn_step(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    o64, s64 = gdn_seq_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    np.testing.assert_allclose(out, o64, atol=2e-6)
    np.testing.assert_allclose(st, s64, atol=2e-6)


def test_step_qk_head_mapping_is_modulo():
    """V head h reads q/k head h % nk (cpu.rs:219), not h // (nv/nk): perturb k head 0 and check
    that exactly V heads 0 and 2 (nv=4, nk=2) change."""
    d = small()
    base, _ = oracle.gdn_step(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    co = d["co"].copy()
    co[:, 2 * 128:3 * 128] *= -1.0        # k head 0 (k block starts at nk*S = 256)
    pert, _ = oracle.gdn_step(co, d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    changed = [not np.allclose(base[:, h * 128:(h + 1) * 128], pert[:, h * 128:(h + 1) * 128]) for h in range(4)]
    assert changed == [True, False, True, False]


def test_step_beta_zero_only_decays():
    d = small(nt=1)
    br = np.full_like(d["beta_raw"], -200.0)       # sigmoid -> 0
    out, st = oracle.gdn_step(d["co"], br, d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    g = np.log1p(np.exp(d["alpha_raw"][0].astype(np.float64))) * d["a"]
    want = d["state"] * np.exp(g)[:, None, None]
    np.testing.assert_allclose(st, want, rtol=1e-6, atol=1e-9)
    q = d["co"][0, :128]  # kh = h % 2 -> q heads 0,1,0,1
    for h in range(4):
        qh = d["co"][0, (h % 2) * 128:(h % 2 + 1) * 128]
        np.testing.assert_allclose(out[0, h * 128:(h + 1) * 128], want[h].T @ qh / np.sqrt(128), atol=1e-6)
    del q


def test_step_full_decay_resets_to_outer_product():
    d = small(nt=1)
    ar = np.full_like(d["alpha_raw"], 200.0)       # softplus = 200, times a <= -0.37 -> e^g == 0
    out, st = oracle.gdn_step(d["co"], d["beta_raw"], ar, d["dt"], d["a"], d["state"], 4, 2)
    beta = 1 / (1 + np.exp(-d["beta_raw"][0].astype(np.float64)))
    for h in range(4):
        k = d["co"][0, 256 + (h % 2) * 128:256 + (h % 2 + 1) * 128].astype(np.float64)
        v = d["co"][0, 512 + h * 128:512 + (h + 1) * 128].astype(np.float64)
        np.testing.assert_allclose(st[h], beta[h] * np.outer(k, v), atol=1e-6)


def test_conv_multi_token_equals_single_calls():
    d = gdn_inputs(6, nt=9, nv=2, nk=1)
    out, st = oracle.gdn_conv(d["x"], d["w"], d["conv_state"])
    s = d["conv_state"].copy()
    for t in range(9):
        o1, s = oracle.gdn_conv(d["x"][t:t + 1], d["w"], s)
        np.testing.assert_array_equal(o1[0], out[t])
    np.testing.assert_array_equal(s, st)
    np.testing.assert_array_equal(st, d["x"][-3:])


def test_conv_closed_form():
    """silu(sum_i w_i x_{t-3+i}) in float64, with the carried state as x_{-3..-1}."""
    d = gdn_inputs(7, nt=5, nv=2, nk=1)
    out, _ = oracle.gdn_conv(d["x"], d["w"], d["conv_state"])
    xs = np.concatenate([d["conv_state"], d["x"]]).astype(np.float64)
    pre = sum(xs[i:i + 5] * d["w"][:, i].astype(np.float64) for i in range(4))
    np.testing.assert_allclose(out, pre / (1 + np.exp(-pre)), rtol=1e-5, atol=1e-6)


def test_l2norm_unit_rows():
    x = np.random.default_rng(1).standard_normal((3, 512)).astype(np.float32)
    y = oracle.l2norm_heads(x, 4, 128)
    np.testing.assert_allclose(np.linalg.norm(y.reshape(3, 4, 128), axis=-1), 1.0, rtol=1e-6)


@pytest.mark.parametrize("nt,C", [(1, 64), (64, 64), (100, 64), (130, 16), (37, 8)])
def test_chunked_f64_equals_sequential(nt, C):
    d = gdn_step_inputs(8, nt, nv=4, nk=2)
    o1, s1 = gdn_seq_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    o2, s2 = gdn_chunked_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2, C=C)
    np.testing.assert_allclose(o2, o1, atol=1e-10)
    np.testing.assert_allclose(s2, s1, atol=1e-10)



@pytest.mark.parametrize("nt,C", [(1, 64), (64, 64), (100, 64), (130, 16), (37, 32)])
def test_chunked_folded_f64_equals_sequential(nt, C):
    """The regrouping the GPU chunk kernels compute (Kh and P by a blocked backward solve, Y from
    the raw V and K rows) equals the token-sequential recurrence, partial last chunks included."""
    d = gdn_step_inputs(9, nt, nv=4, nk=2)
    o1, s1 = gdn_seq_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    o2, s2 = gdn_chunked_folded_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2, C=C)
    np.testing.assert_allclose(o2, o1, atol=1e-10)
    np.testing.assert_allclose(s2, s1, atol=1e-10)


def test_chunked_folded_f64_strong_decay_zero_beta():
    """Near-total decay and beta ~ 0 on some tokens: the fold has no division by a decay or beta."""
    d = gdn_step_inputs(10, 150, nv=4, nk=2)
    d["alpha_raw"][10:20] = 30.0
    d["beta_raw"][40:60] = -60.0
    o1, s1 = gdn_seq_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    o2, s2 = gdn_chunked_folded_f64(d["co"], d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], 4, 2)
    np.testing.assert_allclose(o2, o1, atol=1e-9)
    np.testing.assert_allclose(s2, s1, atol=1e-9)

def test_layer_matches_pieces():
    """conv -> L2 -> recurrence, one token at a time (cpu.rs:201-232)."""
    nv, nk, S, nt = 4, 2, 128, 3
    d = gdn_inputs(9, nt=nt, nv=nv, nk=nk)
    co, _ = oracle.gdn_conv(d["x"], d["w"], d["conv_state"])
    co = oracle.l2norm_heads(co, 2 * nk, S)
    o1, s1 = oracle.gdn_step(co, d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], nv, nk)
    o64, s64 = gdn_seq_f64(co, d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], nv, nk)
    np.testing.assert_allclose(o1, o64, atol=2e-6)
    np.testing.assert_allclose(s1, s64, atol=2e-6)


def test_gated_norm_closed_forms():
    """cpu.rs:234-238 gated RMSNorm: z = 0 gives 0; large z gives rmsnorm(o)*w*z; a constant row c
    gives c/sqrt(c^2+eps)*w*silu(z); random rows against a float64 statement."""
    rng = np.random.default_rng(5)
    nv, hv, nt = 4, 128, 3
    o = rng.standard_normal((nt, nv * hv)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(hv)).astype(np.float32)
    np.testing.assert_array_equal(oracle.gdn_gated_norm(o, np.zeros_like(o), w, nv), np.zeros_like(o))
    big = np.full_like(o, 40.0)
    o64 = o.reshape(nt, nv, hv).astype(np.float64)
    rn = o64 / np.sqrt((o64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(oracle.gdn_gated_norm(o, big, w, nv).reshape(nt, nv, hv), rn * 40.0, rtol=2e-6, atol=1e-6)
    c = np.full_like(o, -2.5)
    z = rng.standard_normal(o.shape).astype(np.float32)
    silu = z / (1 + np.exp(-z.astype(np.float64)))
    want = (-2.5 / np.sqrt(6.25 + 1e-6)) * np.tile(w, nv)[None, :] * silu
    np.testing.assert_allclose(oracle.gdn_gated_norm(c, z, w, nv), want, rtol=2e-6, atol=1e-7)
    want = (rn * silu.reshape(nt, nv, hv)).reshape(nt, -1)
    np.testing.assert_allclose(oracle.gdn_gated_norm(o, z, w, nv), want, rtol=1e-5, atol=1e-6)


def _conv_l2_f64(x, w, state, nnorm, S=128, eps=1e-6):
    """cpu.rs:201-214 in float64, written independently: per token the K-tap window (the K-1 state
    rows oldest first, then x_t) times w[ch, :], SiLU, state shift; then each of the first nnorm
    S-wide heads divided by max(||row||, eps)."""
    x = x.astype(np.float64); w = w.astype(np.float64); st = state.astype(np.float64).copy()
    nt, cd = x.shape
    out = np.zeros((nt, cd))
    for t in range(nt):
        win = np.vstack([st, x[t:t + 1]])                  # [K, cd]
        y = (win.T * w).sum(axis=1)
        y = y / (1.0 + np.exp(-y))
        for h in range(nnorm):
            r = y[h * S:(h + 1) * S]
            y[h * S:(h + 1) * S] = r / max(np.sqrt((r * r).sum()), eps)
        out[t] = y
        st = np.vstack([st[1:], x[t:t + 1]])
    return out, st


def test_ref_gdn_layer_direct_strided():
    """it_ref_gdn_layer itself (the oracle of every GPU GDN-layer test) at nt > 1 with padded token
    strides: equal bit for bit to its pieces (conv -> l2norm -> step) called separately, and within
    f32 rounding of an independent float64 statement (conv + L2 above, then gdn_seq_f64)."""
    nt, nv, nk, S, K = 7, 4, 2, 128, 4
    d = gdn_inputs(9, nt=nt, nv=nv, nk=nk)
    cd = d["cd"]
    xs, bs, os_ = cd + 64, nv + 3, nv * S + 32           # padded token strides
    xbuf = np.full((nt, xs), np.nan, np.float32); xbuf[:, :cd] = d["x"]
    bbuf = np.full((nt, bs), np.nan, np.float32); bbuf[:, :nv] = d["beta_raw"]
    abuf = np.full((nt, bs), np.nan, np.float32); abuf[:, :nv] = d["alpha_raw"]
    obuf = np.full((nt, os_), 7.0, np.float32)
    co = np.zeros((nt, cd), np.float32)
    cst, sst = d["conv_state"].copy(), d["state"].copy()
    P = lambda a: a.ctypes.data
    oracle.lib().it_ref_gdn_layer(P(xbuf), xs, P(d["w"]), P(cst), K, P(bbuf), P(abuf), bs, P(d["dt"]), P(d["a"]),
                                  P(sst), P(obuf), os_, P(co), nt, nv, nk, S, 1e-6, 4)
    assert np.all(obuf[:, nv * S:] == 7.0)               # nothing written into the stride padding
    out = obuf[:, :nv * S]
    # the pieces, each called on its own
    co2, cst2 = oracle.gdn_conv(d["x"], d["w"], d["conv_state"])
    co2 = oracle.l2norm_heads(co2, 2 * nk, S)
    out2, sst2 = oracle.gdn_step(co2, d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], nv, nk)
    np.testing.assert_array_equal(co, co2)
    np.testing.assert_array_equal(cst, cst2)
    np.testing.assert_array_equal(out, out2)
    np.testing.assert_array_equal(sst, sst2)
    # independent float64 truth
    co64, st64 = _conv_l2_f64(d["x"], d["w"], d["conv_state"], 2 * nk)
    np.testing.assert_allclose(co, co64, atol=2e-6)
    np.testing.assert_allclose(cst, st64, atol=0)
    o64, s64 = gdn_seq_f64(co64.astype(np.float32), d["beta_raw"], d["alpha_raw"], d["dt"], d["a"], d["state"], nv, nk)
    np.testing.assert_allclose(out, o64, atol=2e-5)
    np.testing.assert_allclose(sst, s64, atol=2e-5)


def test_conv_oracle_kparity_inputs():
    """The oracle conv on the reference's kernel-parity conv inputs (kparity.rs:32, cd 1000, 5 tokens,
    K 4) against the float64 statement: outputs within f32 rounding, the state exactly the last
    three input rows."""
    MB = 1 << 20
    arena, params = oracle.kparity_draws(5 << 20, 1 << 16)
    params = params.copy()
    params[16:20] = -np.abs(params[16:20]) - 0.1     # set before every case (kparity.rs:63)
    cd, nt, K = 1000, 5, 4
    x = arena[:nt * cd].reshape(nt, cd)
    w = params[:cd * K].reshape(cd, K)
    st0 = arena[2 * MB:2 * MB + (K - 1) * cd].reshape(K - 1, cd)
    out, st = oracle.gdn_conv(x, w, st0)
    o64, s64 = _conv_l2_f64(x, w, st0, nnorm=0)
    np.testing.assert_allclose(out, o64, atol=1e-6)
    np.testing.assert_array_equal(st, x[-3:])
    np.testing.assert_array_equal(s64.astype(np.float32), x[-3:])


def test_oracle_gdn_kparity_inputs():
    """The oracle recurrence on the reference's kernel-parity gdn inputs (kparity.rs:35, unnormalised
    q/k) against the float64 recurrence, relative to max(1, |x|) as the harness measures."""
    MB = 1 << 20
    a, p = oracle.kparity_draws(5 << 20, 1 << 16)
    p = p.copy()
    p[16:20] = -np.abs(p[16:20]) - 0.1
    co = a[:6 * 1024].reshape(6, 1024)
    br, ar = a[MB:MB + 24].reshape(6, 4), a[MB + 64:MB + 88].reshape(6, 4)
    st = a[2 * MB:2 * MB + 4 * 128 * 128].reshape(4, 128, 128)
    out, sn = oracle.gdn_step(co, br, ar, p[0:4], p[16:20], st, 4, 2)
    o64, s64 = gdn_seq_f64(co, br, ar, p[0:4], p[16:20], st, 4, 2)
    rel = lambda x, y: np.max(np.abs(x - y) / np.maximum(1.0, np.abs(y)))
    assert rel(out, o64) <= 1e-4 and rel(sn, s64) <= 1e-4
