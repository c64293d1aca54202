"""The prefill oracle (token-sequential recurrence, float64) on the CPU.

Pinned by: single tokens against the C delta_step/prepare restatement (itself
pinned to core.py:5-15 and kernels/fused.py:155-179); the closed-form chunked
(WY) form of the same recurrence, written here independently; the prefix
property of checkpoints; sequence boundaries.
"""
import numpy as np
import torch
import pytest

from oracle import oracle as O


def _inputs(rng, T, H, HK, K, V):
    q = rng.standard_normal((T, HK, K))
    k = rng.standard_normal((T, HK, K))
    v = rng.standard_normal((T, H, V))
    g = -np.log1p(np.exp(rng.standard_normal((T, H))))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((T, H))))
    return q, k, v, g, beta


@pytest.mark.parametrize("raw", [False, True])
def test_single_token_equals_delta_step(raw):
    rng = np.random.default_rng(0)
    H, HK, K, V, B = 4, 2, 16, 8, 3
    q, k, v, g, beta = (x.astype(np.float32) for x in _inputs(rng, B, H, HK, K, V))
    state = (rng.standard_normal((B, H, K, V)) * .3).astype(np.float32)
    a_log = rng.standard_normal(H).astype(np.float32) if raw else None
    dt_bias = rng.standard_normal(H).astype(np.float32) if raw else None
    cu = np.arange(B + 1)
    out, _, final = O.prefill(q, k, v, g, beta, state, cu, normalize=True, scale=K ** -.5,
                              a_log=a_log, dt_bias=dt_bias)
    qp, kp, ld, bo = O.prepare(q.reshape(B, -1), k.reshape(B, -1), g, beta, H, K, False, True, K ** -.5,
                               a_log, dt_bias)
    ref_out, ref_state = O.delta_step(state, qp, kp, v, ld, bo)
    np.testing.assert_allclose(out, ref_out, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(final, ref_state, rtol=2e-5, atol=2e-6)


def _chunked(q, k, v, g, beta, S, C):
    """Closed-form chunk (WY/UT) recurrence for one sequence, heads batched.

    With Gamma_t = prod_{s<=t} g_s inside a chunk and A_ts = beta_t
    (Gamma_t/Gamma_s) k_t.k_s (s < t): Delta = (I + A)^{-1} beta (V - Gamma K S0),
    O = Gamma Q S0 + (M o Q K^T) Delta with M_ts = Gamma_t/Gamma_s (s <= t),
    S_C = Gamma_C S0 + (K Gamma_C / Gamma)^T Delta.
    """
    T = q.shape[0]
    out = np.zeros((T,) + v.shape[1:])
    for c0 in range(0, T, C):
        sl = slice(c0, min(c0 + C, T))
        Q, Kc, Vc = q[sl].transpose(1, 0, 2), k[sl].transpose(1, 0, 2), v[sl].transpose(1, 0, 2)
        lg = np.cumsum(g[sl].T, axis=1)  # [H, n]
        n = lg.shape[1]
        ratio = np.exp(lg[:, :, None] - lg[:, None, :])
        kk = np.einsum("htd,hsd->hts", Kc, Kc)
        A = np.tril(beta[sl].T[:, :, None] * ratio * kk, -1)
        Tm = np.linalg.inv(np.eye(n)[None] + A)
        R = beta[sl].T[:, :, None] * (Vc - np.exp(lg)[:, :, None] * np.einsum("htd,hdv->htv", Kc, S))
        D = Tm @ R
        qk = np.einsum("htd,hsd->hts", Q, Kc)
        O_ = np.exp(lg)[:, :, None] * np.einsum("htd,hdv->htv", Q, S) + (np.tril(ratio * qk)) @ D
        out[sl] = O_.transpose(1, 0, 2)
        S = np.exp(lg[:, -1])[:, None, None] * S + np.einsum(
            "htd,htv->hdv", Kc * np.exp(lg[:, -1:] - lg)[:, :, None], D)
    return out, S


@pytest.mark.parametrize("C", [1, 4, 8, 16])
def test_chunked_closed_form_equals_sequential(C):
    rng = np.random.default_rng(C)
    H, K, V, T = 3, 8, 6, 29
    q, k, v, g, beta = _inputs(rng, T, H, H, K, V)
    S0 = rng.standard_normal((1, H, K, V))
    out, _, final = O.prefill(q, k, v, g, beta, S0, np.array([0, T]))
    o2, s2 = _chunked(q, k, v, g, beta, S0[0], C)
    np.testing.assert_allclose(out, o2, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(final[0], s2, rtol=1e-9, atol=1e-10)


def test_checkpoints_are_prefix_states_and_sequences_are_independent():
    rng = np.random.default_rng(5)
    H, HK, K, V = 4, 2, 8, 4
    lens = [13, 0, 7]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = cu[-1]
    q, k, v, g, beta = _inputs(rng, T, H, HK, K, V)
    S0 = rng.standard_normal((3, H, K, V))
    ck = np.array([[5, 13, 0], [1, 0, 0], [7, 3, 9]])
    out, states, final = O.prefill(q, k, v, g, beta, S0, cu, ck, normalize=True, scale=.5)
    np.testing.assert_array_equal(final[1], S0[1])          # empty sequence keeps its state
    assert not states[1].any() and not states[2, 2].any()   # unused / out-of-range checkpoints
    for b, c in [(0, 0), (0, 1), (2, 0), (2, 1)]:
        n = ck[b, c]
        s0 = cu[b]
        _, _, f = O.prefill(q[s0:s0 + n], k[s0:s0 + n], v[s0:s0 + n], g[s0:s0 + n], beta[s0:s0 + n],
                            S0[b:b + 1], np.array([0, n]), normalize=True, scale=.5)
        np.testing.assert_allclose(states[b, c], f[0], rtol=1e-12, atol=1e-12)
    # sequence 2 alone gives the same outputs as inside the batch
    o2, _, _ = O.prefill(q[13:], k[13:], v[13:], g[13:], beta[13:], S0[2:], np.array([0, 7]),
                         normalize=True, scale=.5)
    np.testing.assert_allclose(out[13:], o2, rtol=1e-12, atol=1e-12)


def test_no_write_strength_only_decays():
    rng = np.random.default_rng(2)
    H, K, V, T = 2, 4, 3, 6
    q, k, v, g, beta = _inputs(rng, T, H, H, K, V)
    S0 = rng.standard_normal((1, H, K, V))
    _, _, final = O.prefill(q, k, v, g, np.zeros_like(beta), S0, np.array([0, T]))
    np.testing.assert_allclose(final[0], S0[0] * np.exp(g.sum(0))[:, None, None], rtol=1e-12)


def _kda_gates(rng, T, H, K):
    return -np.log1p(np.exp(rng.standard_normal((T, H, K)) * .5))


@pytest.mark.parametrize("raw", [False, True])
def test_kda_single_token_equals_delta_step(raw):
    """Per-channel decay: one token of the prefill is core.py:5-15 with the
    KDA log decay [B, H, K] (each key row of the state decays on its own)."""
    rng = np.random.default_rng(3)
    H, HK, K, V, B = 4, 4, 16, 8, 3
    q, k, v, _, beta = (x.astype(np.float32) for x in _inputs(rng, B, H, HK, K, V))
    g = _kda_gates(rng, B, H, K).astype(np.float32)
    state = (rng.standard_normal((B, H, K, V)) * .3).astype(np.float32)
    a_log = rng.standard_normal(H).astype(np.float32) if raw else None
    dt_bias = rng.standard_normal(H * K).astype(np.float32) if raw else None
    cu = np.arange(B + 1)
    out, _, final = O.prefill(q, k, v, g, beta, state, cu, normalize=True, scale=K ** -.5,
                              a_log=a_log, dt_bias=dt_bias)
    qp, kp, ld, bo = O.prepare(q.reshape(B, -1), k.reshape(B, -1), g.reshape(B, -1), beta, H, K, True, True,
                               K ** -.5, a_log, dt_bias)
    assert ld.shape == (B, H, K)
    ref_out, ref_state = O.delta_step(state, qp, kp, v, ld, bo)
    np.testing.assert_allclose(out, ref_out, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(final, ref_state, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("kda", [False, True])
def test_raw_gate_with_post_sigmoid_beta(kda):
    """The chunk kernels' KDA convention (raw gate with A_log/dt_bias, beta
    already through the sigmoid): the same recurrence as the log decay
    -exp(A_log) softplus(g + dt_bias), computed here with torch, and beta
    taken as given; with beta_logits the sigmoid is applied."""
    rng = np.random.default_rng(8)
    H, HK, K, V, T = 2, 2, 8, 4, 9
    q, k, v, _, beta = (x.astype(np.float32) for x in _inputs(rng, T, H, HK, K, V))
    gshape = (T, H, K) if kda else (T, H)
    raw = rng.standard_normal(gshape).astype(np.float32)
    a_log = (rng.standard_normal(H) * .5).astype(np.float32)
    dt_bias = (rng.standard_normal(H * K if kda else H) * .5).astype(np.float32)
    S0 = (rng.standard_normal((1, H, K, V)) * .3).astype(np.float32)
    cu = np.array([0, T])
    bias = torch.from_numpy(dt_bias).double().reshape((H, K) if kda else (H,))
    rate = torch.from_numpy(a_log).double().exp().reshape((H, 1) if kda else (H,))
    logd = (-rate * torch.nn.functional.softplus(torch.from_numpy(raw).double() + bias)).numpy()
    want = O.prefill(q, k, v, logd, beta, S0, cu, normalize=True, scale=.3)
    got = O.prefill(q, k, v, raw, beta, S0, cu, normalize=True, scale=.3, a_log=a_log, dt_bias=dt_bias,
                    beta_logits=False)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    b64 = beta.astype(np.float64)
    logits = np.log(b64 / (1 - b64))
    again = O.prefill(q, k, v, raw, logits, S0, cu, normalize=True, scale=.3, a_log=a_log, dt_bias=dt_bias)
    for a, b in zip(again, want):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-9)


def _kda_chunk_closed_form(q, k, v, g, beta, S0):
    """One chunk of the KDA recurrence in closed (WY) form, written from the
    algebra, not from the oracle: with G_t = sum_{s<=t} g_s per channel,
    A_ts = beta_t sum_i k_ti k_si e^{G_ti - G_si} (s < t), T = (I + A)^-1,
    Delta = T beta (V - (K o e^G) S0), S_C = e^{G_C} o S0 + (K o e^{G_C - G})^T Delta,
    O = (Q o e^G) S0 + (M o (Q o e^G)(K o e^-G)^T) Delta, M causal incl. the diagonal.
    q, k: [C, K]; v: [C, V]; g: [C, K]; beta: [C]; S0: [K, V]."""
    C = q.shape[0]
    G = np.cumsum(g, 0)
    A = np.zeros((C, C))
    for t in range(C):
        for s in range(t):
            A[t, s] = beta[t] * np.sum(k[t] * k[s] * np.exp(G[t] - G[s]))
    Tm = np.linalg.inv(np.eye(C) + A)
    delta = Tm @ (beta[:, None] * (v - (k * np.exp(G)) @ S0))
    SC = np.exp(G[-1])[:, None] * S0 + (k * np.exp(G[-1] - G)).T @ delta
    P = np.zeros((C, C))
    for t in range(C):
        for s in range(t + 1):
            P[t, s] = np.sum(q[t] * k[s] * np.exp(G[t] - G[s]))
    out = (q * np.exp(G)) @ S0 + P @ delta
    return out, SC


@pytest.mark.parametrize("C", [1, 5, 16])
def test_kda_prefill_equals_closed_form_chunk(C):
    rng = np.random.default_rng(C)
    H, HK, K, V = 2, 2, 8, 6
    q, k, v, _, beta = _inputs(rng, C, H, HK, K, V)
    g = _kda_gates(rng, C, H, K)
    S0 = rng.standard_normal((1, H, K, V)) * .3
    out, _, final = O.prefill(q, k, v, g, beta, S0, np.array([0, C]))
    for h in range(H):
        ref_out, ref_S = _kda_chunk_closed_form(q[:, h], k[:, h], v[:, h], g[:, h], beta[:, h], S0[0, h])
        np.testing.assert_allclose(out[:, h], ref_out, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(final[0, h], ref_S, rtol=1e-10, atol=1e-12)


def test_kda_checkpoint_is_the_prefix_state():
    rng = np.random.default_rng(11)
    H, HK, K, V, T = 2, 1, 8, 4, 40
    q, k, v, _, beta = _inputs(rng, T, H, HK, K, V)
    g = _kda_gates(rng, T, H, K)
    S0 = rng.standard_normal((1, H, K, V)) * .2
    out, states, final = O.prefill(q, k, v, g, beta, S0, np.array([0, T]), checkpoints=np.array([[17, T]]))
    o1, _, mid = O.prefill(q[:17], k[:17], v[:17], g[:17], beta[:17], S0, np.array([0, 17]))
    o2, _, end = O.prefill(q[17:], k[17:], v[17:], g[17:], beta[17:], mid, np.array([0, T - 17]))
    np.testing.assert_allclose(states[0, 0], mid[0], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(states[0, 1], final[0], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(end, final, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(np.concatenate([o1, o2]), out, rtol=1e-12, atol=1e-14)
