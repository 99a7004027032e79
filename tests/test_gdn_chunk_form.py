"""The chunk-parallel form of the Gated DeltaNet recurrence equals the serial
recurrence (CPU, float64).

hipllm_gdn_scan_chunked evaluates the scan of metal_gdn_recurrence_f32
(metal_llm.metal:1370-1420) in 64-token chunks: per chunk, with G_t the
cumulative log decay, T = (I + A)^-1 for A[t][i] = beta_t e^(G_t - G_i)
k_t . k_i (i < t), Delta = T (beta (V - e^G K S0)), outputs
(e^G Q S0 + (e^(G_t - G_i) q_t . k_i)_{i <= t} Delta) / sqrt(D), and the
state e^(G_last) S0 + K^T (e^(G_last - G) Delta). This restates that
algebra in numpy, with the kernels' padding of a partial last chunk (zero
keys, beta 0, decay 1), and checks it against the oracle's serial step
(oracle/moe_ref.py gdn_step) on several lengths, ragged ones included, with
a nonzero starting state; a dropped decay factor or a wrong triangle fails.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_ref

C = 64


def chunked(S, q, k, v, decay, beta, key_heads):
    """Float64 chunked scan. S [Hv, D, D]; q, k [T, Hk, D]; v [T, Hv, D];
    decay, beta [T, Hv]. Returns (S, o [T, Hv, D])."""
    T, Hv, D = v.shape
    S = S.copy()
    o = np.zeros((T, Hv, D))
    for h in range(Hv):
        kh = h % key_heads
        for t0 in range(0, T, C):
            n = min(C, T - t0)
            K = np.zeros((C, D)); Q = np.zeros((C, D)); V = np.zeros((C, D))
            g = np.zeros(C); b = np.zeros(C)
            K[:n], Q[:n], V[:n] = k[t0:t0 + n, kh], q[t0:t0 + n, kh], v[t0:t0 + n, h]
            g[:n], b[:n] = np.log(decay[t0:t0 + n, h]), beta[t0:t0 + n, h]
            G = np.cumsum(g)
            dec = np.exp(G[:, None] - G[None, :])
            A = np.tril(b[:, None] * dec * (K @ K.T), -1)
            Tm = np.linalg.inv(np.eye(C) + A)
            P = np.tril(dec * (Q @ K.T))
            R = b[:, None] * (V - np.exp(G)[:, None] * (K @ S[h]))
            Dl = Tm @ R
            out = (np.exp(G)[:, None] * (Q @ S[h]) + P @ Dl) / np.sqrt(D)
            o[t0:t0 + n, h] = out[:n]
            S[h] = np.exp(G[-1]) * S[h] + K.T @ (np.exp(G[-1] - G)[:, None] * Dl)
    return S, o


@pytest.mark.parametrize("T", [1, 5, 64, 65, 150])
def test_chunked_form_equals_serial_steps(T):
    rng = np.random.default_rng(T)
    Hv, G, D = 4, 2, 16
    S0 = rng.normal(size=(Hv, D, D)) * 0.3
    q = rng.normal(size=(T, G, D)); k = rng.normal(size=(T, G, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True); k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(T, Hv, D))
    decay = rng.uniform(0.6, 1.0, size=(T, Hv)); beta = rng.uniform(0.0, 1.0, size=(T, Hv))
    S = S0.copy()
    o_ref = np.zeros((T, Hv, D))
    for t in range(T):
        S, o_ref[t] = moe_ref.gdn_step(S, q[t], k[t], v[t], decay[t], beta[t], G)
    S_c, o_c = chunked(S0, q, k, v, decay, beta, G)
    np.testing.assert_allclose(o_c, o_ref, rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(S_c, S, rtol=1e-9, atol=1e-9)
