"""Pins the float64 qwen35moe host reference (oracle/moe_ref.py).

The reference has no CPU path for qwen35moe, so its oracle is this float64
restatement of MoeLLM's graph. Each operator is checked against what the
mathematics fixes, so a dropped term, a transposed state or a wrong tie rule
fails here:
* Gated DeltaNet step: against an explicit per-column loop written from
  metal_gdn_recurrence_f32 (metal_llm.metal:1370-1420); beta = 0 only decays
  the state; decay 1, beta 1 and a unit key make S^T k equal v (the delta
  rule); value head h reads key head h % G.
* causal conv: a unit current tap is the identity, a unit oldest tap is a
  shift by k - 1 tokens, and the history rolls.
* top-k: ties go to the lower expert id; renormalised weights sum to 1.
* softplus branch points, sigmoid symmetry, RMSNorm / L2 closed forms.
* partial RoPE: position 0 is the identity, pair norms are preserved, dims
  past the rotary width are untouched.
* the whole model: prefill(p + [t]) gives the same last logits as
  prefill(p) then decode(t) (state carry), and reset() restores the start.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import moe_ref


def test_gdn_step_matches_per_column_loop():
    rng = np.random.default_rng(0)
    Hv, G, D = 4, 2, 5
    S = rng.normal(size=(Hv, D, D))
    q, k = rng.normal(size=(G, D)), rng.normal(size=(G, D))
    v = rng.normal(size=(Hv, D))
    decay, beta = rng.uniform(0.5, 1.0, Hv), rng.uniform(0.0, 1.0, Hv)
    S2, o = moe_ref.gdn_step(S.copy(), q, k, v, decay, beta, G)
    # Per-column loop in the order of the Metal kernel.
    Sx = S.copy()
    ox = np.zeros((Hv, D))
    for h in range(Hv):
        kh = h % G
        for col in range(D):
            pred = 0.0
            for row in range(D):
                Sx[h, row, col] *= decay[h]
                pred += Sx[h, row, col] * k[kh, row]
            delta = beta[h] * (v[h, col] - pred)
            res = 0.0
            for row in range(D):
                Sx[h, row, col] += k[kh, row] * delta
                res += Sx[h, row, col] * q[kh, row] / math.sqrt(D)
            ox[h, col] = res
    np.testing.assert_allclose(S2, Sx, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(o, ox, rtol=1e-12, atol=1e-12)


def test_gdn_beta_zero_only_decays():
    rng = np.random.default_rng(1)
    S = rng.normal(size=(2, 4, 4))
    q, k, v = rng.normal(size=(1, 4)), rng.normal(size=(1, 4)), rng.normal(size=(2, 4))
    S2, o = moe_ref.gdn_step(S.copy(), q, k, v, np.array([0.5, 0.25]), np.zeros(2), 1)
    np.testing.assert_allclose(S2, S * np.array([0.5, 0.25])[:, None, None])
    np.testing.assert_allclose(o[0], S2[0].T @ q[0] / 2.0)


def test_gdn_delta_rule_recalls_value():
    rng = np.random.default_rng(2)
    S = rng.normal(size=(1, 6, 6))
    k = rng.normal(size=(1, 6))
    k /= np.linalg.norm(k)
    v = rng.normal(size=(1, 6))
    S2, _ = moe_ref.gdn_step(S, k, k, v, np.ones(1), np.ones(1), 1)
    np.testing.assert_allclose(S2[0].T @ k[0], v[0], atol=1e-12)


def test_conv_taps_identity_and_shift():
    rng = np.random.default_rng(3)
    C, k = 5, 4
    hist = rng.normal(size=(k - 1, C))
    x = rng.normal(size=C)
    w_cur = np.zeros((C, k))
    w_cur[:, -1] = 1.0
    out, h2 = moe_ref.conv_step(hist, x, w_cur)
    np.testing.assert_array_equal(out, x)
    np.testing.assert_array_equal(h2, np.vstack([hist[1:], x[None]]))
    w_old = np.zeros((C, k))
    w_old[:, 0] = 1.0
    out, _ = moe_ref.conv_step(hist, x, w_old)
    np.testing.assert_array_equal(out, hist[0])


def test_topk_ties_lowest_id_and_renorm():
    p = np.array([0.1, 0.3, 0.3, 0.05, 0.3, 0.2])
    ids, vals = moe_ref.topk_insertion(p, 3)
    assert ids.tolist() == [1, 2, 4]
    ids, vals = moe_ref.topk_insertion(p, 4)
    assert ids.tolist() == [1, 2, 4, 5]
    assert abs(moe_ref.renorm(vals).sum() - 1.0) < 1e-15
    assert moe_ref.renorm(np.zeros(3)).sum() == 0.0


def test_scalar_functions():
    assert moe_ref.softplus(25.0) == 25.0
    assert moe_ref.softplus(-25.0) == pytest.approx(math.exp(-25.0), rel=1e-15)
    assert moe_ref.softplus(0.0) == pytest.approx(math.log(2.0))
    x = np.linspace(-30, 30, 61)
    np.testing.assert_allclose(moe_ref.sigmoid(x) + moe_ref.sigmoid(-x), 1.0, atol=1e-15)
    np.testing.assert_allclose(moe_ref.silu(x), x / (1 + np.exp(-x)), rtol=1e-12, atol=1e-300)
    v = np.array([3.0, 4.0])
    np.testing.assert_allclose(moe_ref.l2norm(v, 0.0), [0.6, 0.8])
    np.testing.assert_allclose(moe_ref.rmsnorm(v, np.ones(2), 0.0), v / math.sqrt(12.5))
    np.testing.assert_allclose(moe_ref.softmax(np.array([0.0, math.log(3.0)])), [0.25, 0.75])


def test_partial_rope():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3, 16))
    np.testing.assert_allclose(moe_ref.rope_partial(x, 0, 8, 1e4), x)
    y = moe_ref.rope_partial(x, 7, 8, 1e4)
    np.testing.assert_array_equal(y[:, 8:], x[:, 8:])
    for i in range(4):
        np.testing.assert_allclose(np.hypot(y[:, i], y[:, i + 4]), np.hypot(x[:, i], x[:, i + 4]))
    # angle of pair 0 advances by exactly pos * theta^0 = pos radians
    ang = np.arctan2(y[:, 4], y[:, 0]) - np.arctan2(x[:, 4], x[:, 0])
    np.testing.assert_allclose(np.mod(ang, 2 * np.pi), 7.0 % (2 * np.pi), atol=1e-9)


@pytest.fixture(scope="module")
def tiny_moe(tmp_path_factory):
    from myllm_amd import synth
    path = tmp_path_factory.mktemp("moe") / "moe-tiny.gguf"
    return synth.write_qwen35moe(path, synth.MOE_SHAPES["moe-tiny"], seed=3)


def test_model_state_carry_and_reset(tiny_moe):
    from myllm_amd import synth
    ids = synth.uniform_ids(6, 512, seed=5).tolist()
    m = moe_ref.MoeRef(tiny_moe)
    t = m.prefill(ids[:5])
    m.decode(ids[5])
    l1 = m.logits.copy()
    m.reset()
    m.prefill(ids)
    np.testing.assert_allclose(m.logits, l1, rtol=1e-12, atol=1e-12)
    m.reset()
    assert m.prefill(ids[:5]) == t
    assert m.pos == 5
    # routes: K distinct experts per layer, weights sum to 1
    for ids_l, w in m.last_routes.values():
        assert len(set(ids_l.tolist())) == m.K
        assert abs(w.sum() - 1.0) < 1e-12
