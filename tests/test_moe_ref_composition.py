"""Pins how oracle/moe_ref.py wires the qwen35moe graph together.

The operator tests (test_moe_ref.py) pin each function; these pin the
composition, so that a miswired projection, a swapped slice or a norm in the
wrong place fails one of them. Each test swaps small hand-chosen weights into
a MoeRef built on the tiny synthetic qwen35moe file and compares one
sub-graph with an independent statement of it:

* a single routed expert (E = K = 1) with a zero shared expert is exactly a
  dense SwiGLU FFN: compared with the FP32 FFN of the CPU oracle's decode
  layer (oracle.ffn, cpu_llm.cpp:907-913, pinned bit for bit by the
  reference's golden vectors);
* routed experts with zero down projections leave the shared expert scaled by
  its gate: sigmoid(w . n) (moe_llm.mm:2807-2842), 1/2 exactly when w . n = 0;
* zero attention / DeltaNet output projections: the mixers add exactly
  nothing, every layer's residual is the MoE of its post-attention norm;
* a brute-force tiny gated-attention layer written element by element from
  the kernels' index formulas: the interleaved [Q_h | gate_h] split
  (metal_llm.metal:1167-1184), per-head RMSNorm (785-823), partial NeoX RoPE
  (928-967), scaled QK / softmax / AV over the cache (826-890, 995-1061), the
  sigmoid output gate (moe_llm.mm:2420-2428);
* a brute-force tiny DeltaNet layer over three tokens: the causal conv and
  its history (metal_llm.metal:1320-1365, tap t reads concat row token + t,
  weight[channel * k + tap]), SiLU, the q | k | v slices and per-head L2 norm
  (moe_llm.mm:2563-2600, metal_llm.metal:1280-1316), the gates
  (moe_llm.mm:2462-2496), the per-column recurrence with value head h on key
  head h % G (1370-1420), the per-head state RMSNorm times SiLU(z)
  (moe_llm.mm:2617-2638).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from oracle import moe_ref


@pytest.fixture(scope="module")
def tiny_moe_path(tmp_path_factory):
    from myllm_amd import synth
    path = tmp_path_factory.mktemp("moe_comp") / "moe-tiny.gguf"
    return synth.write_qwen35moe(path, synth.MOE_SHAPES["moe-tiny"], seed=11)


def fresh(path):
    return moe_ref.MoeRef(path, max_sequence=16)


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


# ------------------------------------------------------------------ MoE
def _dense_expert_weights(rng, H, FF, scale=0.2):
    f32 = lambda *s: (rng.normal(size=s) * scale).astype(np.float32)
    return f32(FF, H), f32(FF, H), f32(H, FF)


def test_single_expert_moe_is_dense_ffn(tiny_moe_path):
    m = fresh(tiny_moe_path)
    rng = np.random.default_rng(1)
    H, FF, i = m.H, m.FF, 0
    p = f"blk.{i}."
    wg, wu, wd = _dense_expert_weights(rng, H, FF)
    m.K = 1
    m._cache[p + "ffn_gate_inp.weight"] = rng.normal(size=(1, H))
    m._cache[(p + "ffn_gate_exps.weight", 0)] = wg.astype(np.float64)
    m._cache[(p + "ffn_up_exps.weight", 0)] = wu.astype(np.float64)
    m._cache[(p + "ffn_down_exps.weight", 0)] = wd.astype(np.float64)
    m._cache[p + "ffn_gate_inp_shexp.weight"] = rng.normal(size=(1, H))
    for name, shape in (("ffn_gate_shexp", (m.FFs, H)), ("ffn_up_shexp", (m.FFs, H)),
                        ("ffn_down_shexp", (H, m.FFs))):
        m._cache[p + name + ".weight"] = np.zeros(shape)
    n = rng.normal(size=H).astype(np.float32)
    got = m.moe(i, n.astype(np.float64))
    ref = oracle.ffn(wg, wu, wd, n)
    ids, w = m.last_routes[i]
    assert ids.tolist() == [0] and w.tolist() == [1.0]
    assert rel(got, ref) <= 1e-5
    # Gate and up swapped would compute silu(up) * gate instead:
    assert rel(oracle.ffn(wu, wg, wd, n), ref) > 1e-2


def test_shared_expert_gate_closed_form(tiny_moe_path):
    m = fresh(tiny_moe_path)
    rng = np.random.default_rng(2)
    H, i = m.H, 1
    p = f"blk.{i}."
    sg, su, sd = _dense_expert_weights(rng, H, m.FFs)
    m._cache[p + "ffn_gate_shexp.weight"] = sg.astype(np.float64)
    m._cache[p + "ffn_up_shexp.weight"] = su.astype(np.float64)
    m._cache[p + "ffn_down_shexp.weight"] = sd.astype(np.float64)
    # Routed experts contribute nothing: zero down projections for all.
    for e in range(m.E):
        m._cache[(p + "ffn_down_exps.weight", e)] = np.zeros((H, m.FF))
    n = rng.normal(size=H).astype(np.float32)
    shared = oracle.ffn(sg, su, sd, n).astype(np.float64)
    w = rng.normal(size=H)
    w_perp = w - (w @ n) / (n.astype(np.float64) @ n) * n  # w . n = 0
    for gate_w, factor in ((w_perp, 0.5), (w, 1.0 / (1.0 + math.exp(-float(w @ n))))):
        m._cache[p + "ffn_gate_inp_shexp.weight"] = gate_w[None, :]
        got = m.moe(i, n.astype(np.float64))
        assert rel(got, factor * shared) <= 1e-5


def test_zeroed_mixers_add_nothing(tiny_moe_path):
    m = fresh(tiny_moe_path)
    ref = fresh(tiny_moe_path)
    rng = np.random.default_rng(5)
    for i in range(m.L):
        name = "attn_output.weight" if m.is_full(i) else "ssm_out.weight"
        rows, cols = (m.H, m.Hq * m.D) if m.is_full(i) else (m.H, m.inner)
        m._cache[f"blk.{i}.{name}"] = np.zeros((rows, cols))
        # Distinct norm gains (the synthetic files hold 1.0), so the MoE
        # reading the wrong norm would show.
        for norm in ("attn_norm.weight", "post_attention_norm.weight"):
            gain = rng.uniform(0.5, 1.5, size=(1, m.H))
            m._cache[f"blk.{i}.{norm}"] = gain
            ref._cache[f"blk.{i}.{norm}"] = gain
    tok = 17
    m.step(tok, False)
    # The same layer stack with the mixers left out.
    x = ref.g.f32_rows("token_embd.weight", tok, tok + 1)[0].astype(np.float64)
    for i in range(ref.L):
        n2 = moe_ref.rmsnorm(x, ref.vec(f"blk.{i}.post_attention_norm.weight"), ref.eps)
        x = x + ref.moe(i, n2)
    h = moe_ref.rmsnorm(x, ref.vec("output_norm.weight"), ref.eps)
    m.reset()
    logits = m.step(tok, True)
    ref_logits = ref.g.f32_rows("output.weight").astype(np.float64) @ h
    assert rel(logits, ref_logits) <= 1e-12
    # The mixers still ran: DeltaNet states and the KV caches hold this token.
    assert all(np.abs(s).max() > 0 for s in m.state.values())
    assert all(len(k) == 1 for k in m.kc.values())


# ------------------------------------------------------ gated attention
def _attention_brute_force(mixed_rows, k_rows, v_rows, qn, kn, Hq, Hkv, D, R, theta, eps):
    """Element-by-element gated attention over len(mixed_rows) tokens."""
    T = len(mixed_rows)
    q = np.zeros((T, Hq, D))
    gate = np.zeros((T, Hq, D))
    for t in range(T):
        for idx in range(Hq * D):  # metal_split_interleaved_q_gate_f32
            head, local = idx // D, idx % D
            src = head * D * 2 + local
            q[t, head, local] = mixed_rows[t][src]
            gate[t, head, local] = mixed_rows[t][src + D]
    k = np.array(k_rows, dtype=np.float64).reshape(T, Hkv, D)
    v = np.array(v_rows, dtype=np.float64).reshape(T, Hkv, D)

    def head_norm(x, g):
        ss = 0.0
        for d in range(D):
            ss += x[d] * x[d]
        inv = 1.0 / math.sqrt(ss / D + eps)
        return np.array([x[d] * inv * g[d] for d in range(D)])

    def rope(x, pos):
        y = x.copy()
        for i in range(R // 2):
            freq = theta ** (-2.0 * i / R)
            c, s = math.cos(pos * freq), math.sin(pos * freq)
            a, b = x[i], x[i + R // 2]
            y[i] = a * c - b * s
            y[i + R // 2] = a * s + b * c
        return y

    for t in range(T):
        for h in range(Hq):
            q[t, h] = rope(head_norm(q[t, h], qn), t)
        for g in range(Hkv):
            k[t, g] = rope(head_norm(k[t, g], kn), t)
    outs = []
    for t in range(T):
        o = np.zeros(Hq * D)
        for h in range(Hq):
            g = h // (Hq // Hkv)
            scores = [sum(k[j, g, d] * q[t, h, d] for d in range(D)) / math.sqrt(D) for j in range(t + 1)]
            mx = max(scores)
            e = [math.exp(s - mx) for s in scores]
            z = sum(e)
            for d in range(D):
                acc = sum(e[j] / z * v[j, g, d] for j in range(t + 1))
                o[h * D + d] = acc / (1.0 + math.exp(-gate[t, h, d]))
        outs.append(o)
    return outs


def test_gated_attention_matches_brute_force(tiny_moe_path):
    m = fresh(tiny_moe_path)
    i = 1
    assert m.is_full(i)
    p = f"blk.{i}."
    rng = np.random.default_rng(3)
    H, Hq, Hkv, D, R = 16, 4, 2, 4, 2
    m.H, m.Hq, m.Hkv, m.D, m.R = H, Hq, Hkv, D, R
    m.reset()
    wq = rng.normal(size=(Hq * 2 * D, H))
    wk = rng.normal(size=(Hkv * D, H))
    wv = rng.normal(size=(Hkv * D, H))
    qn, kn = rng.uniform(0.5, 1.5, D), rng.uniform(0.5, 1.5, D)
    wo = np.eye(H, Hq * D)  # output projection = identity on the first Hq * D dims
    for name, w in (("attn_q.weight", wq), ("attn_k.weight", wk), ("attn_v.weight", wv),
                    ("attn_q_norm.weight", qn[None, :]), ("attn_k_norm.weight", kn[None, :]),
                    ("attn_output.weight", wo)):
        m._cache[p + name] = w
    ns = [rng.normal(size=H) for _ in range(3)]
    got = []
    for t, n in enumerate(ns):
        m.pos = t
        got.append(m.attention(i, n)[: Hq * D])
    ref = _attention_brute_force([wq @ n for n in ns], [wk @ n for n in ns], [wv @ n for n in ns], qn, kn, Hq, Hkv,
                                 D, R, m.theta, m.eps)
    for a, b in zip(got, ref):
        assert rel(a, b) <= 1e-12


# ------------------------------------------------------------- DeltaNet
def test_deltanet_matches_brute_force(tiny_moe_path):
    m = fresh(tiny_moe_path)
    i = 0
    assert not m.is_full(i)
    p = f"blk.{i}."
    rng = np.random.default_rng(4)
    H, G, S, Hv, K = 12, 2, 3, 4, 3
    inner = Hv * S
    C = 2 * G * S + inner
    m.H, m.G, m.S, m.Hv, m.inner, m.conv_k = H, G, S, Hv, inner, K
    m.reset()
    w = {"attn_qkv.weight": rng.normal(size=(C, H)), "attn_gate.weight": rng.normal(size=(inner, H)),
         "ssm_beta.weight": rng.normal(size=(Hv, H)), "ssm_alpha.weight": rng.normal(size=(Hv, H)),
         "ssm_dt.bias": rng.normal(size=(1, Hv)), "ssm_a": -rng.uniform(0.1, 1.0, size=(1, Hv)),
         "ssm_conv1d.weight": rng.normal(size=(C, K)), "ssm_norm.weight": rng.uniform(0.5, 1.5, size=(1, S)),
         "ssm_out.weight": np.eye(H, inner)}
    for name, val in w.items():
        m._cache[p + name] = val
    ns = [rng.normal(size=H) for _ in range(3)]
    got = [m.deltanet(i, n)[:inner] for n in ns]

    # Brute force, one element at a time.
    hist = np.zeros((K - 1, C))
    state = np.zeros((Hv, S, S))
    sig = lambda x: 1.0 / (1.0 + math.exp(-x))
    for t, n in enumerate(ns):
        x = w["attn_qkv.weight"] @ n
        conv = np.zeros(C)
        for ch in range(C):  # metal_depthwise_conv1d_causal_f32, one token
            acc = 0.0
            for tap in range(K):
                row = tap  # token 0 of this call + tap
                val = hist[row, ch] if row < K - 1 else x[ch]
                acc += val * w["ssm_conv1d.weight"][ch, tap]
            conv[ch] = acc
        new_hist = np.zeros_like(hist)
        for ch in range(C):  # metal_conv_history_commit_f32, tokens = 1
            for row in range(K - 1):
                src = 1 + row
                new_hist[row, ch] = hist[src, ch] if src < K - 1 else x[ch]
        hist = new_hist
        act = np.array([c * sig(c) for c in conv])
        q = act[: G * S].reshape(G, S)
        k = act[G * S: 2 * G * S].reshape(G, S)
        v = act[2 * G * S:].reshape(Hv, S)
        for g in range(G):
            q[g] = q[g] / math.sqrt(sum(e * e for e in q[g]) + m.eps)
            k[g] = k[g] / math.sqrt(sum(e * e for e in k[g]) + m.eps)
        beta = [sig(b) for b in w["ssm_beta.weight"] @ n]
        alpha = w["ssm_alpha.weight"] @ n + w["ssm_dt.bias"][0]
        decay = [math.exp(math.log1p(math.exp(a)) * w["ssm_a"][0][h]) for h, a in enumerate(alpha)]
        o = np.zeros((Hv, S))
        for h in range(Hv):
            kh = h % G
            for col in range(S):
                pred = 0.0
                for row in range(S):
                    state[h, row, col] *= decay[h]
                    pred += state[h, row, col] * k[kh, row]
                delta = beta[h] * (v[h, col] - pred)
                res = 0.0
                for row in range(S):
                    state[h, row, col] += k[kh, row] * delta
                    res += state[h, row, col] * q[kh, row]
                o[h, col] = res / math.sqrt(S)
        z = w["attn_gate.weight"] @ n
        out = np.zeros(inner)
        for h in range(Hv):
            inv = 1.0 / math.sqrt(sum(e * e for e in o[h]) / S + m.eps)
            for col in range(S):
                j = h * S + col
                out[j] = o[h, col] * inv * w["ssm_norm.weight"][0][col] * (z[j] * sig(z[j]))
        assert rel(got[t], out) <= 1e-12, t
    assert rel(m.state[i], state) <= 1e-12
    assert rel(m.hist[i], hist) <= 1e-12
