"""Float64 host implementation of the qwen35moe graph (the MoE path's oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/ and the bench's checks, never by
the product. The reference has no CPU path for qwen35moe (its only backend
for it is MoeLLM on Metal), so this restates that backend's graph, in float64
over the bit-exact FP32 dequantized weights:

  forward per token         moe_llm.mm:2887-3039 (embedding, 40 x [norm ->
                            attention or DeltaNet -> residual -> norm -> MoE ->
                            residual], final norm, LM head on the last row)
  layer kind                moe_model.cpp:164-166 ((i + 1) % interval == 0 ->
                            full attention)
  gated full attention      moe_llm.mm:2238-2434; Q/gate split
                            metal_llm.metal:1167-1184; per-head RMSNorm
                            785-823; partial NeoX RoPE 928-967; QK/softmax/AV
                            826-890, 995-1061; sigmoid gate 1186-1197
  Gated DeltaNet            moe_llm.mm:2436-2640; softplus 1213-1224; causal
                            conv 1320-1341 + history 1345-1365; SiLU 1199-1211;
                            L2 norm 1280-1316 (eps inside the root); recurrence
                            1370-1420 (value head h reads key head h % G)
  router                    moe_llm.mm:2642-2690; softmax 826-890; top-k
                            insertion 1424-1459 (strict >, lowest id on ties);
                            renorm 1461-1474
  experts + shared expert   moe_llm.mm:2692-2843; expert products 1476-1521;
                            weighted reduce 1525-1542; SwiGLU 895-911

Prompt tokens go through the same per-token step as decode: the reference's
chunked prefill computes the same function (causal attention over the cache,
serial DeltaNet scan), so the states and the last row's logits agree.
"""

from __future__ import annotations

import numpy as np

from .gguf import GgufFile


# ---------------------------------------------------------------- operators
def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(x >= 0, 1.0 / (1.0 + np.exp(-np.abs(x))), np.exp(-np.abs(x)) / (1.0 + np.exp(-np.abs(x))))


def silu(x):
    return np.asarray(x, dtype=np.float64) * sigmoid(x)


def softplus(x):
    """metal_llm.metal:1213-1224: x > 20 -> x; x < -20 -> exp(x); else log(1 + exp(x))."""
    x = np.asarray(x, dtype=np.float64)
    mid = np.log1p(np.exp(np.clip(x, -20.0, 20.0)))
    return np.where(x > 20.0, x, np.where(x < -20.0, np.exp(np.minimum(x, 0.0)), mid))


def rmsnorm(x, gamma, eps):
    """y = x * 1/sqrt(mean(x^2) + eps) * gamma over the last axis."""
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(gamma, dtype=np.float64)


def l2norm(x, eps):
    """metal_l2norm_heads_f32: x * rsqrt(sum(x^2) + eps) over the last axis."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + eps)


def softmax(x):
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - np.max(x))
    return e / np.sum(e)


def topk_insertion(p, k):
    """metal_topk_f32: insertion scan with strict '>', so the lower id wins ties."""
    best_v = [-np.inf] * k
    best_i = [0xFFFFFFFF] * k
    for col, v in enumerate(p):
        for rank in range(k):
            if v > best_v[rank]:
                best_v.insert(rank, v)
                best_i.insert(rank, col)
                best_v.pop()
                best_i.pop()
                break
    return np.array(best_i, dtype=np.int64), np.array(best_v, dtype=np.float64)


def renorm(w):
    s = float(np.sum(w))
    return w * (1.0 / s if s > 0 else 0.0)


def rope_partial(x, pos, rot, theta):
    """NeoX RoPE on the first `rot` dims of every head row of x [heads, D]."""
    x = np.array(x, dtype=np.float64)
    half = rot // 2
    i = np.arange(half, dtype=np.float64)
    freq = theta ** (-2.0 * i / rot)
    ang = pos * freq
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:, :half].copy(), x[:, half:rot].copy()
    x[:, :half] = a * c - b * s
    x[:, half:rot] = a * s + b * c
    return x


def gdn_step(S, q, k, v, decay, beta, key_heads):
    """One token of the Gated DeltaNet recurrence, all value heads.

    S [Hv, Dk, Dv] (row = key dim, column = value dim), q/k [Hk, Dk],
    v [Hv, Dv], decay/beta [Hv]. Value head h reads key head h % Hk.
    Returns (S', o [Hv, Dv]), o = S'^T q / sqrt(Dk) (metal_llm.metal:1370-1420).
    """
    Hv, Dk, _ = S.shape
    S = S * decay[:, None, None]
    kk = k[np.arange(Hv) % key_heads]
    qq = q[np.arange(Hv) % key_heads]
    pred = np.einsum("hrc,hr->hc", S, kk)
    delta = beta[:, None] * (v - pred)
    S = S + kk[:, :, None] * delta[:, None, :]
    o = np.einsum("hrc,hr->hc", S, qq) / np.sqrt(Dk)
    return S, o


def conv_step(history, x, w):
    """Causal depthwise conv over [history (k-1 rows); x] for one token.

    history [k-1, C], x [C], w [C, k] (tap order oldest -> current).
    Returns (out [C], new history)."""
    window = np.vstack([history, x[None, :]])
    out = np.einsum("tc,ct->c", window, w)
    return out, window[1:]


# ---------------------------------------------------------------- the model
class MoeRef:
    """reset()/prefill()/decode() over a qwen35moe GGUF, float64 math."""

    def __init__(self, path, max_sequence=1024):
        g = self.g = GgufFile(path)
        m = g.meta
        a = "qwen35moe."
        if m.get("general.architecture") != "qwen35moe":
            raise ValueError("MoeRef requires a qwen35moe GGUF")
        self.L = int(m[a + "block_count"]) - int(m.get(a + "nextn_predict_layers", 0))
        self.H = int(m[a + "embedding_length"])
        self.Hq = int(m[a + "attention.head_count"])
        self.Hkv = int(m[a + "attention.head_count_kv"])
        self.D = int(m[a + "attention.key_length"])
        self.R = int(m[a + "rope.dimension_count"])
        self.theta = float(m.get(a + "rope.freq_base", 1e6))
        self.eps = float(m.get(a + "attention.layer_norm_rms_epsilon", 1e-6))
        self.E = int(m[a + "expert_count"])
        self.K = int(m[a + "expert_used_count"])
        self.FF = int(m[a + "expert_feed_forward_length"])
        self.FFs = int(m[a + "expert_shared_feed_forward_length"])
        self.interval = int(m[a + "full_attention_interval"])
        self.conv_k = int(m[a + "ssm.conv_kernel"])
        self.S = int(m[a + "ssm.state_size"])
        self.G = int(m[a + "ssm.group_count"])
        self.Hv = int(m[a + "ssm.time_step_rank"])
        self.inner = int(m[a + "ssm.inner_size"])
        self.V = int(m["tokenizer.ggml.tokens_count"])
        self.max_sequence = max_sequence
        self._cache = {}
        self.reset()

    # -- weights (FP32 dequant, then float64), cached per tensor / expert
    def W(self, name):
        if name not in self._cache:
            self._cache[name] = self.g.f32_rows(name).astype(np.float64)
        return self._cache[name]

    def vec(self, name):
        return self.W(name).reshape(-1)

    def expert(self, name, e, rows):
        key = (name, e)
        if key not in self._cache:
            self._cache[key] = self.g.f32_rows(name, e * rows, (e + 1) * rows).astype(np.float64)
        return self._cache[key]

    def is_full(self, i):
        return (i + 1) % self.interval == 0

    def reset(self):
        self.pos = 0
        qkv_w = 2 * self.G * self.S + self.inner
        self.state = {i: np.zeros((self.Hv, self.S, self.S)) for i in range(self.L) if not self.is_full(i)}
        self.hist = {i: np.zeros((self.conv_k - 1, qkv_w)) for i in range(self.L) if not self.is_full(i)}
        self.kc = {i: [] for i in range(self.L) if self.is_full(i)}
        self.vc = {i: [] for i in range(self.L) if self.is_full(i)}
        self.last_routes = {}

    # -- sub-graphs
    def attention(self, i, n):
        p = f"blk.{i}."
        D, Hq, Hkv = self.D, self.Hq, self.Hkv
        mixed = self.W(p + "attn_q.weight") @ n
        mixed = mixed.reshape(Hq, 2 * D)
        q, gate = mixed[:, :D], mixed[:, D:]
        k = (self.W(p + "attn_k.weight") @ n).reshape(Hkv, D)
        v = (self.W(p + "attn_v.weight") @ n).reshape(Hkv, D)
        q = rmsnorm(q, self.vec(p + "attn_q_norm.weight"), self.eps)
        k = rmsnorm(k, self.vec(p + "attn_k_norm.weight"), self.eps)
        q = rope_partial(q, self.pos, self.R, self.theta)
        k = rope_partial(k, self.pos, self.R, self.theta)
        self.kc[i].append(k)
        self.vc[i].append(v)
        K = np.stack(self.kc[i])  # [T, Hkv, D]
        Vv = np.stack(self.vc[i])
        out = np.empty((Hq, D))
        group = Hq // Hkv
        for h in range(Hq):
            g = h // group
            scores = (K[:, g, :] @ q[h]) * (1.0 / np.sqrt(D))
            out[h] = softmax(scores) @ Vv[:, g, :]
        o = (out * sigmoid(gate)).reshape(-1)
        return self.W(p + "attn_output.weight") @ o

    def deltanet(self, i, n):
        p = f"blk.{i}."
        qkv = self.W(p + "attn_qkv.weight") @ n
        z = self.W(p + "attn_gate.weight") @ n
        beta = sigmoid(self.W(p + "ssm_beta.weight") @ n)
        alpha = self.W(p + "ssm_alpha.weight") @ n
        decay = np.exp(softplus(alpha + self.vec(p + "ssm_dt.bias")) * self.vec(p + "ssm_a"))
        conv, self.hist[i] = conv_step(self.hist[i], qkv, self.W(p + "ssm_conv1d.weight"))
        act = silu(conv)
        kw = self.G * self.S
        q = l2norm(act[:kw].reshape(self.G, self.S), self.eps)
        k = l2norm(act[kw:2 * kw].reshape(self.G, self.S), self.eps)
        v = act[2 * kw:].reshape(self.Hv, self.S)
        self.state[i], o = gdn_step(self.state[i], q, k, v, decay, beta, self.G)
        on = rmsnorm(o, self.vec(p + "ssm_norm.weight"), self.eps).reshape(-1)
        return self.W(p + "ssm_out.weight") @ (on * silu(z))

    def moe(self, i, n):
        p = f"blk.{i}."
        probs = softmax(self.W(p + "ffn_gate_inp.weight") @ n)
        ids, vals = topk_insertion(probs, self.K)
        w = renorm(vals)
        self.last_routes[i] = (ids, w)
        routed = np.zeros(self.H)
        for e, we in zip(ids, w):
            g = self.expert(p + "ffn_gate_exps.weight", int(e), self.FF) @ n
            u = self.expert(p + "ffn_up_exps.weight", int(e), self.FF) @ n
            d = self.expert(p + "ffn_down_exps.weight", int(e), self.H) @ (silu(g) * u)
            routed = routed + we * d
        sg = sigmoid(self.vec(p + "ffn_gate_inp_shexp.weight") @ n)
        sh = self.W(p + "ffn_down_shexp.weight") @ (
            silu(self.W(p + "ffn_gate_shexp.weight") @ n) * (self.W(p + "ffn_up_shexp.weight") @ n))
        return routed + sh * sg

    def step(self, token, want_logits):
        x = self.g.f32_rows("token_embd.weight", token, token + 1)[0].astype(np.float64)
        for i in range(self.L):
            p = f"blk.{i}."
            n = rmsnorm(x, self.vec(p + "attn_norm.weight"), self.eps)
            x = x + (self.attention(i, n) if self.is_full(i) else self.deltanet(i, n))
            n2 = rmsnorm(x, self.vec(p + "post_attention_norm.weight"), self.eps)
            x = x + self.moe(i, n2)
        self.pos += 1
        if not want_logits:
            return None
        h = rmsnorm(x, self.vec("output_norm.weight"), self.eps)
        logits = np.empty(self.V)
        chunk = 8192
        for r0 in range(0, self.V, chunk):
            r1 = min(self.V, r0 + chunk)
            logits[r0:r1] = self.g.f32_rows("output.weight", r0, r1).astype(np.float64) @ h
        return logits

    def prefill(self, ids):
        if self.pos != 0:
            raise ValueError("prefill requires an empty state; call reset first")
        logits = None
        for t, tok in enumerate(ids):
            logits = self.step(int(tok), t + 1 == len(ids))
        self.logits = logits
        return int(np.argmax(logits))

    def decode(self, token):
        self.logits = self.step(int(token), True)
        return int(np.argmax(self.logits))
