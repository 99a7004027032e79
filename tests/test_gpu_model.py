"""End-to-end HipLLM parity on the GPU, through the C ABI handle API.

Golden vectors come from the reference's own CPULLM (tests/golden):
* tiny model (every block type): the 32 greedy tokens match and every step's
  logits satisfy max|l - ref| / max|ref| <= 1e-3;
* Qwen2.5-0.5B-shaped Q4_K_M model: the 32 greedy tokens match, and the
  top-64 reference logits of each step are reproduced within the same bound;
  the top-1/top-2 margin of each step is reported so a flip could be judged.
Also the reference's error contract (metal_llm.mm:3190-3314) and memory stats.
"""

from __future__ import annotations

import numpy as np
import pytest

from myllm_amd import synth
from myllm_amd.hipllm import kernels, HipLLM, LengthError, generate

pytestmark = pytest.mark.gpu


def run_with_logits(model, prompt, n):
    logits = []
    toks = generate(model, list(prompt), n, on_step=lambda m: logits.append(m.logits()))
    return toks, np.stack(logits)


# Token-serial prefill runs the FP32 decode kernels (bound 1e-3); the batched
# prefill runs fp16 MFMA matmuls, whose contract bound is 2e-2 on logits.
LOGIT_BOUND = {False: 1e-3, True: 2e-2}


@pytest.mark.parametrize("batched", [False, True])
def test_tiny_matches_reference(cuda, golden_model, batched):
    path, g = golden_model("tiny")
    with HipLLM(path, int(g["max_sequence"])) as m:
        m.set_batched_prefill(batched)
        toks, logits = run_with_logits(m, g["prompt"], len(g["tokens"]))
    ref = g["logits"].astype(np.float64)
    err = np.abs(logits - ref).max(axis=1) / np.abs(ref).max(axis=1)
    print("max rel logit error per step:", err.max())
    assert toks == g["tokens"].tolist()
    assert err.max() <= LOGIT_BOUND[batched], err


@pytest.mark.parametrize("batched", [False, True])
def test_qwen05b_greedy_tokens_match_reference(cuda, golden_model, batched):
    path, g = golden_model("qwen2.5-0.5b")
    with HipLLM(path, int(g["max_sequence"])) as m:
        m.set_batched_prefill(batched)
        toks, logits = run_with_logits(m, g["prompt"], len(g["tokens"]))
    top = np.take_along_axis(logits, g["top_index"], axis=1).astype(np.float64)
    ref = g["top_logit"].astype(np.float64)
    margins = ref[:, 0] - ref[:, 1]
    print("top1-top2 margins (min, median):", margins.min(), np.median(margins))
    err = np.abs(top - ref).max(axis=1) / np.abs(ref).max(axis=1)
    print("max rel logit error per step:", err.max())
    assert toks == g["tokens"].tolist()
    assert err.max() <= LOGIT_BOUND[batched]


def test_attention_head_kernel_matches_split_kernel(cuda, golden_model):
    """Decode attention at a capacity of 2 to 4 chunks of 64 keys runs one
    block per head that merges its chunks in LDS; at larger capacities one
    block per chunk and a merge launch. Both compute each chunk and the
    merge the same way, so a decode crossing from 2 into 3 and 4 chunks gives
    the same tokens and logit bits at capacity 256 as at capacity 1024."""
    path, g = golden_model("qwen2.5-0.5b")
    prompt = (list(g["prompt"]) * 40)[:100]
    runs = []
    for cap in (256, 1024):
        with HipLLM(path, cap) as m:
            toks, logits = run_with_logits(m, prompt, 120)
        runs.append((toks, logits))
    assert runs[0][0] == runs[1][0]
    assert np.array_equal(runs[0][1].view(np.int32), runs[1][1].view(np.int32))


def test_fused_norms_match_separate_norms(cuda, golden_model):
    """With x16 copies of every projection the decode RMSNorms ride in the
    GEMVs (norm data from the attention output and FFN down epilogues, the
    scaling in QKV, gate / up and the LM head): same greedy tokens as the
    reference's CPULLM and as separate norm launches, logits within FP32
    rounding of them."""
    path, g = golden_model("qwen2.5-7b")
    runs = {}
    for fused in (True, False):
        with HipLLM(path, int(g["max_sequence"])) as m:
            m.set_fused_norms(fused)
            runs[fused] = run_with_logits(m, g["prompt"], len(g["tokens"]))
    assert runs[True][0] == runs[False][0] == g["tokens"].tolist()
    a, b = runs[True][1].astype(np.float64), runs[False][1].astype(np.float64)
    assert (np.abs(a - b).max(axis=1) / np.abs(b).max(axis=1)).max() <= 1e-4


def test_batched_prefill_is_default_and_switchable(cuda, golden_model):
    path, g = golden_model("tiny")
    with HipLLM(path, 64) as m:
        batched = m.prefill(list(g["prompt"]))
        lb = m.logits()
        m.reset()
        m.set_batched_prefill(False)
        serial = m.prefill(list(g["prompt"]))
        ls = m.logits()
    assert batched == serial == int(g["tokens"][0])
    assert np.abs(lb - ls).max() / np.abs(ls).max() <= 2e-2


def test_contract_errors(cuda, golden_model):
    path, _ = golden_model("tiny")
    with HipLLM(path, 20) as m:
        assert m.uses_gpu and m.device_name
        with pytest.raises(ValueError):
            m.decode(1)
        with pytest.raises(ValueError):
            m.prefill([])
        with pytest.raises(IndexError):
            m.prefill([1, 2, 5000])
        with pytest.raises(LengthError):
            m.prefill(list(range(21)))
        m.prefill([1, 2, 3])
        with pytest.raises(ValueError):
            m.prefill([1])
        with pytest.raises(IndexError):
            m.decode(-1)
        for _ in range(17):
            m.decode(4)
        with pytest.raises(LengthError):
            m.decode(4)
        m.reset()
        assert m.position == 0
        m.prefill([7])
        assert m.position == 1
    with pytest.raises(ValueError):
        HipLLM(path, 10 ** 6)  # beyond the context length


def test_memory_stats(cuda, golden_model):
    path, _ = golden_model("tiny")
    from myllm_amd.hipllm import inspect_gguf
    cfg = inspect_gguf(path)
    with HipLLM(path, 64) as m:
        s = m.memory_stats()
        m.set_packed_decode(False)
    # The GGUF payload plus the x16 decode copies of the Q4_K / Q6_K
    # projections (tiny: Q4_K fused QKV and gate / up pair, Q6_K down and LM
    # head; the attention output is Q5_0), each 256-byte aligned.
    h, f, kv = cfg["embedding_size"], cfg["feed_forward_size"], cfg["kv_head_count"] * cfg["head_size"]
    v = cfg["vocabulary_size"]

    def packed(qtype, n, k):
        return -(-kernels.x16_bytes(qtype, n, k) // 256) * 256

    per_layer = packed(synth.Q4_K, h + 2 * kv, h) + 2 * packed(synth.Q4_K, f, h) + packed(synth.Q6_K, h, f)
    x16 = cfg["layer_count"] * per_layer + packed(synth.Q6_K, v, h)
    assert per_layer > 0
    assert s["weight_bytes"] == cfg["stored_weight_bytes"] + x16
    kv = cfg["kv_head_count"] * cfg["head_size"]
    assert s["kv_cache_bytes"] == 2 * cfg["layer_count"] * 64 * kv * 4
    assert s["recurrent_state_bytes"] == 0 and s["intermediate_bytes"] > 0
    assert s["intermediate_is_estimate"] == 0


def test_reset_reproduces_same_tokens(cuda, golden_model):
    path, g = golden_model("tiny")
    with HipLLM(path) as m:
        a = generate(m, list(g["prompt"]), 8)
        b = generate(m, list(g["prompt"]), 8)
    assert a == b == g["tokens"][:8].tolist()


def test_batched_prefill_is_bit_reproducible(cuda, golden_model):
    """A 64-row prompt on the 0.5B shape splits its prefill matmuls along k;
    the partial sums are added in a fixed order, so the same prompt gives the
    same logits bit for bit on every run."""
    path, g = golden_model("qwen2.5-0.5b")
    prompt = (list(g["prompt"]) * 4)[:64]
    runs = []
    with HipLLM(path, 128) as m:
        for _ in range(3):
            m.reset()
            m.prefill(prompt)
            runs.append(m.logits().copy())
    for r in runs[1:]:
        assert np.array_equal(runs[0].view(np.int32), r.view(np.int32))


def test_packed_decode_matches_gguf_row_decode(cuda, golden_model):
    """The x16 MFMA GEMVs and the vector GEMVs compute the same exact integer
    digit sums: decode logits agree to FP32 summation rounding and the greedy
    tokens are the same, graph or eager."""
    path, g = golden_model("tiny")
    prompt = list(g["prompt"])
    out = {}
    for packed in (True, False):
        with HipLLM(path, 64) as m:
            m.set_packed_decode(packed)
            m.set_batched_prefill(False)  # serial prefill through the decode GEMVs
            t = m.prefill(prompt)
            toks, logits = [t], [m.logits()]
            for _ in range(12):
                t = m.decode(t)
                toks.append(t)
                logits.append(m.logits())
            out[packed] = (toks, logits)
    assert out[True][0] == out[False][0] == g["tokens"][:13].tolist()
    for a, b in zip(out[True][1], out[False][1]):
        assert np.abs(a - b).max() / np.abs(b).max() <= 1e-5


def _decode_run(path, prompts, steps, graphs, max_sequence=64):
    """Tokens and logits of prefill + `steps` greedy decodes for each prompt
    in turn (reset between prompts), with decode graphs on or off."""
    toks, logits = [], []
    with HipLLM(path, max_sequence) as m:
        m.set_decode_graphs(graphs)
        for prompt in prompts:
            m.reset()
            t = m.prefill(prompt)
            toks.append(t)
            for _ in range(steps):
                t = m.decode(t)
                toks.append(t)
                logits.append(m.logits())
    return toks, logits


def test_decode_graph_matches_eager_launches(cuda, golden_model):
    # The second, longer prompt regrows the activation arena, which must
    # drop and re-record the decode graph.
    path, g = golden_model("tiny")
    prompts = [list(g["prompt"])[:4], list(g["prompt"]) * 2]
    tg, lg = _decode_run(path, prompts, 10, True)
    te, le = _decode_run(path, prompts, 10, False)
    assert tg == te
    for a, b in zip(lg, le):
        assert np.abs(a - b).max() / np.abs(b).max() <= 1e-5


def _edit_gguf(src, dst, edit):
    data = bytearray(open(src, "rb").read())
    edit(data)
    with open(dst, "wb") as f:
        f.write(bytes(data))
    return dst


def test_loader_rejects_schema_errors(cuda, golden_model, tmp_path):
    # The weight loader's tensor-schema checks (GgufReader take /
    # validate_all_consumed, the F32 norm rule of metal_llm.mm:866-871), each
    # raised while the tensor map is built, before anything is uploaded.
    import struct

    from tests.test_native_lib import tensor_info

    path, _ = golden_model("tiny")

    def missing(d):  # blk.0.ffn_up.weight -> blk.0.ffn_uq.weight
        t = tensor_info(d, "blk.0.ffn_up.weight")
        d[t["name_at"] + 10] = ord("q")

    def shape(d):  # attention Q with half its rows
        t = tensor_info(d, "blk.0.attn_q.weight")
        struct.pack_into("<Q", d, t["dims_at"] + 8, t["dims"][1] // 2)

    def unconsumed(d):  # block_count 2 -> 1: layer 1's tensors are left over
        key = b"qwen2.block_count"
        at = d.index(struct.pack("<Q", len(key)) + key) + 8 + len(key)
        assert struct.unpack_from("<I", d, at)[0] == 4  # GGUF uint32 value
        struct.pack_into("<I", d, at + 4, 1)

    def f16_norm(d):  # an F32 norm retyped F16
        t = tensor_info(d, "blk.0.attn_norm.weight")
        struct.pack_into("<I", d, t["type_at"], 1)

    cases = [(missing, RuntimeError, "missing tensor: blk.0.ffn_up.weight"),
             (shape, RuntimeError, "unexpected shape for tensor blk.0.attn_q.weight"),
             (unconsumed, RuntimeError, "not mapped by the loader: .*blk.1."),
             (f16_norm, ValueError, "must be F32: blk.0.attn_norm.weight")]
    for edit, exc, msg in cases:
        bad = _edit_gguf(path, tmp_path / f"{edit.__name__}.gguf", edit)
        with pytest.raises(exc, match=msg):
            HipLLM(bad, 32)


@pytest.mark.parametrize("batched", [False, True])
def test_qwen7b_greedy_tokens_match_reference(cuda, golden_model, batched):
    # Qwen2.5-7B-shaped Q4_K_M model (28 layers, hidden 3584, FFN 18944):
    # the reference CPULLM's 16 greedy tokens from an 8-token prompt, and its
    # top-64 logits of every step within the logits bound.
    path, g = golden_model("qwen2.5-7b")
    with HipLLM(path, int(g["max_sequence"])) as m:
        m.set_batched_prefill(batched)
        toks, logits = run_with_logits(m, g["prompt"], len(g["tokens"]))
    top = np.take_along_axis(logits, g["top_index"], axis=1).astype(np.float64)
    ref = g["top_logit"].astype(np.float64)
    margins = ref[:, 0] - ref[:, 1]
    print("top1-top2 margins (min, median):", margins.min(), np.median(margins))
    err = np.abs(top - ref).max(axis=1) / np.abs(ref).max(axis=1)
    print("max rel logit error per step:", err.max())
    assert toks == g["tokens"].tolist()
    assert err.max() <= LOGIT_BOUND[batched]


def test_qwen14b_full_size_properties(cuda, tmp_path):
    # Qwen2.5-14B-shaped Q4_K_M model (48 layers, hidden 5120, 40/8 heads of
    # 128, FFN 13824, vocabulary 152064) with a KV cache of 4096 rows, a
    # 128-token prompt and 128 greedy decode steps. Its CPU reference does
    # not fit a test (about 60 GB of FP32 weights, minutes per token), so the
    # checks are size-independent properties of the GPU paths:
    # * batched (fp16 MFMA) prefill against token-serial prefill (the FP32
    #   decode kernels): logits within 2e-2, the same first token unless the
    #   serial top-2 margin is inside that error;
    # * 128 decode steps replayed as one recorded graph per token against the
    #   same steps launched eagerly (splits fixed by the capacity vs by the
    #   length): identical tokens, logits within 1e-4 at every step.
    from myllm_amd import synth
    shape = synth.SHAPES["qwen2.5-14b"]
    path = synth.write_qwen2(tmp_path / "qwen14b.gguf", shape, seed=0)
    prompt = synth.uniform_ids(128, shape.vocab, seed=0).tolist()
    print("14B-shaped model written", flush=True)
    with HipLLM(path, 4096) as m:
        tb = m.prefill(prompt)
        lb = m.logits().astype(np.float64)
        runs = {}
        for graphs in (True, False):
            m.reset()
            m.set_batched_prefill(False)
            m.set_decode_graphs(graphs)
            t = m.prefill(prompt)
            ls = m.logits().astype(np.float64)
            toks, logits = [t], []
            for _ in range(128):
                t = m.decode(t)
                toks.append(t)
                logits.append(m.logits())
            runs[graphs] = (toks, np.stack(logits).astype(np.float64), ls)
    err = np.abs(lb - ls).max() / np.abs(ls).max()
    top2 = np.sort(ls)[-2:]
    print(f"batched vs serial prefill: rel err {err:.3e}, serial top-2 margin {top2[1] - top2[0]:.3e}")
    assert err <= 2e-2
    if top2[1] - top2[0] > 2 * np.abs(lb - ls).max():
        assert tb == runs[False][0][0]
    (tg, lg, _), (te, le, _) = runs[True], runs[False]
    step_err = np.abs(lg - le).max(axis=1) / np.abs(le).max(axis=1)
    print("graph vs eager decode: max rel logit err", step_err.max())
    assert tg == te
    assert step_err.max() <= 1e-4
