"""Pins the CPU oracle (oracle/liboracle.so, a restatement of CPULLM).

* Against the golden vectors produced by the reference's own compiled CPULLM
  (tests/golden): bit-exact logits for every step of the tiny model, greedy
  tokens and top-64 logits for the Qwen2.5-0.5B-shaped model.
* Against oracle/_ref (the reference compiled from its sources) on a fresh
  seed, when that binary is present.
* The contract checks of CPULLM::prefill/decode (cpu_llm.cpp:978-1046): the
  error type for each precondition.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle


def test_tiny_bit_exact_against_reference_golden(golden_model):
    path, g = golden_model("tiny")
    m = oracle.CpuOracle(path, int(g["max_sequence"]))
    logits = []
    toks = oracle.generate(m, g["prompt"], len(g["tokens"]), logits_sink=logits.append)
    assert toks == g["tokens"].tolist()
    got = np.stack(logits)
    assert got.shape == g["logits"].shape
    # Same bits, every step.
    assert np.array_equal(got.view(np.uint32), g["logits"].view(np.uint32))


def test_qwen05b_tokens_and_top_logits_against_reference_golden(golden_model):
    path, g = golden_model("qwen2.5-0.5b")
    m = oracle.CpuOracle(path, int(g["max_sequence"]))
    logits = []
    toks = oracle.generate(m, g["prompt"], len(g["tokens"]), logits_sink=logits.append)
    assert toks == g["tokens"].tolist()
    got = np.stack(logits)
    top = np.take_along_axis(got, g["top_index"], axis=1)
    assert np.array_equal(top.view(np.uint32), g["top_logit"].view(np.uint32))


@pytest.mark.skipif(not oracle.REF_BIN.exists(), reason="oracle/_ref not built (reference sources absent)")
def test_oracle_matches_compiled_reference_on_fresh_seed(model_dir, tmp_path):
    from myllm_amd import synth
    shape = synth.Qwen2Shape("mini", 3, 512, 8, 2, 768, 700, 64, eos_token_id=5)
    types = dict(type_embd=synth.Q5_0, type_attn_qkv=synth.Q8_0, type_attn_out=synth.Q4_K,
                 type_ffn_gate_up=synth.Q6_K, type_ffn_down=synth.Q5_0, type_output=synth.Q4_K)
    path = synth.write_qwen2(model_dir / "mini.gguf", shape, types, seed=99)
    prompt = synth.uniform_ids(9, shape.vocab, seed=3)
    lf = tmp_path / "l.bin"
    ref = oracle.run_reference(path, prompt, 12, logits_path=lf)
    ref_logits = np.fromfile(lf, dtype=np.float32).reshape(-1, shape.vocab)
    m = oracle.CpuOracle(path)
    logits = []
    toks = oracle.generate(m, prompt, 12, logits_sink=logits.append)
    assert toks == ref["tokens"]
    assert np.array_equal(np.stack(logits).view(np.uint32), ref_logits.view(np.uint32))


def test_contract_errors(golden_model):
    path, g = golden_model("tiny")
    m = oracle.CpuOracle(path, 20)
    with pytest.raises(ValueError):
        m.decode(1)  # decode before prefill
    with pytest.raises(ValueError):
        m.prefill([])
    with pytest.raises(IndexError):
        m.prefill([1, 2, 5000])
    with pytest.raises(oracle.LengthError):
        m.prefill(list(range(21)))
    m.prefill([1, 2, 3])
    with pytest.raises(ValueError):
        m.prefill([1])  # prefill without reset
    with pytest.raises(IndexError):
        m.decode(-1)
    for _ in range(17):
        m.decode(4)
    with pytest.raises(oracle.LengthError):
        m.decode(4)
    m.reset()
    assert m.position == 0
    m.prefill([7])
    assert m.position == 1
