"""The chat front end end to end on the GPU: chat::run and the chat command
over synthetic models that carry the tokenizer tables of
tests/golden/tokenizer_golden.json (vocabulary and merges written by the
reference's own tokenizer harness).

* hipllm_run (chat.cpp:831-878) gives the tokens of the Python greedy loop
  over prefill / decode, honours stop tokens and the sequence limit, and
  raises the reference's validation errors;
* make_stop_tokens (chat.cpp:708-726) is eos, <|im_end|>, </s>, then every
  special id in order;
* hipllm_chat --gpu (chat.cpp:998-1040) prints, byte for byte, the transcript
  that the tokenizer, ChatML and chat::run give for the same turns, for the
  dense and the MoE backend, and writes the profile CSVs under output/.
"""

from __future__ import annotations

import dataclasses
import json
import pathlib
import re
import subprocess

import numpy as np
import pytest

from myllm_amd import synth
from myllm_amd import hipllm as H
from myllm_amd.hipllm import HipLLM, generate

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "tokenizer_golden.json"
CHAT = pathlib.Path(H.__file__).resolve().parent / "lib" / "hipllm_chat"
SYSTEM = "You are a concise and helpful assistant."


@pytest.fixture(scope="module")
def tables():
    g = json.loads(GOLDEN.read_text())
    return g["vocabulary"], g["merges"]


@pytest.fixture(scope="module")
def chat_models(tmp_path_factory, tables):
    vocab, merges = tables
    d = tmp_path_factory.mktemp("chat")
    eos = vocab.index("<|endoftext|>")
    dense = dataclasses.replace(synth.SHAPES["tiny"], name="tiny-chat", vocab=len(vocab), context=256,
                                eos_token_id=eos)
    p = synth.write_qwen2(d / "dense-raw.gguf", dense, types=synth.tiny_all_types(), seed=21)
    dense_path = synth.add_tokenizer(p, d / "dense.gguf", vocab, merges, "qwen2")
    moe = dataclasses.replace(synth.MOE_SHAPES["moe-tiny"], name="moe-chat", vocab=len(vocab), eos_token_id=eos)
    p = synth.write_qwen35moe(d / "moe-raw.gguf", moe, seed=22)
    moe_path = synth.add_tokenizer(p, d / "moe.gguf", vocab, merges, "qwen35")
    return {"dense": dense_path, "moe": moe_path}


def test_tokenizer_tables_reach_the_model(cuda, chat_models, tables):
    vocab, merges = tables
    with HipLLM(chat_models["moe"], 64) as m:
        assert m.vocabulary == [v.encode() for v in vocab] and m.merges == [v.encode() for v in merges]
        assert m.tokenizer_pre == "qwen35"
        tok = H.QwenTokenizer.from_model(m)
        ref = H.QwenTokenizer(vocab, merges, "qwen35")
        text = "مُحَمَّدٌ It's 42 tokens\n\n  z͑a"
        assert tok.encode(text) == ref.encode(text)


def test_stop_tokens(cuda, chat_models, tables):
    vocab, _ = tables
    with HipLLM(chat_models["dense"], 64) as m:
        tok = H.QwenTokenizer.from_model(m)
        stops = H.stop_tokens(m, tok)
    special = [i for i, v in enumerate(vocab) if len(v.encode()) >= 4 and v.startswith("<|") and v.endswith("|>")]
    expect = [vocab.index("<|endoftext|>"), vocab.index("<|im_end|>"), vocab.index("</s>")]
    expect += [i for i in special if i not in expect]
    assert stops == expect


@pytest.mark.parametrize("kind", ["dense", "moe"])
def test_run_matches_greedy_loop(cuda, chat_models, kind):
    with HipLLM(chat_models[kind], 96) as m:
        tok = H.QwenTokenizer.from_model(m)
        ids = tok.encode(H.chat_prompt(SYSTEM, "Hello there, how are you?"))
        loop = generate(m, ids, 12)
        seen = []
        toks, stats, line = H.run(m, ids, 12, (), seen.append)
        assert toks == loop == seen
        assert stats["prompt_tokens"] == len(ids) and stats["generated_tokens"] == 12
        assert stats["decode_steps"] == 11 and not stats["stopped"] and stats["used_gpu"]
        assert stats["memory"]["weight_bytes"] > 0
        assert stats["has_expert_cache_stats"] == (kind == "moe")
        assert line.startswith("[chat] generation_stats mode=gpu-kv prompt_tokens=")
        assert line.endswith(" stopped=false") and ("expert_cache_hit_rate=" in line) == (kind == "moe")
        # A stop token ends generation before it is emitted.
        toks, stats, _ = H.run(m, ids, 12, [loop[3]])
        assert toks == loop[:loop.index(loop[3])] and stats["stopped"]
        # The sequence limit caps generation at max_sequence - prompt length.
        toks, stats, _ = H.run(m, (ids * 4)[:90], 50)
        assert len(toks) == 6 and stats["decode_steps"] == 5
        with pytest.raises(ValueError, match="at least one initial token"):
            H.run(m, [], 4)
        with pytest.raises(ValueError, match="max_new_tokens > 0"):
            H.run(m, ids, 0)
        with pytest.raises(ValueError, match="no room for generated tokens"):
            H.run(m, list(range(96)), 4)


def _expected_transcript(path, turns, tokens, kind):
    """stdout the chat command must print for `turns`, from the library's
    tokenizer, ChatML and chat::run (chat.cpp:799-829, 900-964)."""
    out = b"Enter text (/exit to quit, /clear is accepted):\n"
    prompts = []
    with HipLLM(path) as m:
        tok = H.QwenTokenizer.from_model(m)
        stops = H.stop_tokens(m, tok)
        for t in turns:
            out += b"> "
            if t in ("/exit", "/quit"):
                break
            if t == "/clear":
                out += b"[conversation cleared]\n"
                continue
            ids = tok.encode(H.chat_prompt(SYSTEM, t))
            prompts.append(ids)
            gen, _, _ = H.run(m, ids, tokens, stops)
            out += tok.decode(gen) + b"\n"
    return out + b"\n", prompts


@pytest.mark.parametrize("kind", ["dense", "moe"])
def test_chat_command_transcript(cuda, chat_models, kind, tmp_path):
    turns = ["Hello world", "/clear", "It's 42 — 中文 and مُحَمَّد", "/exit"]
    expect, prompts = _expected_transcript(chat_models[kind], turns, 10, kind)
    r = subprocess.run([str(CHAT), "--gpu", "--model", str(chat_models[kind]), "--tokens", "10", "--no-profile"],
                       input=("\n".join(turns) + "\n").encode(), capture_output=True, cwd=tmp_path, timeout=300)
    err = r.stderr.decode(errors="replace")
    assert r.returncode == 0, err
    assert r.stdout == expect
    backend = "HIP MoE device=" if kind == "moe" else "HIP device="
    assert re.search(r"\[chat\] layers=\d+ embedding=\d+ vocab=\d+ merges=\d+ context=\d+ capacity=\d+ backend=" +
                     re.escape(backend), err)
    got = [list(map(int, l.split("ids=")[1].split())) for l in err.splitlines() if l.startswith("[chat] prompt_tokens=")]
    assert got == prompts
    stats = [l for l in err.splitlines() if "generation_stats" in l]
    assert len(stats) == 2 and all("mode=gpu-kv" in l for l in stats)
    assert all(("expert_cache_requests=" in l) == (kind == "moe") for l in stats)


def test_chat_command_profile_files(cuda, chat_models, tmp_path):
    r = subprocess.run([str(CHAT), "--gpu", "--model", str(chat_models["dense"]), "--tokens", "4",
                        "--profile-csv", "run/prof.csv", "--kernel-profile"],
                       input=b"hi\n/exit\n", capture_output=True, cwd=tmp_path, timeout=300)
    err = r.stderr.decode(errors="replace")
    assert r.returncode == 0, err
    assert "[chat] profile_csv=output/run/prof.csv" in err
    for name in ("prof.csv", "prof_metal_commands.csv", "prof_metal_kernels.csv", "prof_metal_ops.csv"):
        f = tmp_path / "output" / "run" / name
        assert f.exists() and f.stat().st_size > 0, name
    rows = (tmp_path / "output" / "run" / "prof.csv").read_text().splitlines()
    assert len(rows) > 2 and any("prefill.gpu_resident" in l for l in rows)


def test_chat_command_rejects_model_without_tokenizer(cuda, tmp_path):
    path = synth.write_qwen2(tmp_path / "plain.gguf", synth.SHAPES["tiny"], types=synth.tiny_all_types(), seed=3)
    r = subprocess.run([str(CHAT), "--gpu", "--model", str(path), "--no-profile"], input=b"/exit\n",
                       capture_output=True, cwd=tmp_path, timeout=300)
    assert r.returncode == 1
    assert "chat: model does not contain Qwen tokenizer vocabulary/merges" in r.stderr.decode()
    np.testing.assert_equal(r.stdout, b"")
