"""QwenTokenizer parity (chat.cpp:207-529) and the ChatML / CLI contract.

The tokenizer is host code in libhipllm.so, so these run without a GPU:

* against tests/golden/tokenizer_golden.json, written by the reference's own
  QwenTokenizer (chat.cpp compiled from its sources into
  oracle/_ref/ref_tokenizer; see tests/golden/make_tokenizer_golden.py): ids,
  encode errors and pre-tokenizer pieces of 237 texts in both pre-tokenizer
  modes, and decode_piece / is_special of every id;
* against the live reference harness, where it is built, on fresh random
  texts;
* by what byte-level BPE fixes regardless of the reference: decoding the ids
  of ordinary text gives back its bytes, pieces tile the text, and a merge
  table that contains every pair merges a piece into one token.
"""

from __future__ import annotations

import json
import pathlib
import random
import subprocess
import unicodedata

import pytest

from myllm_amd import hipllm as H
from tests.tokenizer_ref import REF_TOKENIZER, SPECIALS, gpt2_byte_symbols, random_text, run_reference

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "tokenizer_golden.json"
CHAT = pathlib.Path(H.__file__).resolve().parent / "lib" / "hipllm_chat"


@pytest.fixture(scope="module")
def golden():
    return json.loads(GOLDEN.read_text())


@pytest.fixture(scope="module")
def tokenizers(golden):
    return {pre: H.QwenTokenizer(golden["vocabulary"], golden["merges"], pre) for pre in ("qwen2", "qwen35")}


@pytest.mark.parametrize("pre", ["qwen2", "qwen35"])
def test_encode_matches_reference_golden(golden, tokenizers, pre):
    tok, ref = tokenizers[pre], golden["modes"][pre]
    texts = [bytes.fromhex(t) for t in golden["texts"]]
    failures = 0
    for text, status, ids in zip(texts, ref["status"], ref["ids"]):
        if status:
            with pytest.raises(RuntimeError, match="missing piece"):
                tok.encode(text)
            failures += 1
        else:
            assert tok.encode(text) == ids, text
    assert failures >= 2  # the texts holding the byte without a symbol


@pytest.mark.parametrize("pre", ["qwen2", "qwen35"])
def test_pieces_match_reference_golden(golden, tokenizers, pre):
    tok, ref = tokenizers[pre], golden["modes"][pre]
    for text_hex, pieces in zip(golden["texts"], ref["pieces"]):
        text = bytes.fromhex(text_hex)
        assert tok.pieces(text) == [tuple(p) for p in pieces], text


def test_modes_differ_only_where_marks_attach(golden):
    """qwen35 attaches combining marks to letter runs; qwen2 does not. The
    fixture must exercise the difference, or the mode switch is unpinned."""
    a, b = golden["modes"]["qwen2"]["pieces"], golden["modes"]["qwen35"]["pieces"]
    differ = [bytes.fromhex(t) for t, p, q in zip(golden["texts"], a, b) if p != q]
    assert len(differ) >= 5
    for t in differ:
        chars = t.decode("utf-8", errors="replace")
        assert any(unicodedata.category(c).startswith("M") for c in chars), t


@pytest.mark.parametrize("pre", ["qwen2", "qwen35"])
def test_decode_and_special_match_reference_golden(golden, tokenizers, pre):
    tok, ref = tokenizers[pre], golden["modes"][pre]
    for i, (sp, dec) in enumerate(zip(ref["special"], ref["decoded"])):
        assert tok.is_special(i) == bool(sp), i
        assert tok.decode_piece(i) == bytes.fromhex(dec), i
    assert tok.id("<|im_end|>") == ref["im_end"]
    assert tok.id("</s>") == ref["slash_s"]
    assert tok.decode_piece(-1) == b"" and tok.decode_piece(len(ref["special"])) == b""
    assert tok.id("no such token") == -1


def test_duplicate_vocabulary_entry_keeps_first_id(golden, tokenizers):
    voc = golden["vocabulary"]
    dup = voc[-1]
    assert voc.index(dup) < len(voc) - 1
    assert tokenizers["qwen2"].id(dup) == voc.index(dup)


def test_special_tokens_split_longest_first(tokenizers, golden):
    tok = tokenizers["qwen2"]
    voc = golden["vocabulary"]
    assert tok.encode("<|x|>y|>") == [voc.index("<|x|>y|>")]
    assert tok.encode("<|x|>y")[0] == voc.index("<|x|>")
    assert tok.encode("<||>") == [voc.index("<||>")]
    assert not tok.is_special(voc.index("<|>"))


@pytest.mark.skipif(not REF_TOKENIZER.exists(), reason="reference tokenizer harness not built")
@pytest.mark.parametrize("pre", ["qwen2", "qwen35"])
def test_encode_matches_live_reference_on_random_texts(golden, tokenizers, pre):
    rng = random.Random(hash(pre) & 0xffff)
    texts = [random_text(rng, max_len=40) for _ in range(1500)]
    ref = run_reference(golden["vocabulary"], golden["merges"], pre, texts)
    tok = tokenizers[pre]
    for text, status, ids, pieces in zip(texts, ref["status"], ref["ids"], ref["pieces"]):
        assert tok.pieces(text) == pieces, text
        if status:
            with pytest.raises(RuntimeError):
                tok.encode(text)
        else:
            assert tok.encode(text) == ids, text


def test_ordinary_text_round_trips(tokenizers):
    """Byte-level BPE loses nothing: decode(encode(t)) == t for any bytes the
    vocabulary can spell (every byte but 0x01 here), malformed UTF-8
    included."""
    rng = random.Random(7)
    tok = tokenizers["qwen35"]
    for _ in range(400):
        t = random_text(rng, max_len=60).replace(b"\x01", b"")
        for s in SPECIALS:
            t = t.replace(s.encode(), b"")
        assert tok.decode(tok.encode(t)) == t, t


def test_pieces_tile_the_text(tokenizers):
    rng = random.Random(11)
    for pre, tok in tokenizers.items():
        for _ in range(300):
            t = random_text(rng, max_len=50)
            p = tok.pieces(t)
            assert all(b < e for b, e in p)
            bounds = [0] + [e for _, e in p]
            assert [b for b, _ in p] == bounds[:-1] and bounds[-1] == len(t)


def test_full_merge_table_gives_one_token_per_piece():
    """With every prefix-extending merge present, a piece merges into exactly
    its own vocabulary entry, and ranks decide between overlapping merges:
    "aaa" with only "a a" gives ["aa", "a"] (leftmost first)."""
    sym = gpt2_byte_symbols()
    voc = list(sym)
    merges = []
    word = [sym[b] for b in b"hello"]
    for i in range(1, len(word)):
        merges.append(f"{''.join(word[:i])} {word[i]}")
        voc.append("".join(word[:i + 1]))
    merges.append("a a")
    voc.append("aa")
    tok = H.QwenTokenizer(voc, merges, "qwen2")
    assert tok.encode("hello") == [voc.index("hello")]
    assert tok.encode("aaa") == [voc.index("aa"), voc.index("a")]
    assert tok.encode("aaaa") == [voc.index("aa")] * 2


def test_chat_prompt_is_chatml():
    assert H.chat_prompt("S", "U") == ("<|im_start|>system\nS<|im_end|>\n<|im_start|>user\nU<|im_end|>\n"
                                       "<|im_start|>assistant\n")


# ---------------------------------------------------------------- chat CLI

def _chat(args, cwd, stdin=""):
    return subprocess.run([str(CHAT), *args], cwd=cwd, input=stdin, capture_output=True, text=True, timeout=60)


@pytest.mark.skipif(not CHAT.exists(), reason="hipllm_chat not built")
def test_cli_option_errors(tmp_path):
    """run_cli / parse_options (chat.cpp:596-653, 998-1017): help, usage on an
    incomplete command line, unknown options, the kernel-profile
    constraints, profile path escape, and the missing CPU backend. None of
    these reaches a GPU call."""
    r = _chat(["--help"], tmp_path)
    assert r.returncode == 0 and "--model MODEL.gguf" in r.stderr and "--gpu" in r.stderr
    r = _chat([], tmp_path)
    assert r.returncode == 1 and r.stderr.startswith("Usage:")
    r = _chat(["--model", "m.gguf", "--tokens", "0"], tmp_path)
    assert r.returncode == 1 and r.stderr.startswith("Usage:")
    r = _chat(["--model", "m.gguf", "--bogus"], tmp_path)
    assert r.returncode == 1 and "chat: unknown option: --bogus" in r.stderr
    r = _chat(["--model"], tmp_path)
    assert r.returncode == 1 and "chat: missing value for --model" in r.stderr
    r = _chat(["--model", "m.gguf", "--metal-kernel-profile"], tmp_path)
    assert r.returncode == 1 and "--metal-kernel-profile requires --gpu" in r.stderr
    r = _chat(["--model", "m.gguf", "--gpu", "--kernel-profile", "--no-profile"], tmp_path)
    assert r.returncode == 1 and "cannot be combined with --no-profile" in r.stderr
    r = _chat(["--model", "m.gguf", "--profile-csv", "../x.csv"], tmp_path)
    assert r.returncode == 1 and "cannot escape the output directory" in r.stderr
    r = _chat(["--model", "m.gguf", "--profile-csv", ""], tmp_path)
    assert r.returncode == 1 and "cannot be empty" in r.stderr
    r = _chat(["--model", "m.gguf", "--profile-csv", "sub/p.csv"], tmp_path)
    assert r.returncode == 1 and "pass --gpu" in r.stderr
    assert (tmp_path / "output" / "sub").is_dir()  # created before the model loads, as in the reference
    r = _chat(["--model", str(tmp_path / "absent.gguf"), "--gpu", "--no-profile"], tmp_path)
    assert r.returncode == 1 and "[chat] loading model:" in r.stderr and r.stderr.strip().splitlines()[-1].startswith(
        "chat: ")
