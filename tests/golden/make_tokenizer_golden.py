"""Writes tests/golden/tokenizer_golden.json from the reference's own tokenizer.

Run in a container that holds the reference sources (``make -C oracle ref``
builds oracle/_ref/ref_tokenizer from chat.cpp first). No real Qwen GGUF is
available, so the vocabulary is synthetic but built the way a byte-level BPE
vocabulary is: the 256 GPT-2 byte symbols plus the results of merges learned
on a small multilingual corpus (greedy most-frequent-pair BPE), plus special
tokens. It carries deliberate edge cases:

* the byte 0x01 has no symbol in the vocabulary (encoding it must fail);
* the merge "Ġ Ġ" yields "ĠĠ", which is not a vocabulary entry (per-symbol
  fallback), while "ĠĠ Ġ" yields "ĠĠĠ", which is;
* malformed merge lines (no separator, empty right operand), a line with a
  leading space, a repeated merge at a later rank, and a duplicated
  vocabulary entry;
* special tokens where one is a prefix of another ("<|x|>" / "<|x|>y|>"), the
  4-byte "<||>", and the 3-byte "<|>", which is not special; "</s>" as an
  ordinary entry.

For each pre-tokenizer mode ("qwen2", "qwen35") the file holds the ids,
encode status and piece ranges of every text, and is_special / decode_piece of
every id. Texts and decoded pieces are stored as hex, since some are not
UTF-8.

Usage: python tests/golden/make_tokenizer_golden.py
"""

from __future__ import annotations

import collections
import json
import pathlib
import random
import sys

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from tests.tokenizer_ref import REF_TOKENIZER, gpt2_byte_symbols, random_text, run_reference  # noqa: E402

CORPUS = """
The quick brown fox jumps over the lazy dog. It's what we're told: they'll say I'm fine, you've seen it, he'd know.
THE QUICK BROWN FOX! Don't stop; won't stop... can't stop?! "Quoted" (parenthesised) [bracketed] {braced}.
def main(argc, argv):\n    for i in range(10):\n        print(f"{i:04d} -> {i * i}")\n    return 0\n
int main(int argc, char** argv) {\r\n\treturn argc > 1 ? atoi(argv[1]) : 42;\r\n}\r\n
Numbers 1234567890 and 3.14159, 2,718 and 1e-9; prices $19.99, 50% off, #1 ranked @home.
Ünïcödé façade naïve café résumé Straße Ærø œuvre. Ελληνικά κείμενα. Русский текст здесь.
中文文本处理与分词。今天天气很好，我们去公园散步吧！日本語のテキスト、カタカナとひらがな。
한국어 텍스트 처리. 안녕하세요 여러분. สวัสดีครับ ภาษาไทย. ქართული ენა.
مرحبا بالعالم، هذا نص عربي مع تشكيل: مُحَمَّدٌ وَكِتَابٌ. الأرقام ٠١٢٣٤٥٦٧٨٩ و ۰۱۲۳.
שָׁלוֹם עוֹלָם. नमस्ते दुनिया, यह हिंदी पाठ है। संख्या ०१२३४५६७८९.
Combining marks: é à ö ñ and zalgo z͑͒a͓l͔g͕o.
Emoji 😀😃😄 👍🏽 ❤️ and symbols ™ © ® ± × ÷ → ← ∞ ≠ ≤ ≥.
Whitespace   runs\t\ttabs\n\n\nnewlines  nbsp　ideographic em space   trailing   \n
Full-width ０１２３ ＡＢＣ and half-width 0123 ABC. URLs https://example.com/path?q=1&r=2#frag.
""" * 3


def train_bpe(text: str, merges: int) -> list:
    """Greedy byte-level BPE: repeatedly merge the most frequent adjacent pair
    (ties broken by the pair itself) over whitespace-separated words, each
    word carrying its leading space as GPT-2 tokenizers do."""
    sym = gpt2_byte_symbols()
    words = collections.Counter()
    for raw in text.replace("\n", " \n ").split(" "):
        if raw:
            words[tuple(sym[b] for b in (" " + raw).encode("utf-8"))] += 1
    vocab = dict(words)
    out = []
    for _ in range(merges):
        pairs = collections.Counter()
        for w, c in vocab.items():
            for a, b in zip(w, w[1:]):
                pairs[(a, b)] += c
        if not pairs:
            break
        best = max(pairs.items(), key=lambda kv: (kv[1], kv[0]))[0]
        out.append(best)
        merged = {}
        for w, c in vocab.items():
            nw, i = [], 0
            while i < len(w):
                if i + 1 < len(w) and (w[i], w[i + 1]) == best:
                    nw.append(w[i] + w[i + 1])
                    i += 2
                else:
                    nw.append(w[i])
                    i += 1
            merged[tuple(nw)] = merged.get(tuple(nw), 0) + c
        vocab = merged
    return out


def build_tables():
    sym = gpt2_byte_symbols()
    learned = train_bpe(CORPUS, 900)
    merges = [f"{a} {b}" for a, b in learned]
    vocabulary = [s for b, s in enumerate(sym) if b != 0x01]
    seen = set(vocabulary)
    for a, b in learned:
        if a + b not in seen:
            seen.add(a + b)
            vocabulary.append(a + b)
    sp = sym[ord(" ")]
    if sp + sp in seen:
        vocabulary.remove(sp + sp)
        seen.discard(sp + sp)
    merges = [m for m in merges if m != f"{sp} {sp}"]
    merges[5:5] = [f"{sp} {sp}", f"{sp}{sp} {sp}"]
    if sp * 3 not in seen:
        vocabulary.append(sp * 3)
    merges += ["nospace", "trailing ", f" {sym[ord('a')]} {sym[ord('b')]}", merges[0]]
    vocabulary += ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|x|>", "<|x|>y|>", "<||>", "<|>", "</s>",
                   vocabulary[300]]
    return vocabulary, merges


TEXTS = [
    "", " ", "  ", "a", "Hello world", "Hello  world", "Hello   world  ", "\n", "\r\n", " \n \n x",
    "It's we're they'll I'M YOU'VE he'd don't", "'s'S'sx", "x's", "''", "'", "rock'n'roll",
    "1234567890", "3.14159", "x1y2", "$19.99", "٠١٢ ۰۱ ०१ ０１",
    "naïve café é", "á̂b", " ́abc", "́", "מִשְׁפָּט", "مُحَمَّدٌ", "नमस्ते",
    "中文文本处理", "日本語のテキスト", "안녕하세요", "สวัสดี", "ქართული", "Ελληνικά", "Русский",
    "😀😃 👍🏽 ❤️", "a b", "a　b", "a  b", "tab\t\tx", "\f\v x",
    "line\r\rbreak", "  !!!\n\n", " !x", "!!", "...\r\n", " .", "a\x01b", "\x01",
    b"\x80\xff bad", b"\xc3", b"\xe4\xb8", b"\xf0\x9f\x98", b"\xc0\x80", b"\xa0x", b"\xc3\xa9\xcc",
    "<|im_start|>system\nYou are helpful.<|im_end|>\n<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n",
    "<|x|>y|>", "<|x|>y", "<|x|><|x|>", "<||>", "<|>", "<|", "|>", "a<|endoftext|>b", "</s>",
    "<|im_end", "x<|im_end|>", "<|unknown|>",
    "def f(x):\n    return x * 2\n", "int main() {\r\n\treturn 0;\r\n}", "https://example.com/a?b=1&c=2",
    "   leading", "trailing   ", "   ", "\n\n\n", " \t\n",
]


def main() -> None:
    if not REF_TOKENIZER.exists():
        raise SystemExit(f"{REF_TOKENIZER} is missing: run `make -C oracle ref` where the reference sources are")
    vocabulary, merges = build_tables()
    rng = random.Random(20261202)
    texts = [t.encode("utf-8") if isinstance(t, str) else t for t in TEXTS]
    texts += [random_text(rng) for _ in range(160)]
    golden = {"vocabulary": vocabulary, "merges": merges, "texts": [t.hex() for t in texts], "modes": {}}
    for pre in ("qwen2", "qwen35"):
        r = run_reference(vocabulary, merges, pre, texts)
        golden["modes"][pre] = {
            "status": r["status"], "ids": r["ids"], "pieces": r["pieces"], "special": r["special"],
            "decoded": [d.hex() for d in r["decoded"]], "im_end": r["im_end"], "slash_s": r["slash_s"],
        }
    out = HERE / "tokenizer_golden.json"
    out.write_text(json.dumps(golden, ensure_ascii=False, separators=(",", ":")))
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(vocabulary)} tokens, {len(merges)} merges, "
          f"{len(texts)} texts)")


if __name__ == "__main__":
    main()
