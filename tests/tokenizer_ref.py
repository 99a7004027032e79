"""Helpers for the tokenizer parity tests: the reference tokenizer harness
(oracle/_ref/ref_tokenizer, chat.cpp's QwenTokenizer compiled from the
reference sources) and the inputs shared by the golden script and the tests.

Test infrastructure only.
"""

from __future__ import annotations

import pathlib
import random
import struct
import subprocess
import tempfile

ROOT = pathlib.Path(__file__).resolve().parents[1]
REF_TOKENIZER = ROOT / "oracle" / "_ref" / "ref_tokenizer"


def gpt2_byte_symbols() -> list:
    """GPT-2's byte -> symbol map (the published bytes_to_unicode table),
    written independently of the product code: printable Latin-1 bytes map
    to themselves, the others to 256, 257, ... in byte order."""
    keep = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    out, extra = [], 0
    for b in range(256):
        if b in keep:
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


def _string(s) -> bytes:
    data = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<I", len(data)) + data


def run_reference(vocabulary, merges, pre: str, texts) -> dict:
    """Runs oracle/_ref/ref_tokenizer; returns ids / status / pieces per text,
    and is_special / decode_piece per vocabulary id."""
    blob = bytearray()
    for table in (vocabulary, merges):
        blob += struct.pack("<I", len(table))
        for s in table:
            blob += _string(s)
    blob += _string(pre)
    blob += struct.pack("<I", len(texts))
    for t in texts:
        blob += _string(t)
    with tempfile.TemporaryDirectory() as d:
        src, dst = pathlib.Path(d) / "in.bin", pathlib.Path(d) / "out.bin"
        src.write_bytes(bytes(blob))
        subprocess.run([str(REF_TOKENIZER), str(src), str(dst)], check=True, timeout=600)
        out = dst.read_bytes()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, out, pos)
        pos += struct.calcsize(fmt)
        return v

    status, ids, pieces = [], [], []
    for _ in texts:
        (st,) = take("<i")
        (n,) = take("<I")
        ids.append(list(take(f"<{n}i")) if n else [])
        status.append(st)
        (m,) = take("<I")
        flat = take(f"<{2 * m}Q") if m else ()
        pieces.append([(flat[2 * i], flat[2 * i + 1]) for i in range(m)])
    special, decoded = [], []
    for _ in vocabulary:
        (sp,) = take("<B")
        (n,) = take("<I")
        decoded.append(out[pos:pos + n])
        pos += n
        special.append(sp)
    im_end, slash_s = take("<ii")
    assert pos == len(out)
    return dict(status=status, ids=ids, pieces=pieces, special=special, decoded=decoded, im_end=im_end,
                slash_s=slash_s)


# Codepoints of every class the pre-tokenizer separates, in both modes:
# ASCII letters / digits / punctuation / whitespace, Latin-1 and Greek
# letters, combining marks (Latin, Hebrew, Arabic), Arabic-Indic and
# fullwidth digits, Devanagari, Thai, Hangul, CJK, kana, emoji, the Unicode
# spaces (NBSP, ogham, en quad .. hair space, line / paragraph separators,
# narrow NBSP, medium math space, ideographic space), and the edges of the
# class ranges.
ALPHABET = (
    list("abcXYZ019 '\t\n\r\f\v.,;:!?-_()[]{}<>|/\\\"#$%&*+=@^`~")
    + ["é", "ß", "×", "÷", "À", "˿", "̀", "́", "ͯ", "Ͱ",
       "α", "А", "֑", "ֿ", "א", "ؐ", "ا", "ً", "٠", "٩",
       "ٰ", "۰", "ܑ", "ܰ", "क", "ा", "०", "ก", "ა", "ᄀ",
       "᪰", "᷀", "⃐", "あ", "ア", "中", "文", "가", "豈", "︀",
       "︠", "０", "９", " ", " ", " ", " ", " ", " ", " ",
       " ", "　", "­", "¡", "\U0001f600", "\U00020000", "\U000323af", "\U000e0100"]
)

SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|x|>", "<|x|>y|>", "<||>"]


def random_text(rng: random.Random, max_len: int = 24) -> bytes:
    """A random string over ALPHABET, sometimes with a special token, an
    apostrophe contraction or a raw malformed byte spliced in."""
    parts = []
    for _ in range(rng.randint(0, max_len)):
        r = rng.random()
        if r < 0.04:
            parts.append(rng.choice(SPECIALS).encode())
        elif r < 0.08:
            parts.append(rng.choice(["'s", "'T", "'re", "'VE", "'ll", "'d", "'M", "'x"]).encode())
        elif r < 0.10:
            parts.append(bytes([rng.choice([0x80, 0xbf, 0xc3, 0xe4, 0xf0, 0xff, 0xa0, 0x01])]))
        else:
            parts.append(rng.choice(ALPHABET).encode("utf-8"))
    return b"".join(parts)
