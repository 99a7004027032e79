"""CPU checks of the drop-in boundary (no GPU calls).

* libhipllm.so and libhipllm_tools.so load and export every function their
  headers declare.
* The streaming GGUF reader (used through hipllm_inspect_gguf, which needs no
  GPU) accepts the synthetic schema and rejects malformed files with the
  reference's error kinds (metal_model.cpp:451-562, 690-696, 960-976).
"""

from __future__ import annotations

import pathlib
import struct

import pytest

from myllm_amd import _native, hipllm, synth

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("header,loader", [("hipllm.h", _native.hipllm), ("hipllm_tools.h", _native.tools)])
def test_library_exports_every_declared_symbol(header, loader):
    names = hipllm.header_functions((ROOT / "include" / header).read_text())
    assert len(names) >= 5
    lib = loader()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    names = set(hipllm.header_functions((ROOT / "include" / "hipllm.h").read_text()))
    assert names == set(hipllm.SIGNATURES), names ^ set(hipllm.SIGNATURES)


def test_inspect_synthetic_model(golden_model):
    path, _ = golden_model("tiny")
    cfg = hipllm.inspect_gguf(path)
    s = synth.SHAPES["tiny"]
    assert cfg["architecture"] == "qwen2"
    assert (cfg["layer_count"], cfg["embedding_size"], cfg["feed_forward_size"]) == (s.layers, s.hidden, s.ffn)
    assert (cfg["attention_head_count"], cfg["kv_head_count"], cfg["head_size"]) == (s.heads, s.kv_heads, 64)
    assert cfg["vocabulary_size"] == s.vocab and cfg["eos_token_id"] == s.eos_token_id
    assert cfg["rope_theta"] == 1e6 and abs(cfg["norm_epsilon"] - 1e-6) < 1e-12
    assert cfg["stored_weight_bytes"] > 0


def _corrupt(src: pathlib.Path, dst: pathlib.Path, edit) -> pathlib.Path:
    data = bytearray(src.read_bytes())
    edit(data)
    dst.write_bytes(bytes(data))
    return dst


def test_reader_rejects_malformed_files(golden_model, tmp_path):
    path, _ = golden_model("tiny")
    cases = {
        "magic": lambda d: d.__setitem__(slice(0, 4), b"GGUX"),
        "version": lambda d: d.__setitem__(slice(4, 8), struct.pack("<I", 7)),
        "truncated": lambda d: d.__delitem__(slice(200, len(d))),
        "tensor_count": lambda d: d.__setitem__(slice(8, 16), struct.pack("<Q", 10 ** 6)),
    }
    for name, edit in cases.items():
        bad = _corrupt(path, tmp_path / f"{name}.gguf", edit)
        with pytest.raises(RuntimeError):
            hipllm.inspect_gguf(bad)
    with pytest.raises(RuntimeError):
        hipllm.inspect_gguf(tmp_path / "missing.gguf")


def test_reader_rejects_bad_tensor_type(golden_model, tmp_path):
    path, _ = golden_model("tiny")
    data = bytearray(path.read_bytes())
    # The first tensor info follows the metadata; find token_embd's type field
    # (name, n_dims, dims..., type) and set an unknown type id.
    name = b"token_embd.weight"
    at = data.index(name) + len(name)
    ndims = struct.unpack_from("<I", data, at)[0]
    type_at = at + 4 + 8 * ndims
    struct.pack_into("<I", data, type_at, 99)
    bad = tmp_path / "badtype.gguf"
    bad.write_bytes(bytes(data))
    with pytest.raises(RuntimeError, match="unsupported GGUF tensor type"):
        hipllm.inspect_gguf(bad)


def tensor_info(data: bytearray, name: str) -> dict:
    """Byte positions of one tensor-info record of a GGUF file: the name
    string (u64 length + bytes), n_dims u32, dims u64 x n_dims, type u32,
    offset u64."""
    key = name.encode()
    at = data.index(struct.pack("<Q", len(key)) + key)
    name_at = at + 8
    nd_at = name_at + len(key)
    nd = struct.unpack_from("<I", data, nd_at)[0]
    dims_at = nd_at + 4
    dims = list(struct.unpack_from(f"<{nd}Q", data, dims_at))
    return {"name_at": name_at, "dims_at": dims_at, "dims": dims, "type_at": dims_at + 8 * nd}


def edited(path: pathlib.Path, dst: pathlib.Path, edit) -> pathlib.Path:
    data = bytearray(path.read_bytes())
    edit(data)
    dst.write_bytes(bytes(data))
    return dst


def test_reader_rejects_duplicate_tensor(golden_model, tmp_path):
    # Renaming blk.1's attention norm to blk.0's (same length) leaves two
    # records of one name (gguf_reader.cpp, tensor index).
    path, _ = golden_model("tiny")

    def dup(d):
        t = tensor_info(d, "blk.1.attn_norm.weight")
        d[t["name_at"]:t["name_at"] + 5] = b"blk.0"

    with pytest.raises(RuntimeError, match="duplicate GGUF tensor: blk.0.attn_norm.weight"):
        hipllm.inspect_gguf(edited(path, tmp_path / "dup.gguf", dup))


def test_reader_rejects_row_not_block_aligned(golden_model, tmp_path):
    # A Q4_K tensor whose row length (dims[0]) is not a multiple of its
    # 256-value block (metal_model.cpp:417-448 row-byte rule).
    path, _ = golden_model("tiny")

    def misalign(d):
        t = tensor_info(d, "blk.0.attn_q.weight")
        struct.pack_into("<Q", d, t["dims_at"], t["dims"][0] - 16)

    with pytest.raises(RuntimeError, match="row is not block aligned"):
        hipllm.inspect_gguf(edited(path, tmp_path / "misaligned.gguf", misalign))
