"""Seeded synthetic inputs: GGUF models, quantized weight matrices, prompts.

Weights are N(0, stddev) values quantized with the GGML block quantizers in
``csrc/tools`` (a restatement of ggml's reference quantizers). Models use the
qwen2 tensor schema the reference loaders require (model.cpp:861-919,
metal_model.cpp:851-910): ``token_embd``, ``output_norm``, an explicit
``output`` and twelve tensors per block.

The Q4_K_M mix is: Q4_K for attention and FFN gate/up, Q6_K for ffn_down and
the output head, Q8_0 for the embedding. Rows whose length is not a multiple
of 256 cannot hold a K-quant super-block, so they take the 32-element type of
the same family, as llama.cpp's Q4_K_M does for such tensors: Q4_K -> Q5_0 and
Q6_K -> Q8_0 (Qwen2.5-0.5B's hidden size 896 is the case in point).
"""

from __future__ import annotations

import ctypes
import dataclasses
import hashlib
import os
import pathlib

import numpy as np

from . import _native

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
BLOCK = {F32: 1, F16: 1, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}


class _Spec(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
        ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
        ("ffn", ctypes.c_uint32), ("vocab", ctypes.c_uint32),
        ("context", ctypes.c_uint32), ("eos_token_id", ctypes.c_uint32),
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float),
        ("type_embd", ctypes.c_uint32), ("type_attn_qkv", ctypes.c_uint32),
        ("type_attn_out", ctypes.c_uint32), ("type_ffn_gate_up", ctypes.c_uint32),
        ("type_ffn_down", ctypes.c_uint32), ("type_output", ctypes.c_uint32),
        ("seed", ctypes.c_uint64), ("stddev", ctypes.c_float),
        ("bias_stddev", ctypes.c_float), ("threads", ctypes.c_uint32),
    ]


@dataclasses.dataclass(frozen=True)
class Qwen2Shape:
    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    ffn: int
    vocab: int
    context: int
    rope_theta: float = 1e6
    norm_eps: float = 1e-6
    eos_token_id: int = 151645

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


SHAPES = {
    # Small shape for golden vectors and fast CPU tests.
    "tiny": Qwen2Shape("tiny", 2, 256, 4, 2, 512, 1024, 128, eos_token_id=1023),
    "qwen2.5-0.5b": Qwen2Shape("qwen2.5-0.5b", 24, 896, 14, 2, 4864, 151936, 32768),
    "qwen2.5-7b": Qwen2Shape("qwen2.5-7b", 28, 3584, 28, 4, 18944, 152064, 32768),
    "qwen2.5-14b": Qwen2Shape("qwen2.5-14b", 48, 5120, 40, 8, 13824, 152064, 32768),
}


class _MoeSpec(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "layers", "hidden", "heads", "kv_heads", "head_dim", "rotary_dim", "vocab", "context",
        "eos_token_id")] + [("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float)] + [
        (n, ctypes.c_uint32) for n in (
        "experts", "experts_used", "expert_ffn", "shared_ffn", "full_attention_interval",
        "conv_kernel", "state_size", "group_count", "time_step_rank",
        "type_embd", "type_output", "type_attn_qgate", "type_attn_kv", "type_attn_out",
        "type_ssm_qkv", "type_ssm_gate", "type_ssm_out", "type_expert_gate_up",
        "type_expert_down", "type_shared")] + [
        ("seed", ctypes.c_uint64), ("stddev", ctypes.c_float), ("small_stddev", ctypes.c_float),
        ("conv_stddev", ctypes.c_float), ("threads", ctypes.c_uint32)]


@dataclasses.dataclass(frozen=True)
class Qwen35MoeShape:
    """Text-only Qwen3.5/3.6 MoE with Gated DeltaNet layers (qwen35moe)."""
    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    vocab: int
    context: int
    experts: int
    experts_used: int
    expert_ffn: int
    shared_ffn: int
    full_attention_interval: int
    conv_kernel: int
    state_size: int
    group_count: int
    time_step_rank: int
    rope_theta: float = 1e7
    norm_eps: float = 1e-6
    eos_token_id: int = 151645

    @property
    def inner(self) -> int:
        return self.time_step_rank * self.state_size

    @property
    def qkv_width(self) -> int:
        return 2 * self.group_count * self.state_size + self.inner


MOE_SHAPES = {
    # Small shape for CPU-checkable parity: 2 DeltaNet + 2 gated-attention layers.
    "moe-tiny": Qwen35MoeShape("moe-tiny", 4, 256, 4, 2, 64, 16, 512, 256, 16, 4, 256, 256, 2, 4, 64, 2, 4,
                               eos_token_id=511),
    # Qwen3.5/3.6-35B-A3B widths with the first 4 layers (3 DeltaNet : 1 attention).
    "qwen3.5-35b-a3b-4l": Qwen35MoeShape("qwen3.5-35b-a3b-4l", 4, 2048, 16, 2, 256, 64, 151936, 4096, 256, 8, 512,
                                         512, 4, 4, 128, 16, 32),
    # The full 40-layer Qwen3.5/3.6-35B-A3B text shape.
    "qwen3.5-35b-a3b": Qwen35MoeShape("qwen3.5-35b-a3b", 40, 2048, 16, 2, 256, 64, 151936, 4096, 256, 8, 512,
                                      512, 4, 4, 128, 16, 32),
}

MOE_TYPES = dict(type_embd=Q8_0, type_output=Q6_K, type_attn_qgate=Q4_K, type_attn_kv=Q8_0,
                 type_attn_out=Q4_K, type_ssm_qkv=Q6_K, type_ssm_gate=Q4_K, type_ssm_out=Q4_K,
                 type_expert_gate_up=Q4_K, type_expert_down=Q6_K, type_shared=Q8_0)


def write_qwen35moe(path, shape: Qwen35MoeShape, seed: int = 0, stddev: float = 0.02,
                    small_stddev: float = 0.02, conv_stddev: float = 0.3, types: dict | None = None,
                    threads: int | None = None) -> pathlib.Path:
    """Writes a synthetic qwen35moe GGUF (Q4_K experts, Q6_K expert down
    projections) and returns its path."""
    t = dict(MOE_TYPES, **(types or {}))
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    spec = _MoeSpec(shape.layers, shape.hidden, shape.heads, shape.kv_heads, shape.head_dim, shape.rotary_dim,
                    shape.vocab, shape.context, shape.eos_token_id, shape.rope_theta, shape.norm_eps,
                    shape.experts, shape.experts_used, shape.expert_ffn, shape.shared_ffn,
                    shape.full_attention_interval, shape.conv_kernel, shape.state_size, shape.group_count,
                    shape.time_step_rank, t["type_embd"], t["type_output"], t["type_attn_qgate"],
                    t["type_attn_kv"], t["type_attn_out"], t["type_ssm_qkv"], t["type_ssm_gate"],
                    t["type_ssm_out"], t["type_expert_gate_up"], t["type_expert_down"], t["type_shared"],
                    seed, stddev, small_stddev, conv_stddev, threads)
    err = ctypes.create_string_buffer(512)
    path = pathlib.Path(path)
    rc = _native.tools().hipllm_tools_write_qwen35moe(str(path).encode(), ctypes.byref(spec), err, 512)
    if rc != 0:
        raise RuntimeError(f"synthetic qwen35moe writer failed: {err.value.decode()}")
    return path


def fallback_type(qtype: int, cols: int) -> int:
    """The Q4_K_M fallback for rows that are not a multiple of 256."""
    if cols % BLOCK[qtype] == 0:
        return qtype
    if qtype == Q4_K:
        return Q5_0
    if qtype == Q6_K:
        return Q8_0
    raise ValueError(f"{TYPE_NAMES[qtype]} cannot hold rows of {cols}")


def q4_k_m_types(shape: Qwen2Shape) -> dict:
    h, f = shape.hidden, shape.ffn
    return dict(
        type_embd=Q8_0,
        type_attn_qkv=fallback_type(Q4_K, h),
        type_attn_out=fallback_type(Q4_K, h),
        type_ffn_gate_up=fallback_type(Q4_K, h),
        type_ffn_down=fallback_type(Q6_K, f),
        type_output=fallback_type(Q6_K, h),
    )


def tiny_all_types() -> dict:
    """Mix for the tiny golden model: every supported block type appears."""
    return dict(type_embd=Q8_0, type_attn_qkv=Q4_K, type_attn_out=Q5_0,
                type_ffn_gate_up=Q4_K, type_ffn_down=Q6_K, type_output=Q6_K)


def write_qwen2(path, shape: Qwen2Shape, types: dict | None = None, seed: int = 0,
                stddev: float = 0.02, bias_stddev: float = 0.02,
                threads: int | None = None, context: int | None = None) -> pathlib.Path:
    """Writes a synthetic qwen2 GGUF and returns its path."""
    types = dict(q4_k_m_types(shape) if types is None else types)
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    spec = _Spec(shape.layers, shape.hidden, shape.heads, shape.kv_heads, shape.ffn,
                 shape.vocab, context or shape.context, shape.eos_token_id,
                 shape.rope_theta, shape.norm_eps,
                 types["type_embd"], types["type_attn_qkv"], types["type_attn_out"],
                 types["type_ffn_gate_up"], types["type_ffn_down"], types["type_output"],
                 seed, stddev, bias_stddev, threads)
    err = ctypes.create_string_buffer(512)
    path = pathlib.Path(path)
    rc = _native.tools().hipllm_tools_write_qwen2(str(path).encode(), ctypes.byref(spec), err, 512)
    if rc != 0:
        raise RuntimeError(f"synthetic GGUF writer failed: {err.value.decode()}")
    return path


def normal(n: int, seed: int, stream: int = 0, stddev: float = 1.0, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _native.tools().hipllm_tools_fill_normal(seed, stream, first, n, stddev, out.ctypes.data)
    return out


def uniform_ids(n: int, bound: int, seed: int, stream: int = 1) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    _native.tools().hipllm_tools_fill_uniform_int(seed, stream, 0, n, bound, out.ctypes.data)
    return out


def row_bytes(qtype: int, cols: int) -> int:
    rb = _native.tools().hipllm_tools_row_bytes(qtype, cols)
    if rb == 0:
        raise ValueError(f"{TYPE_NAMES.get(qtype, qtype)} cannot hold rows of {cols}")
    return rb


def quantize(w: np.ndarray, qtype: int, threads: int | None = None) -> np.ndarray:
    """Quantizes a [rows, cols] float32 matrix into [rows, row_bytes] uint8."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    rb = row_bytes(qtype, cols)
    out = np.empty((rows, rb), dtype=np.uint8)
    threads = threads or min(16, os.cpu_count() or 1)
    rc = _native.tools().hipllm_tools_quantize_rows(qtype, w.ctypes.data, rows, cols,
                                                      out.ctypes.data, threads)
    if rc != 0:
        raise RuntimeError("quantization failed")
    return out


def random_quantized(rows: int, cols: int, qtype: int, seed: int, stddev: float = 0.02,
                     threads: int | None = None) -> np.ndarray:
    """N(0, stddev) weights quantized to qtype, generated in row slabs."""
    rb = row_bytes(qtype, cols)
    out = np.empty((rows, rb), dtype=np.uint8)
    slab = max(1, (64 << 20) // (cols * 4))
    for r0 in range(0, rows, slab):
        r1 = min(rows, r0 + slab)
        w = normal((r1 - r0) * cols, seed, stream=0x5EED, stddev=stddev, first=r0 * cols)
        out[r0:r1] = quantize(w.reshape(r1 - r0, cols), qtype, threads)
    return out


def file_sha256(path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


# ------------------------------------------------------------ tokenizer tables

_GGUF_SCALAR_SIZE = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
_GGUF_STRING, _GGUF_ARRAY = 8, 9


def _skip_value(buf: bytes, pos: int, vtype: int) -> int:
    if vtype in _GGUF_SCALAR_SIZE:
        return pos + _GGUF_SCALAR_SIZE[vtype]
    if vtype == _GGUF_STRING:
        (n,) = np.frombuffer(buf, "<u8", 1, pos)
        return pos + 8 + int(n)
    if vtype == _GGUF_ARRAY:
        etype = int(np.frombuffer(buf, "<u4", 1, pos)[0])
        count = int(np.frombuffer(buf, "<u8", 1, pos + 4)[0])
        pos += 12
        if etype in _GGUF_SCALAR_SIZE:
            return pos + count * _GGUF_SCALAR_SIZE[etype]
        for _ in range(count):
            pos = _skip_value(buf, pos, etype)
        return pos
    raise ValueError(f"unknown GGUF value type {vtype}")


def _gguf_str(s) -> bytes:
    data = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return len(data).to_bytes(8, "little") + data


def add_tokenizer(src, dst, tokens, merges, tokenizer_pre: str = "qwen2") -> pathlib.Path:
    """Copies GGUF ``src`` to ``dst`` with the tokenizer tables the chat front
    end reads (tokenizer.ggml.tokens / .merges / .pre, as string arrays and a
    string), replacing any present. The tensor directory and data are copied
    unchanged; the data start moves to the next ``general.alignment``
    boundary."""
    src, dst = pathlib.Path(src), pathlib.Path(dst)
    with open(src, "rb") as f:
        head = f.read(1 << 20)
        while True:
            try:
                return _add_tokenizer(src, dst, head, tokens, merges, tokenizer_pre)
            except (IndexError, ValueError) as e:  # header longer than what was read
                more = f.read(len(head))
                if not more:
                    raise ValueError(f"{src}: malformed GGUF header") from e
                head += more


def _add_tokenizer(src, dst, head, tokens, merges, pre):
    if head[:4] != b"GGUF":
        raise ValueError("not a GGUF file")
    tensor_count = int.from_bytes(head[8:16], "little")
    kv_count = int.from_bytes(head[16:24], "little")
    pos, alignment = 24, 32
    keep = []
    replaced = {"tokenizer.ggml.tokens", "tokenizer.ggml.merges", "tokenizer.ggml.pre"}
    for _ in range(kv_count):
        start = pos
        klen = int.from_bytes(head[pos:pos + 8], "little")
        key = head[pos + 8:pos + 8 + klen].decode()
        pos += 8 + klen
        vtype = int.from_bytes(head[pos:pos + 4], "little")
        vpos = pos + 4
        pos = _skip_value(head, vpos, vtype)
        if pos > len(head):
            raise IndexError("short header")
        if key == "general.alignment":
            alignment = int.from_bytes(head[vpos:vpos + 4], "little")
        if key not in replaced:
            keep.append(head[start:pos])
    info_start = pos
    for _ in range(tensor_count):
        nlen = int.from_bytes(head[pos:pos + 8], "little")
        pos += 8 + nlen
        ndim = int.from_bytes(head[pos:pos + 4], "little")
        pos += 4 + 8 * ndim + 4 + 8
        if pos > len(head):
            raise IndexError("short header")
    infos = head[info_start:pos]
    data_start = (pos + alignment - 1) // alignment * alignment

    def string_array(key, values):
        out = _gguf_str(key) + _GGUF_ARRAY.to_bytes(4, "little") + _GGUF_STRING.to_bytes(4, "little")
        out += len(values).to_bytes(8, "little")
        return out + b"".join(_gguf_str(v) for v in values)

    extra = [string_array("tokenizer.ggml.tokens", tokens), string_array("tokenizer.ggml.merges", merges),
             _gguf_str("tokenizer.ggml.pre") + _GGUF_STRING.to_bytes(4, "little") + _gguf_str(pre)]
    new_head = head[:8] + tensor_count.to_bytes(8, "little") + (len(keep) + len(extra)).to_bytes(8, "little")
    new_head += b"".join(keep) + b"".join(extra) + infos
    new_head += b"\0" * ((-len(new_head)) % alignment)
    with open(src, "rb") as fin, open(dst, "wb") as fout:
        fout.write(new_head)
        fin.seek(data_start)
        while chunk := fin.read(1 << 24):
            fout.write(chunk)
    return dst
