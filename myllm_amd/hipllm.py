"""Python view of libhipllm.so: the HipLLM backend and its kernel launchers.

``HipLLM`` mirrors the reference backend classes (MetalLLM, metal_llm.h:20-52;
CPULLM, cpu_llm.h:165-194): reset(), prefill(ids) -> int, decode(id) -> int,
config, position, max_sequence, uses_gpu, memory_stats(), device_name,
enable_profiling(). Errors map the reference's C++ exception types onto
Python ones (see ``ERRORS``).

The ``kernels`` namespace exposes each C-ABI launcher over torch device
tensors (torch only provides device memory and the current stream). There is
no CPU fallback: without libhipllm.so or a GPU these raise.
"""

from __future__ import annotations

import ctypes
import re
import types

import numpy as np

from . import _native

OK, INVALID_ARGUMENT, OUT_OF_RANGE, LENGTH_ERROR, RUNTIME_ERROR, OVERFLOW_ERROR = range(6)


class LengthError(OverflowError):
    """std::length_error: sequence capacity exceeded."""


class OverflowErrorStd(OverflowError):
    """std::overflow_error."""


ERRORS = {INVALID_ARGUMENT: ValueError, OUT_OF_RANGE: IndexError, LENGTH_ERROR: LengthError,
          RUNTIME_ERROR: RuntimeError, OVERFLOW_ERROR: OverflowErrorStd}


class HipllmConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "layer_count", "embedding_size", "feed_forward_size", "attention_head_count",
        "kv_head_count", "head_size", "rotary_dimension", "vocabulary_size", "context_length",
        "parameter_count", "stored_weight_bytes")] + [
        ("eos_token_id", ctypes.c_int32), ("rope_theta", ctypes.c_float),
        ("norm_epsilon", ctypes.c_float), ("architecture", ctypes.c_char * 32)] + [
        (n, ctypes.c_uint64) for n in (
            "full_attention_interval", "expert_count", "expert_used_count", "expert_feed_forward_size",
            "shared_expert_feed_forward_size", "ssm_conv_kernel", "ssm_state_size", "ssm_group_count",
            "ssm_time_step_rank", "ssm_inner_size")]


class HipllmMemoryStats(ctypes.Structure):
    _fields_ = [("weight_bytes", ctypes.c_uint64), ("kv_cache_bytes", ctypes.c_uint64),
                ("recurrent_state_bytes", ctypes.c_uint64), ("intermediate_bytes", ctypes.c_uint64),
                ("intermediate_is_estimate", ctypes.c_int32)]


class HipllmGenerationStats(ctypes.Structure):
    """GenerationStats (chat.h:20-41)."""
    _fields_ = [("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double), ("total_ms", ctypes.c_double),
                ("prompt_tokens", ctypes.c_uint64), ("generated_tokens", ctypes.c_uint64),
                ("decode_steps", ctypes.c_uint64), ("used_gpu", ctypes.c_int32), ("stopped", ctypes.c_int32),
                ("has_expert_cache_stats", ctypes.c_int32), ("expert_cache_hits", ctypes.c_uint64),
                ("expert_cache_misses", ctypes.c_uint64), ("memory", HipllmMemoryStats)]


TOKEN_SINK = ctypes.CFUNCTYPE(None, ctypes.c_int32, ctypes.c_void_p)


_P = ctypes.c_void_p
_S = ctypes.c_size_t
_U32 = ctypes.c_uint32
_I32 = ctypes.c_int32
_F = ctypes.c_float
_I = ctypes.c_int

SIGNATURES = {
    "hipllm_last_error": (ctypes.c_char_p, []),
    "hipllm_version": (ctypes.c_char_p, []),
    "hipllm_dequant_rows": (_I, [_U32, _P, _S, _S, _S, _P, _P]),
    "hipllm_prep_x": (_I, [_P, _P, _S, _P]),
    "hipllm_gemv_workspace_bytes": (_S, [_S]),
    "hipllm_gemv": (_I, [_U32, _P, _S, _P, _P, _P, _S, _S, _P, _P]),
    "hipllm_gemv_noalloc": (_I, [_U32, _P, _S, _P, _P, _P, _S, _S, _P]),
    "hipllm_gemv_prepped": (_I, [_U32, _P, _S, _P, _P, _P, _P, _P, _S, _S, _I, _P]),
    "hipllm_gemv_swiglu": (_I, [_U32, _P, _P, _S, _P, _P, _P, _P, _S, _S, _I, _P]),
    "hipllm_gemv_norm": (_I, [_U32, _P, _S, _P, _P, _F, _P, _P, _P, _S, _S, _I, _P]),
    "hipllm_gemv_swiglu_norm": (_I, [_U32, _P, _P, _S, _P, _P, _F, _P, _P, _S, _S, _I, _P]),
    "hipllm_to_f16": (_I, [_P, _S, _P, _P, _S, _S, _P]),
    "hipllm_x16_bytes": (_S, [_U32, _S, _S]),
    "hipllm_pack_x16": (_I, [_U32, _P, _S, _S, _S, _P, _P]),
    "hipllm_gemv_x16": (_I, [_U32, _P, _P, _P, _P, _P, _S, _S, _I, _P, _P]),
    "hipllm_gemv_x16_swiglu": (_I, [_U32, _P, _P, _P, _P, _P, _S, _S, _I, _P, _P]),
    "hipllm_gemv_x16_routed": (_I, [_U32, _P, _P, _P, _S, _I, _P, _P, _S, _S, _S, _S, _S, _P, _P, _P, _P, _I, _P]),
    "hipllm_gemm_mfma": (_I, [_U32, _P, _S, _P, _P, _P, _P, _P, _S, _S, _S, _I, _I, _P, _S, _P]),
    "hipllm_gemm_mfma_workspace_bytes": (_S, [_S, _S, _S, _I, _I]),
    "hipllm_gemm_workspace_bytes": (_S, [_S, _S]),
    "hipllm_gemm": (_I, [_U32, _P, _S, _P, _S, _P, _P, _S, _S, _S, _P, _P]),
    "hipllm_rmsnorm": (_I, [_P, _P, _P, _P, _S, _S, _F, _P]),
    "hipllm_embed": (_I, [_U32, _P, _S, _P, _S, _S, _S, _P, _P]),
    "hipllm_rope_kv": (_I, [_P, _P, _S, _S, _S, _S, _S, _S, _S, _P, _P, _P]),
    "hipllm_attn_decode_scratch_floats": (_S, [_S, _S, _S]),
    "hipllm_attn_decode_rope": (_I, [_P, _P, _S, _P, _P, _P, _P, _P, _S, _S, _S, _S, _F, _P]),
    "hipllm_attn_decode": (_I, [_P, _P, _P, _P, _P, _P, _S, _S, _S, _S, _F, _P]),
    "hipllm_argmax_scratch_bytes": (_S, [_S]),
    "hipllm_argmax": (_I, [_P, _S, _P, _P, _P]),
    "hipllm_swiglu": (_I, [_P, _P, _P, _P, _S, _P]),
    "hipllm_create": (_I, [ctypes.c_char_p, _S, _I, ctypes.POINTER(_P)]),
    "hipllm_create_ex": (_I, [ctypes.c_char_p, _S, _I, _S, ctypes.POINTER(_P)]),
    "hipllm_copy_routes": (_I, [_P, _P, _S]),
    "hipllm_expert_cache_count": (_S, [_P]),
    "hipllm_attn_prefill": (_I, [_P, _S, _P, _P, _P, _S, _S, _S, _S, _S, _S, _F, _P]),
    "hipllm_gemv_batched": (_I, [_U32, _P, _P, _S, _P, _P, _P, _P, _P, _P, _S, _S, _S, _P, _S, _S, _S, _I, _S, _S,
                                 _P]),
    "hipllm_router_topk": (_I, [_P, _S, _S, _S, _S, _P, _P, _P]),
    "hipllm_moe_combine": (_I, [_P, _P, _P, _P, _P, _S, _P, _S, _S, _S, _P]),
    "hipllm_moe_combine_norm": (_I, [_P, _P, _P, _P, _P, _S, _P, _P, _P, _P, _S, _S, _S, _F, _P]),
    "hipllm_gemv_multi_norm": (_I, [_P, _S, _P, _P, _F, _S, _P, _P, _P]),
    "hipllm_matmul_f32": (_I, [_P, _S, _P, _S, _P, _S, _S, _S, _S, _P, _S, _P]),
    "hipllm_matmul_f32_scratch_floats": (_S, [_S, _S, _S]),
    "hipllm_route_groups_max": (_S, [_S, _S, _S]),
    "hipllm_route_groups": (_I, [_P, _S, _S, _S, _P, _P, _P, _P]),
    "hipllm_gemm_gather": (_I, [_U32, _P, _S, _P, _P, _P, _S, _S, _S, _P, _P, _P, _S, _S, _S, _I, _P]),
    "hipllm_attn_decode_rope_gated": (_I, [_P, _P, _S, _P, _P, _P, _P, _P, _P, _S, _S, _S, _S, _F, _P]),
    "hipllm_gemv_routed_swiglu": (_I, [_U32, _P, _P, _S, _P, _P, _S, _P, _P, _S, _S, _S, _P, _S, _S, _S, _S, _P, _P,
                                       _P]),
    "hipllm_gemv_moe_combine": (_I, [_U32, _P, _S, _P, _P, _P, _P, _P, _S, _P, _S, _S, _P]),
    "hipllm_gdn_gates": (_I, [_P, _P, _S, _P, _P, _P, _P, _S, _S, _P]),
    "hipllm_conv1d_silu": (_I, [_P, _S, _P, _P, _P, _S, _S, _S, _S, _P]),
    "hipllm_l2norm_heads": (_I, [_P, _S, _S, _S, _S, _F, _P]),
    "hipllm_gdn_chunk_scratch_floats": (_S, [_S, _S]),
    "hipllm_gdn_scan_chunked": (_I, [_P, _P, _S, _P, _S, _P, _P, _P, _P, _S, _S, _S, _S, _S, _P, _S, _P]),
    "hipllm_gdn_scan": (_I, [_P, _P, _S, _P, _S, _P, _P, _P, _P, _S, _S, _S, _S, _S, _P]),
    "hipllm_gated_rmsnorm": (_I, [_P, _S, _P, _P, _S, _P, _P, _S, _S, _S, _S, _F, _P]),
    "hipllm_conv_l2norm": (_I, [_P, _S, _P, _P, _P, _S, _S, _S, _S, _S, _S, _F, _P]),
    "hipllm_gdn_scan_gated": (_I, [_P, _P, _S, _P, _S, _P, _P, _S, _P, _P, _P, _P, _S, _P, _P, _P, _S, _S, _S, _S,
                                   _S, _F, _P]),
    "hipllm_gdn_decode": (_I, [_P, _P, _P, _P, _S, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S, _F, _P]),
    "hipllm_attn_decode_qgate": (_I, [_P, _P, _P, _P, _F, _P, _S, _P, _P, _P, _P, _S, _S, _S, _S, _F, _P]),
    "hipllm_rmsnorm_f16": (_I, [_P, _P, _P, _P, _P, _S, _S, _F, _P]),
    "hipllm_gemm_swiglu_workspace_bytes": (_S, [_S, _S, _S]),
    "hipllm_gemm_mfma_swiglu": (_I, [_U32, _P, _P, _S, _P, _P, _P, _S, _S, _S, _P, _S, _P]),
    "hipllm_gemm_mfma_swiglu_f16": (_I, [_U32, _P, _P, _S, _P, _P, _P, _P, _S, _S, _S, _P, _S, _P]),
    "hipllm_gemv_x16_grouped": (_I, [_U32, _P, _P, _P, _S, _I, _S, _P, _P, _S, _S, _S, _S, _P, _P, _P, _S, _P]),
    "hipllm_gemv_x16_pair": (_I, [_U32, _P, _S, _P, _U32, _P, _S, _P, _S, _P, _P, _F, _P, _P, _S, _P, _P, _P]),
    "hipllm_gemv_x16_moe_down": (_I, [_U32, _P, _P, _S, _P, _S, _S, _U32, _P, _P, _S, _P, _P, _P, _P, _S, _S, _P,
                                      _P]),
    "hipllm_split_qgate_norm": (_I, [_P, _S, _P, _S, _P, _P, _P, _S, _P, _S, _S, _S, _S, _S, _F, _P]),
    "hipllm_gate_mul": (_I, [_P, _P, _P, _P, _S, _P]),
    "hipllm_destroy": (None, [_P]),
    "hipllm_reset": (_I, [_P]),
    "hipllm_prefill": (_I, [_P, _P, _S, ctypes.POINTER(_I32)]),
    "hipllm_decode": (_I, [_P, _I32, ctypes.POINTER(_I32)]),
    "hipllm_config": (_I, [_P, ctypes.POINTER(HipllmConfig)]),
    "hipllm_position": (_S, [_P]),
    "hipllm_max_sequence": (_S, [_P]),
    "hipllm_uses_gpu": (_I, [_P]),
    "hipllm_memory_stats": (_I, [_P, ctypes.POINTER(HipllmMemoryStats)]),
    "hipllm_device_name": (ctypes.c_char_p, [_P]),
    "hipllm_enable_profiling": (_I, [_P, ctypes.c_char_p, _I]),
    "hipllm_set_route_probe": (_I, [_P, _I]),
    "hipllm_copy_router_logits": (_I, [_P, _P, _S]),
    "hipllm_vocabulary_count": (_S, [_P]),
    "hipllm_vocabulary_token": (ctypes.c_char_p, [_P, _S]),
    "hipllm_merge_count": (_S, [_P]),
    "hipllm_merge": (ctypes.c_char_p, [_P, _S]),
    "hipllm_tokenizer_pre": (ctypes.c_char_p, [_P]),
    "hipllm_expert_cache_stats": (_I, [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "hipllm_disable_profiling": (_I, [_P]),
    "hipllm_copy_logits": (_I, [_P, _P, _S]),
    "hipllm_set_batched_prefill": (_I, [_P, _I]),
    "hipllm_set_decode_graphs": (_I, [_P, _I]),
    "hipllm_set_packed_decode": (_I, [_P, _I]),
    "hipllm_set_fused_norms": (_I, [_P, _I]),
    "hipllm_inspect_gguf": (_I, [ctypes.c_char_p, ctypes.POINTER(HipllmConfig)]),
    "hipllm_tokenizer_create": (_I, [ctypes.POINTER(ctypes.c_char_p), _S, ctypes.POINTER(ctypes.c_char_p), _S,
                                     ctypes.c_char_p, ctypes.POINTER(_P)]),
    "hipllm_tokenizer_from_model": (_I, [_P, ctypes.POINTER(_P)]),
    "hipllm_tokenizer_destroy": (None, [_P]),
    "hipllm_tokenize": (_I, [_P, ctypes.c_char_p, _S, _P, _S, ctypes.POINTER(_S)]),
    "hipllm_token_id": (_I32, [_P, ctypes.c_char_p]),
    "hipllm_token_is_special": (_I, [_P, _I32]),
    "hipllm_decode_piece": (_I, [_P, _I32, _P, _S, ctypes.POINTER(_S)]),
    "hipllm_pretokenize": (_I, [_P, ctypes.c_char_p, _S, _P, _S, ctypes.POINTER(_S)]),
    "hipllm_chat_prompt": (_I, [ctypes.c_char_p, ctypes.c_char_p, _P, _S, ctypes.POINTER(_S)]),
    "hipllm_stop_tokens": (_I, [_P, _P, _P, _S, ctypes.POINTER(_S)]),
    "hipllm_run": (_I, [_P, _P, _S, _S, _P, _S, TOKEN_SINK, _P, _P, _S, ctypes.POINTER(_S),
                        ctypes.POINTER(HipllmGenerationStats)]),
    "hipllm_format_generation_stats": (_I, [ctypes.POINTER(HipllmGenerationStats), _P, _S, ctypes.POINTER(_S)]),
    "hipllm_chat_main": (_I, [_I, ctypes.POINTER(ctypes.c_char_p)]),
}


def lib() -> ctypes.CDLL:
    L = _native.hipllm()
    if not getattr(L, "_hipllm_typed", False):
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        L._hipllm_typed = True
    return L


def header_functions(header_text: str) -> list[str]:
    """Names of the functions a C header declares (for export checks)."""
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(hipllm_\w+)\s*\(", header_text, re.M)))


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().hipllm_last_error().decode(errors="replace")
        raise ERRORS.get(rc, RuntimeError)(msg)


def _config_dict(cfg: HipllmConfig) -> dict:
    d = {n: getattr(cfg, n) for n, _ in HipllmConfig._fields_ if n != "architecture"}
    d["architecture"] = cfg.architecture.decode()
    return d


def inspect_gguf(path) -> dict:
    """Parses a GGUF with the streaming reader (no GPU needed)."""
    cfg = HipllmConfig()
    check(lib().hipllm_inspect_gguf(str(path).encode(), ctypes.byref(cfg)))
    return _config_dict(cfg)


class HipLLM:
    """The MI355X qwen2 backend, same contract as the reference's MetalLLM."""

    def __init__(self, gguf_path, max_sequence: int = 0, device: int = -1, expert_cache_count: int = 8):
        self._h = _P()
        check(lib().hipllm_create_ex(str(gguf_path).encode(), max_sequence, device, expert_cache_count,
                                     ctypes.byref(self._h)))
        cfg = HipllmConfig()
        check(lib().hipllm_config(self._h, ctypes.byref(cfg)))
        self.config = _config_dict(cfg)

    def close(self) -> None:
        if self._h:
            lib().hipllm_destroy(self._h)
            self._h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self) -> None:
        check(lib().hipllm_reset(self._h))

    def prefill(self, ids) -> int:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        out = _I32()
        check(lib().hipllm_prefill(self._h, a.ctypes.data if a.size else None, a.size, ctypes.byref(out)))
        return out.value

    def decode(self, token: int) -> int:
        out = _I32()
        check(lib().hipllm_decode(self._h, int(token), ctypes.byref(out)))
        return out.value

    @property
    def position(self) -> int:
        return lib().hipllm_position(self._h)

    @property
    def max_sequence(self) -> int:
        return lib().hipllm_max_sequence(self._h)

    @property
    def uses_gpu(self) -> bool:
        return bool(lib().hipllm_uses_gpu(self._h))

    @property
    def device_name(self) -> str:
        return lib().hipllm_device_name(self._h).decode()

    def memory_stats(self) -> dict:
        s = HipllmMemoryStats()
        check(lib().hipllm_memory_stats(self._h, ctypes.byref(s)))
        return {n: getattr(s, n) for n, _ in HipllmMemoryStats._fields_}

    def enable_profiling(self, csv_path, detailed_kernel_timestamps: bool = False) -> None:
        check(lib().hipllm_enable_profiling(self._h, str(csv_path).encode(), 1 if detailed_kernel_timestamps else 0))

    def disable_profiling(self) -> None:
        check(lib().hipllm_disable_profiling(self._h))

    def logits(self) -> np.ndarray:
        out = np.empty(self.config["vocabulary_size"], dtype=np.float32)
        check(lib().hipllm_copy_logits(self._h, out.ctypes.data, out.size))
        return out

    def set_batched_prefill(self, enabled: bool) -> None:
        check(lib().hipllm_set_batched_prefill(self._h, 1 if enabled else 0))

    def set_packed_decode(self, enabled: bool) -> None:
        check(lib().hipllm_set_packed_decode(self._h, int(bool(enabled))))

    def set_fused_norms(self, enabled: bool) -> None:
        check(lib().hipllm_set_fused_norms(self._h, int(bool(enabled))))

    def set_decode_graphs(self, enabled: bool) -> None:
        """True (default): each decode step replays one recorded HIP graph."""
        check(lib().hipllm_set_decode_graphs(self._h, 1 if enabled else 0))

    def routes(self) -> np.ndarray:
        """qwen35moe: expert ids of the last row of the last forward, [layers, top-k]."""
        L = self.config["layer_count"]
        k = self.config["expert_used_count"]
        out = np.empty((L, k), dtype=np.int32)
        check(lib().hipllm_copy_routes(self._h, out.ctypes.data, out.size))
        return out

    def set_route_probe(self, enabled: bool) -> None:
        check(lib().hipllm_set_route_probe(self._h, 1 if enabled else 0))

    def router_logits(self) -> np.ndarray:
        """qwen35moe with the route probe on: [layers, experts + 1] router
        logits (last column: shared-expert gate) of the last row of the last
        forward."""
        L = self.config["layer_count"]
        E = self.config["expert_count"]
        out = np.empty((L, E + 1), dtype=np.float32)
        check(lib().hipllm_copy_router_logits(self._h, out.ctypes.data, out.size))
        return out

    @property
    def expert_cache_count(self) -> int:
        return lib().hipllm_expert_cache_count(self._h)

    def expert_cache_stats(self) -> dict:
        hits, misses = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().hipllm_expert_cache_stats(self._h, ctypes.byref(hits), ctypes.byref(misses)))
        return {"hits": hits.value, "misses": misses.value}

    @property
    def vocabulary(self) -> list:
        """tokenizer.ggml.tokens as raw UTF-8 bytes per entry."""
        return [lib().hipllm_vocabulary_token(self._h, i) for i in range(lib().hipllm_vocabulary_count(self._h))]

    @property
    def merges(self) -> list:
        return [lib().hipllm_merge(self._h, i) for i in range(lib().hipllm_merge_count(self._h))]

    @property
    def tokenizer_pre(self) -> str:
        return lib().hipllm_tokenizer_pre(self._h).decode()


def _bytes(text) -> bytes:
    return text.encode("utf-8") if isinstance(text, str) else bytes(text)


def _read_sized(call, what: str) -> bytes:
    """Two-pass read of a (buffer, capacity, *length) C-ABI call."""
    n = _S(0)
    rc = call(None, 0, ctypes.byref(n))
    if rc not in (OK, LENGTH_ERROR):
        check(rc)
    buf = ctypes.create_string_buffer(max(1, n.value))
    check(call(buf, n.value, ctypes.byref(n)))
    return buf.raw[:n.value]


class QwenTokenizer:
    """QwenTokenizer (chat.cpp:349-529) in libhipllm.so: encode, id,
    decode_piece, is_special, plus the pre-tokenizer's piece ranges.
    Host code only; usable without a GPU."""

    def __init__(self, vocabulary, merges, tokenizer_pre: str = "", *, _handle=None):
        if _handle is not None:
            self._h = _handle
            return
        voc = [_bytes(v) for v in vocabulary]
        mer = [_bytes(m) for m in merges]
        varr = (ctypes.c_char_p * max(1, len(voc)))(*voc)
        marr = (ctypes.c_char_p * max(1, len(mer)))(*mer)
        h = _P()
        check(lib().hipllm_tokenizer_create(varr, len(voc), marr, len(mer), _bytes(tokenizer_pre), ctypes.byref(h)))
        self._h = h

    @classmethod
    def from_model(cls, model: "HipLLM") -> "QwenTokenizer":
        h = _P()
        check(lib().hipllm_tokenizer_from_model(model._h, ctypes.byref(h)))
        return cls(None, None, _handle=h)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().hipllm_tokenizer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text) -> list:
        data = _bytes(text)
        n = _S(0)
        cap = len(data) + 1
        while True:
            out = (ctypes.c_int32 * cap)()
            rc = lib().hipllm_tokenize(self._h, data, len(data), out, cap, ctypes.byref(n))
            if rc == LENGTH_ERROR and n.value > cap:
                cap = n.value
                continue
            check(rc)
            return list(out[:n.value])

    def id(self, token) -> int:
        return lib().hipllm_token_id(self._h, _bytes(token))

    def is_special(self, token: int) -> bool:
        return bool(lib().hipllm_token_is_special(self._h, int(token)))

    def decode_piece(self, token: int) -> bytes:
        return _read_sized(lambda b, c, n: lib().hipllm_decode_piece(self._h, int(token), b, c, n), "decode_piece")

    def decode(self, tokens) -> bytes:
        return b"".join(self.decode_piece(t) for t in tokens)

    def pieces(self, text) -> list:
        data = _bytes(text)
        n = _S(0)
        cap = 2 * len(data) + 2
        out = (ctypes.c_size_t * cap)()
        check(lib().hipllm_pretokenize(self._h, data, len(data), out, cap, ctypes.byref(n)))
        return [(out[2 * i], out[2 * i + 1]) for i in range(n.value)]


def chat_prompt(system, user) -> str:
    """ChatML wrapping of one turn (chat.cpp:655-659)."""
    raw = _read_sized(lambda b, c, n: lib().hipllm_chat_prompt(_bytes(system), _bytes(user), b, c, n), "chat_prompt")
    return raw.decode("utf-8")


def stop_tokens(model: "HipLLM", tokenizer: QwenTokenizer) -> list:
    """make_stop_tokens (chat.cpp:708-726)."""
    cap = 64
    while True:
        out = (ctypes.c_int32 * cap)()
        n = _S(0)
        rc = lib().hipllm_stop_tokens(model._h, tokenizer._h, out, cap, ctypes.byref(n))
        if rc == LENGTH_ERROR and n.value > cap:
            cap = n.value
            continue
        check(rc)
        return list(out[:n.value])


def _stats_dict(s: HipllmGenerationStats) -> dict:
    d = {k: getattr(s, k) for k, _ in HipllmGenerationStats._fields_ if k != "memory"}
    d["memory"] = {k: getattr(s.memory, k) for k, _ in HipllmMemoryStats._fields_}
    for k in ("used_gpu", "stopped", "has_expert_cache_stats"):
        d[k] = bool(d[k])
    return d


def run(model: "HipLLM", ids, max_new_tokens: int, stop_token_ids=(), token_sink=None):
    """chat::run (chat.h:59-75) in libhipllm.so: returns (tokens, stats, stats_line)."""
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
    stop = np.ascontiguousarray(np.asarray(list(stop_token_ids), dtype=np.int32))
    cap = max(1, int(max_new_tokens))
    out = (ctypes.c_int32 * cap)()
    n = _S(0)
    stats = HipllmGenerationStats()
    errors = []

    def _sink(token, _user):
        try:
            token_sink(int(token))
        except Exception as e:  # an exception must not cross the C ABI
            errors.append(e)

    sink = TOKEN_SINK(_sink) if token_sink else TOKEN_SINK()
    check(lib().hipllm_run(model._h, ids.ctypes.data if ids.size else None, ids.size, int(max_new_tokens),
                           stop.ctypes.data if stop.size else None, stop.size, sink, None, out, cap,
                           ctypes.byref(n), ctypes.byref(stats)))
    if errors:
        raise errors[0]
    line = _read_sized(lambda b, c, k: lib().hipllm_format_generation_stats(ctypes.byref(stats), b, c, k),
                       "format_generation_stats").decode()
    return list(out[:min(cap, n.value)]), _stats_dict(stats), line


def generate(backend, prompt, max_new_tokens: int, stop_token_ids=(), on_step=None):
    """chat.cpp:831-878 generate(): reset, prefill, then emit/decode."""
    if len(prompt) == 0:
        raise ValueError("Generation requires at least one initial token")
    if max_new_tokens == 0:
        raise ValueError("Generation requires max_new_tokens > 0")
    if backend.max_sequence == 0:
        raise RuntimeError("Backend sequence capacity is zero")
    if len(prompt) >= backend.max_sequence:
        raise ValueError("Initial token sequence leaves no room for generated tokens")
    limit = min(max_new_tokens, backend.max_sequence - len(prompt))
    backend.reset()
    nxt = backend.prefill(prompt)
    if on_step:
        on_step(backend)
    out = []
    for step in range(limit):
        if nxt in stop_token_ids:
            break
        out.append(nxt)
        if step + 1 >= limit:
            break
        nxt = backend.decode(nxt)
        if on_step:
            on_step(backend)
    return out


# ------------------------------------------------------------ kernel wrappers

def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _k_dequant_rows(qtype, w, row_bytes, rows, k, out, stream=None):
    check(lib().hipllm_dequant_rows(qtype, _ptr(w), row_bytes, rows, k, _ptr(out), _stream(stream)))


def _k_prep_x(x, xq, k, stream=None):
    """XGroup form of x into xq (k / 16 groups of 64 bytes: allocate k float32s)."""
    check(lib().hipllm_prep_x(_ptr(x), _ptr(xq), k, _stream(stream)))


def _k_gemv(qtype, w, row_bytes, x, bias, y, n, k, workspace, stream=None):
    check(lib().hipllm_gemv(qtype, _ptr(w), row_bytes, _ptr(x), _ptr(bias), _ptr(y), n, k, _ptr(workspace),
                            _stream(stream)))


def _k_gemv_noalloc(qtype, w, row_bytes, x, bias, y, n, k, stream=None):
    check(lib().hipllm_gemv_noalloc(qtype, _ptr(w), row_bytes, _ptr(x), _ptr(bias), _ptr(y), n, k, _stream(stream)))


def _k_gemv_prepped(qtype, w, row_bytes, x, xq, bias, residual, y, n, k, tiling=0, stream=None):
    check(lib().hipllm_gemv_prepped(qtype, _ptr(w), row_bytes, _ptr(x), _ptr(xq), _ptr(bias), _ptr(residual),
                                    _ptr(y), n, k, tiling, _stream(stream)))


def _k_gemv_swiglu(qtype, wg, wu, row_bytes, x, xq, y, yq, n, k, tiling=0, stream=None):
    check(lib().hipllm_gemv_swiglu(qtype, _ptr(wg), _ptr(wu), row_bytes, _ptr(x), _ptr(xq), _ptr(y), _ptr(yq),
                                   n, k, tiling, _stream(stream)))


def _k_pack_x16(qtype, w, row_bytes, n, k, packed, stream=None):
    check(lib().hipllm_pack_x16(qtype, _ptr(w), row_bytes, n, k, _ptr(packed), _stream(stream)))


class HipllmX16Norm(ctypes.Structure):
    """An RMSNorm fused into an x16 GEMV (include/hipllm.h)."""
    _fields_ = [("sumsq_in", ctypes.c_void_p), ("eps", ctypes.c_float), ("gamma_out", ctypes.c_void_p),
                ("yq_out", ctypes.c_void_p), ("sumsq_out", ctypes.c_void_p)]


def _x16_norm(norm):
    """norm: None or a dict with sumsq_in / eps, or gamma_out / yq_out / sumsq_out (tensors)."""
    if norm is None:
        return None
    def addr(name):
        t = norm.get(name)
        return None if t is None else t.data_ptr()

    n = HipllmX16Norm(addr("sumsq_in"), float(norm.get("eps", 0.0)), addr("gamma_out"), addr("yq_out"),
                      addr("sumsq_out"))
    return ctypes.byref(n)


def _k_gemv_x16(qtype, packed, xq, bias, residual, y, n, k, waves=0, stream=None, norm=None):
    check(lib().hipllm_gemv_x16(qtype, _ptr(packed), _ptr(xq), _ptr(bias), _ptr(residual), _ptr(y), n, k, waves,
                                _x16_norm(norm), _stream(stream)))


def _k_gemv_x16_swiglu(qtype, gate, up, xq, y, yq, n, k, waves=0, stream=None, norm=None):
    check(lib().hipllm_gemv_x16_swiglu(qtype, _ptr(gate), _ptr(up), _ptr(xq), _ptr(y), _ptr(yq), n, k, waves,
                                       _x16_norm(norm), _stream(stream)))


def _k_gemv_x16_routed(qtype, packed, packed2, xq, ldx, x_routed, y, yq, ldy, n, k, experts, routes, ids=None,
                       logits=None, ids_out=None, weights_out=None, waves=0, stream=None):
    check(lib().hipllm_gemv_x16_routed(qtype, _ptr(packed), _ptr(packed2), _ptr(xq), ldx, int(bool(x_routed)),
                                       _ptr(y), _ptr(yq), ldy, n, k, experts, routes, _ptr(ids), _ptr(logits),
                                       _ptr(ids_out), _ptr(weights_out), waves, _stream(stream)))


def _k_rmsnorm_f16(x, gamma, norm, xh, xscale, rows, cols, eps, stream=None):
    check(lib().hipllm_rmsnorm_f16(_ptr(x), _ptr(gamma), _ptr(norm), _ptr(xh), _ptr(xscale), rows, cols, eps,
                                   _stream(stream)))


def _k_gemm_mfma_swiglu(qtype, wg, wu, row_bytes, xh, xscale, y, m, n, k, workspace=None, stream=None):
    if workspace is None:
        import torch
        workspace = torch.empty(max(16, lib().hipllm_gemm_swiglu_workspace_bytes(m, n, k)), dtype=torch.uint8,
                                device=y.device)
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().hipllm_gemm_mfma_swiglu(qtype, _ptr(wg), _ptr(wu), row_bytes, _ptr(xh), _ptr(xscale), _ptr(y), m, n, k,
                                        _ptr(workspace), nbytes, _stream(stream)))


def _k_gemm_mfma_swiglu_f16(qtype, wg, wu, row_bytes, xh, xscale, yh, yscale, m, n, k, workspace=None, stream=None):
    if workspace is None:
        import torch
        workspace = torch.empty(max(16, lib().hipllm_gemm_swiglu_workspace_bytes(m, n, k)), dtype=torch.uint8,
                                device=yh.device)
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().hipllm_gemm_mfma_swiglu_f16(qtype, _ptr(wg), _ptr(wu), row_bytes, _ptr(xh), _ptr(xscale), _ptr(yh),
                                            _ptr(yscale), m, n, k, _ptr(workspace), nbytes, _stream(stream)))


def _k_gemv_x16_grouped(qtype, packed, packed2, xq, ldx, x_routed, routes, y, yq, ldy, n, k, experts, order, groups,
                        ngroups, max_groups, stream=None):
    check(lib().hipllm_gemv_x16_grouped(qtype, _ptr(packed), _ptr(packed2), _ptr(xq), ldx, int(bool(x_routed)), routes,
                                        _ptr(y), _ptr(yq), ldy, n, k, experts, _ptr(order), _ptr(groups), _ptr(ngroups),
                                        max_groups, _stream(stream)))


def _k_gemv_x16_moe_down(type_r, down_packed, ids, experts, xq, ldx, k_r, type_s, shared_packed, sx, k_s, weights,
                         sgate, residual, y, n, routes, norm_out=None, stream=None):
    check(lib().hipllm_gemv_x16_moe_down(type_r, _ptr(down_packed), _ptr(ids), experts, _ptr(xq), ldx, k_r, type_s,
                                         _ptr(shared_packed), _ptr(sx), k_s, _ptr(weights), _ptr(sgate),
                                         _ptr(residual), _ptr(y), n, routes, _x16_norm(norm_out), _stream(stream)))


def _k_to_f16(x, ldx, xh, xscale, m, k, stream=None):
    check(lib().hipllm_to_f16(_ptr(x), ldx, _ptr(xh), _ptr(xscale), m, k, _stream(stream)))


def _k_gemv_norm(qtype, w, row_bytes, x, gamma, eps, bias, residual, y, n, k, tiling=0, stream=None):
    check(lib().hipllm_gemv_norm(qtype, _ptr(w), row_bytes, _ptr(x), _ptr(gamma), eps, _ptr(bias), _ptr(residual),
                                 _ptr(y), n, k, tiling, _stream(stream)))


def _k_gemv_swiglu_norm(qtype, wg, wu, row_bytes, x, gamma, eps, y, yq, n, k, tiling=0, stream=None):
    check(lib().hipllm_gemv_swiglu_norm(qtype, _ptr(wg), _ptr(wu), row_bytes, _ptr(x), _ptr(gamma), eps, _ptr(y),
                                        _ptr(yq), n, k, tiling, _stream(stream)))


def _k_gemm_mfma(qtype, w, row_bytes, xh, xscale, bias, residual, y, m, n, k, tile=-1, stream=None, splits=0,
                 workspace=None):
    """workspace: a device buffer for the K split's partial sums; by default
    one of hipllm_gemm_mfma_workspace_bytes is allocated on y's device."""
    if workspace is None:
        need = lib().hipllm_gemm_mfma_workspace_bytes(m, n, k, tile, max(splits, 0))
        if need:
            import torch
            workspace = torch.empty(need, dtype=torch.uint8, device=y.device)
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().hipllm_gemm_mfma(qtype, _ptr(w), row_bytes, _ptr(xh), _ptr(xscale), _ptr(bias), _ptr(residual),
                                 _ptr(y), m, n, k, tile, splits, _ptr(workspace), nbytes, _stream(stream)))


def _k_gemm(qtype, w, row_bytes, x, ldx, bias, y, m, n, k, workspace, stream=None):
    check(lib().hipllm_gemm(qtype, _ptr(w), row_bytes, _ptr(x), ldx, _ptr(bias), _ptr(y), m, n, k,
                            _ptr(workspace), _stream(stream)))


def _k_attn_prefill(q, q_stride, kcache, vcache, out, out_stride, rows, hq, hkv, d, pos0, scale, stream=None):
    check(lib().hipllm_attn_prefill(_ptr(q), q_stride, _ptr(kcache), _ptr(vcache), _ptr(out), out_stride, rows, hq,
                                    hkv, d, pos0, scale, _stream(stream)))


def _k_gemv_batched(qtype, w, wu, row_bytes, x, xq, bias, residual, y, yq, n, k, vectors, ids=None,
                    experts=1, routes=1, expert_stride=0, x_routed=False, ldx=None, ldy=None, stream=None):
    check(lib().hipllm_gemv_batched(qtype, _ptr(w), _ptr(wu), row_bytes, _ptr(x), _ptr(xq), _ptr(bias),
                                    _ptr(residual), _ptr(y), _ptr(yq), n, k, vectors, _ptr(ids), experts, routes,
                                    expert_stride, 1 if x_routed else 0, ldx or k, ldy or n, _stream(stream)))


def _k_matmul_f32(x, ldx, w, ldw, y, ldy, m, n, k, scratch=None, stream=None):
    check(lib().hipllm_matmul_f32(_ptr(x), ldx, _ptr(w), ldw, _ptr(y), ldy, m, n, k, _ptr(scratch),
                                  0 if scratch is None else scratch.numel(), _stream(stream)))


def _k_route_groups(ids, n, experts, vmax, order, groups, ngroups, stream=None):
    check(lib().hipllm_route_groups(_ptr(ids), n, experts, vmax, _ptr(order), _ptr(groups), _ptr(ngroups),
                                    _stream(stream)))


def _k_gemm_gather(qtype, w, row_bytes, xh, xscale, y, n, k, ldy, order, groups, ngroups, max_groups, expert_stride,
                   routes, x_routed, stream=None):
    check(lib().hipllm_gemm_gather(qtype, _ptr(w), row_bytes, _ptr(xh), _ptr(xscale), _ptr(y), n, k, ldy, _ptr(order),
                                   _ptr(groups), _ptr(ngroups), max_groups, expert_stride, routes,
                                   1 if x_routed else 0, _stream(stream)))


def _k_router_topk(logits, ld, tokens, experts, k, ids, weights, stream=None):
    check(lib().hipllm_router_topk(_ptr(logits), ld, tokens, experts, k, _ptr(ids), _ptr(weights), _stream(stream)))


def _k_moe_combine(residual, down, w, shared, sgate, ld_sgate, out, tokens, h, k, stream=None):
    check(lib().hipllm_moe_combine(_ptr(residual), _ptr(down), _ptr(w), _ptr(shared), _ptr(sgate), ld_sgate,
                                   _ptr(out), tokens, h, k, _stream(stream)))


class GemvJob(ctypes.Structure):
    """HipllmGemvJob (include/hipllm.h)."""

    _fields_ = [("type", ctypes.c_uint32), ("mode", ctypes.c_uint32), ("w", ctypes.c_void_p),
                ("w2", ctypes.c_void_p), ("row_bytes", ctypes.c_size_t), ("bias", ctypes.c_void_p),
                ("residual", ctypes.c_void_p), ("y", ctypes.c_void_p), ("yq", ctypes.c_void_p),
                ("n", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


def _k_gemv_multi_norm(jobs, x, gamma, eps, k, norm=None, normq=None, stream=None):
    """jobs: dicts with type, mode (0/1), w, w2, row_bytes, bias, residual, y, yq, n."""
    arr = (GemvJob * max(1, len(jobs)))()
    for i, j in enumerate(jobs):
        arr[i] = GemvJob(j["type"], j.get("mode", 0), _ptr(j["w"]), _ptr(j.get("w2")), j["row_bytes"],
                         _ptr(j.get("bias")), _ptr(j.get("residual")), _ptr(j["y"]), _ptr(j.get("yq")), j["n"],
                         j.get("reserved", 0))
    check(lib().hipllm_gemv_multi_norm(arr, len(jobs), _ptr(x), _ptr(gamma), eps, k, _ptr(norm), _ptr(normq),
                                       _stream(stream)))


def _k_gemv_routed_swiglu(qtype, wg, wu, row_bytes, x, xq, ldx, y, yq, n, k, tokens, logits, ld_logits, experts,
                          routes, expert_stride, ids_out, weights_out, stream=None):
    check(lib().hipllm_gemv_routed_swiglu(qtype, _ptr(wg), _ptr(wu), row_bytes, _ptr(x), _ptr(xq), ldx, _ptr(y),
                                          _ptr(yq), n, k, tokens, _ptr(logits), ld_logits, experts, routes,
                                          expert_stride, _ptr(ids_out), _ptr(weights_out), _stream(stream)))


def _k_gemv_moe_combine(qtype, w, row_bytes, x, residual, down, weights, sgate, routes, y, n, k, stream=None):
    check(lib().hipllm_gemv_moe_combine(qtype, _ptr(w), row_bytes, _ptr(x), _ptr(residual), _ptr(down),
                                        _ptr(weights), _ptr(sgate), routes, _ptr(y), n, k, _stream(stream)))


def _k_moe_combine_norm(residual, down, w, shared, sgate, ld_sgate, out, gamma, norm, normq, tokens, h, k, eps,
                        stream=None):
    check(lib().hipllm_moe_combine_norm(_ptr(residual), _ptr(down), _ptr(w), _ptr(shared), _ptr(sgate), ld_sgate,
                                        _ptr(out), _ptr(gamma), _ptr(norm), _ptr(normq), tokens, h, k, eps,
                                        _stream(stream)))


def _k_gdn_gates(alpha, beta_raw, ld, dt_bias, a, decay, beta, tokens, heads, stream=None):
    check(lib().hipllm_gdn_gates(_ptr(alpha), _ptr(beta_raw), ld, _ptr(dt_bias), _ptr(a), _ptr(decay), _ptr(beta),
                                 tokens, heads, _stream(stream)))


def _k_conv1d_silu(x, ldx, history, w, out, ldo, tokens, channels, ksize, stream=None):
    check(lib().hipllm_conv1d_silu(_ptr(x), ldx, _ptr(history), _ptr(w), _ptr(out), ldo, tokens, channels, ksize,
                                   _stream(stream)))


def _k_l2norm_heads(x, ld, tokens, heads, d, eps, stream=None):
    check(lib().hipllm_l2norm_heads(_ptr(x), ld, tokens, heads, d, eps, _stream(stream)))


def _k_gdn_scan(q, k, ldqk, v, ldv, decay, beta, state, out, ldo, tokens, value_heads, key_heads, d, stream=None):
    check(lib().hipllm_gdn_scan(_ptr(q), _ptr(k), ldqk, _ptr(v), ldv, _ptr(decay), _ptr(beta), _ptr(state),
                                _ptr(out), ldo, tokens, value_heads, key_heads, d, _stream(stream)))


def _k_gdn_scan_chunked(q, k, ldqk, v, ldv, decay, beta, state, out, ldo, tokens, value_heads, key_heads, d, scratch,
                        stream=None):
    check(lib().hipllm_gdn_scan_chunked(_ptr(q), _ptr(k), ldqk, _ptr(v), ldv, _ptr(decay), _ptr(beta), _ptr(state),
                                        _ptr(out), ldo, tokens, value_heads, key_heads, d, _ptr(scratch),
                                        0 if scratch is None else scratch.numel(), _stream(stream)))


def _k_gated_rmsnorm(o, ldo, gamma, z, ldz, y, yq, ldy, tokens, heads, d, eps, stream=None):
    check(lib().hipllm_gated_rmsnorm(_ptr(o), ldo, _ptr(gamma), _ptr(z), ldz, _ptr(y), _ptr(yq), ldy, tokens,
                                     heads, d, eps, _stream(stream)))


def _k_conv_l2norm(x, ldx, history, w, out, ldo, tokens, channels, ksize, norm_channels, d, eps, stream=None):
    check(lib().hipllm_conv_l2norm(_ptr(x), ldx, _ptr(history), _ptr(w), _ptr(out), ldo, tokens, channels, ksize,
                                   norm_channels, d, eps, _stream(stream)))


def _k_gdn_scan_gated(q, k, ldqk, v, ldv, alpha, beta_raw, ld_ab, dt_bias, a, state, z, ldz, gamma, y, yq, ldy,
                      tokens, value_heads, key_heads, d, eps, stream=None):
    check(lib().hipllm_gdn_scan_gated(_ptr(q), _ptr(k), ldqk, _ptr(v), ldv, _ptr(alpha), _ptr(beta_raw), ld_ab,
                                      _ptr(dt_bias), _ptr(a), _ptr(state), _ptr(z), ldz, _ptr(gamma), _ptr(y), _ptr(yq),
                                      ldy, tokens, value_heads, key_heads, d, eps, _stream(stream)))


def _k_gdn_decode(qkv, x, x_gamma, ab_w, hidden, dt_bias, a, state, z, gamma, y, yq, value_heads, key_heads, d,
                  eps, stream=None):
    check(lib().hipllm_gdn_decode(_ptr(qkv), _ptr(x), _ptr(x_gamma), _ptr(ab_w), hidden, _ptr(dt_bias), _ptr(a),
                                  _ptr(state), _ptr(z), _ptr(gamma), _ptr(y), _ptr(yq), value_heads, key_heads, d, eps,
                                  _stream(stream)))


def _k_gemv_x16_pair(type_a, packed_a, n_a, y_a, type_b, packed_b, n_b, y_b, k, x, gamma, eps, conv_w=None,
                     history=None, ksize=0, xq=None, sumsq=None, stream=None):
    check(lib().hipllm_gemv_x16_pair(type_a, _ptr(packed_a), n_a, _ptr(y_a), type_b, _ptr(packed_b), n_b, _ptr(y_b), k,
                                     _ptr(x), _ptr(gamma), eps, _ptr(conv_w), _ptr(history), ksize, _ptr(xq),
                                     _ptr(sumsq), _stream(stream)))


def _k_split_qgate_norm(mixed, ldm, kv, ldkv, q_gamma, k_gamma, qkv, ldqkv, gate, ldg, tokens, hq, hkv, d, eps,
                        stream=None):
    check(lib().hipllm_split_qgate_norm(_ptr(mixed), ldm, _ptr(kv), ldkv, _ptr(q_gamma), _ptr(k_gamma), _ptr(qkv),
                                        ldqkv, _ptr(gate), ldg, tokens, hq, hkv, d, eps, _stream(stream)))


def _k_gate_mul(a, g, y, yq, n, stream=None):
    check(lib().hipllm_gate_mul(_ptr(a), _ptr(g), _ptr(y), _ptr(yq), n, _stream(stream)))


def _k_rmsnorm(x, gamma, y, yq, rows, cols, eps, stream=None):
    check(lib().hipllm_rmsnorm(_ptr(x), _ptr(gamma), _ptr(y), _ptr(yq), rows, cols, eps, _stream(stream)))


def _k_embed(qtype, table, row_bytes, ids, rows, vocab, cols, out, stream=None):
    check(lib().hipllm_embed(qtype, _ptr(table), row_bytes, _ptr(ids), rows, vocab, cols, _ptr(out),
                             _stream(stream)))


def _k_attn_decode_rope(qkv, cos_sin, rot, kcache, vcache, out, outq, scratch, hq, hkv, d, pos, scale, stream=None):
    check(lib().hipllm_attn_decode_rope(_ptr(qkv), _ptr(cos_sin), rot, _ptr(kcache), _ptr(vcache), _ptr(out),
                                        _ptr(outq), _ptr(scratch), hq, hkv, d, pos, scale, _stream(stream)))


def _k_rope_kv(qkv, cos_sin, rot, hq, hkv, d, pos0, rows, row_stride, kcache, vcache, stream=None):
    check(lib().hipllm_rope_kv(_ptr(qkv), _ptr(cos_sin), rot, hq, hkv, d, pos0, rows, row_stride, _ptr(kcache),
                               _ptr(vcache), _stream(stream)))


def _k_attn_decode_rope_gated(qkv, cos_sin, rot, kcache, vcache, gate, out, outq, scratch, hq, hkv, d, pos, scale,
                              stream=None):
    check(lib().hipllm_attn_decode_rope_gated(_ptr(qkv), _ptr(cos_sin), rot, _ptr(kcache), _ptr(vcache), _ptr(gate),
                                              _ptr(out), _ptr(outq), _ptr(scratch), hq, hkv, d, pos, scale,
                                              _stream(stream)))


def _k_attn_decode_qgate(mixed, kv, q_gamma, k_gamma, eps, cos_sin, rot, kcache, vcache, out, outq, hq, hkv, d, pos,
                         scale, stream=None):
    check(lib().hipllm_attn_decode_qgate(_ptr(mixed), _ptr(kv), _ptr(q_gamma), _ptr(k_gamma), eps, _ptr(cos_sin), rot,
                                         _ptr(kcache), _ptr(vcache), _ptr(out), _ptr(outq), hq, hkv, d, pos, scale,
                                         _stream(stream)))


def _k_attn_decode(q, kcache, vcache, out, outq, scratch, hq, hkv, d, length, scale, stream=None):
    check(lib().hipllm_attn_decode(_ptr(q), _ptr(kcache), _ptr(vcache), _ptr(out), _ptr(outq), _ptr(scratch),
                                   hq, hkv, d, length, scale, _stream(stream)))


def _k_argmax(x, n, out, scratch, stream=None):
    check(lib().hipllm_argmax(_ptr(x), n, _ptr(out), _ptr(scratch), _stream(stream)))


def _k_swiglu(g, u, y, yq, n, stream=None):
    check(lib().hipllm_swiglu(_ptr(g), _ptr(u), _ptr(y), _ptr(yq), n, _stream(stream)))


kernels = types.SimpleNamespace(
    dequant_rows=_k_dequant_rows, prep_x=_k_prep_x, gemv=_k_gemv, gemv_noalloc=_k_gemv_noalloc,
    gemv_prepped=_k_gemv_prepped, pack_x16=_k_pack_x16, gemv_x16=_k_gemv_x16, gemv_x16_swiglu=_k_gemv_x16_swiglu,
    gemv_x16_routed=_k_gemv_x16_routed,
    x16_bytes=lambda qtype, n, k: lib().hipllm_x16_bytes(qtype, n, k),
    gemv_swiglu=_k_gemv_swiglu, gemv_norm=_k_gemv_norm, gemv_swiglu_norm=_k_gemv_swiglu_norm, to_f16=_k_to_f16, gemm_mfma=_k_gemm_mfma, gemm=_k_gemm,
    gemm_workspace_bytes=lambda m, k: lib().hipllm_gemm_workspace_bytes(m, k), rmsnorm=_k_rmsnorm, embed=_k_embed, rope_kv=_k_rope_kv,
    attn_decode=_k_attn_decode, attn_decode_rope_gated=_k_attn_decode_rope_gated, argmax=_k_argmax,
    swiglu=_k_swiglu, attn_prefill=_k_attn_prefill,
    gemv_batched=_k_gemv_batched, matmul_f32=_k_matmul_f32,
    matmul_f32_scratch_floats=lambda m, n, k: lib().hipllm_matmul_f32_scratch_floats(m, n, k), route_groups=_k_route_groups, gemm_gather=_k_gemm_gather,
    route_groups_max=lambda n, e, v: lib().hipllm_route_groups_max(n, e, v), router_topk=_k_router_topk, moe_combine=_k_moe_combine,
    moe_combine_norm=_k_moe_combine_norm,
    gemv_multi_norm=_k_gemv_multi_norm, gemv_routed_swiglu=_k_gemv_routed_swiglu,
    gemv_moe_combine=_k_gemv_moe_combine, gdn_gates=_k_gdn_gates,
    conv1d_silu=_k_conv1d_silu, l2norm_heads=_k_l2norm_heads, gdn_scan=_k_gdn_scan, gated_rmsnorm=_k_gated_rmsnorm,
    gdn_scan_chunked=_k_gdn_scan_chunked,
    gdn_chunk_scratch_floats=lambda t, h: lib().hipllm_gdn_chunk_scratch_floats(t, h),
    conv_l2norm=_k_conv_l2norm, gdn_scan_gated=_k_gdn_scan_gated, gdn_decode=_k_gdn_decode,
    gemv_x16_pair=_k_gemv_x16_pair, gemv_x16_grouped=_k_gemv_x16_grouped, gemm_mfma_swiglu=_k_gemm_mfma_swiglu,
    gemm_mfma_swiglu_f16=_k_gemm_mfma_swiglu_f16,
    rmsnorm_f16=_k_rmsnorm_f16, attn_decode_qgate=_k_attn_decode_qgate, gemv_x16_moe_down=_k_gemv_x16_moe_down,
    split_qgate_norm=_k_split_qgate_norm, gate_mul=_k_gate_mul,
    gemv_workspace_bytes=lambda k: lib().hipllm_gemv_workspace_bytes(k),
    attn_decode_scratch_floats=lambda hq, d, n: lib().hipllm_attn_decode_scratch_floats(hq, d, n),
    attn_decode_rope=_k_attn_decode_rope,
    argmax_scratch_bytes=lambda n: lib().hipllm_argmax_scratch_bytes(n),
)
