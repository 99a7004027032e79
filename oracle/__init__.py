"""Python view of the CPU oracle (liboracle.so) and the compiled reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, as the checker or the timed CPU baseline. The
HipLLM product path never imports it.

``CpuOracle`` mirrors the reference's CPULLM interface (cpu_llm.h:165-194):
reset(), prefill(ids) -> int, decode(id) -> int, config, position,
max_sequence, and raises the Python analogue of the reference's exception for
each error (invalid_argument -> ValueError, out_of_range -> IndexError,
length_error -> OverflowError... see ``ERRORS``).
"""

from __future__ import annotations

import ctypes
import json
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_BIN = HERE / "_ref" / "ref_cpullm"


class LengthError(OverflowError):
    """std::length_error (capacity exceeded)."""


class OverflowErrorStd(OverflowError):
    """std::overflow_error."""


ERRORS = {1: ValueError, 2: IndexError, 3: LengthError, 4: RuntimeError, 5: OverflowErrorStd}


class OracleConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "layer_count", "embedding_size", "feed_forward_size", "attention_head_count",
        "kv_head_count", "head_size", "rotary_dimension", "vocabulary_size",
        "context_length", "parameter_count")] + [
        ("eos_token_id", ctypes.c_int32), ("rope_theta", ctypes.c_float),
        ("norm_epsilon", ctypes.c_float)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} is missing; run `make -C oracle`")
        L = ctypes.CDLL(str(LIB))
        c = ctypes
        P = c.c_void_p
        L.oracle_open.argtypes = [c.c_char_p, c.c_size_t, c.POINTER(P), c.c_char_p, c.c_size_t]
        L.oracle_close.argtypes = [P]
        L.oracle_config.argtypes = [P, c.POINTER(OracleConfig)]
        L.oracle_position.argtypes = [P]
        L.oracle_position.restype = c.c_size_t
        L.oracle_max_sequence.argtypes = [P]
        L.oracle_max_sequence.restype = c.c_size_t
        L.oracle_reset.argtypes = [P, c.c_char_p, c.c_size_t]
        L.oracle_prefill.argtypes = [P, P, c.c_size_t, c.POINTER(c.c_int32), P, c.c_char_p, c.c_size_t]
        L.oracle_decode.argtypes = [P, c.c_int32, c.POINTER(c.c_int32), P, c.c_char_p, c.c_size_t]
        L.oracle_tensor_f32.argtypes = [P, c.c_char_p, P, c.c_size_t, c.c_char_p, c.c_size_t]
        L.oracle_dequant_row.argtypes = [c.c_uint32, P, c.c_size_t, P]
        L.oracle_half_to_float.argtypes = [c.c_uint16]
        L.oracle_half_to_float.restype = c.c_float
        L.oracle_gevmt.argtypes = [P, P, P, c.c_size_t, c.c_size_t, P]
        L.oracle_rmsnorm.argtypes = [P, P, c.c_size_t, c.c_float]
        L.oracle_softmax.argtypes = [P, c.c_size_t]
        L.oracle_swiglu.argtypes = [P, P, c.c_size_t]
        L.oracle_ffn.argtypes = [P, P, P, P, c.c_size_t, c.c_size_t, P]
        L.oracle_rope.argtypes = [P, c.c_size_t, c.c_size_t, c.c_float, c.c_size_t]
        L.oracle_argmax.argtypes = [P, c.c_size_t]
        L.oracle_argmax.restype = c.c_int32
        _lib = L
    return _lib


def _check(rc: int, err) -> None:
    if rc:
        raise ERRORS.get(rc, RuntimeError)(err.value.decode(errors="replace"))


class CpuOracle:
    """CPULLM restated on the CPU, same contract as the reference class."""

    def __init__(self, gguf_path, max_sequence: int = 0):
        self._h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(1024)
        _check(lib().oracle_open(str(gguf_path).encode(), max_sequence, ctypes.byref(self._h), err, 1024), err)
        cfg = OracleConfig()
        lib().oracle_config(self._h, ctypes.byref(cfg))
        self.config = {n: getattr(cfg, n) for n, _ in OracleConfig._fields_}

    def close(self):
        if self._h:
            lib().oracle_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        return lib().oracle_position(self._h)

    @property
    def max_sequence(self) -> int:
        return lib().oracle_max_sequence(self._h)

    def reset(self):
        err = ctypes.create_string_buffer(1024)
        _check(lib().oracle_reset(self._h, err, 1024), err)

    def prefill(self, ids, logits: np.ndarray | None = None) -> int:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        tok = ctypes.c_int32()
        err = ctypes.create_string_buffer(1024)
        lp = None if logits is None else logits.ctypes.data
        _check(lib().oracle_prefill(self._h, a.ctypes.data, a.size, ctypes.byref(tok), lp, err, 1024), err)
        return tok.value

    def decode(self, token: int, logits: np.ndarray | None = None) -> int:
        tok = ctypes.c_int32()
        err = ctypes.create_string_buffer(1024)
        lp = None if logits is None else logits.ctypes.data
        _check(lib().oracle_decode(self._h, int(token), ctypes.byref(tok), lp, err, 1024), err)
        return tok.value

    def tensor(self, name: str, rows: int, cols: int) -> np.ndarray:
        out = np.empty((rows, cols), dtype=np.float32)
        err = ctypes.create_string_buffer(1024)
        _check(lib().oracle_tensor_f32(self._h, name.encode(), out.ctypes.data, out.size, err, 1024), err)
        return out


def dequant_rows(qtype: int, data: np.ndarray, cols: int) -> np.ndarray:
    """FP32 dequantization of [rows, row_bytes] quantized bytes (model.cpp:543-683)."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    rows = data.shape[0]
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        if lib().oracle_dequant_row(qtype, data[r].ctypes.data, cols, out[r].ctypes.data):
            raise RuntimeError("unsupported type or shape")
    return out


def gevmt(w: np.ndarray, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """Sequential FP32 y = W x (+ b), cpu_llm.cpp:512-547."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[0], dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_gevmt(w.ctypes.data, x.ctypes.data, None if b is None else b.ctypes.data,
                       w.shape[0], w.shape[1], y.ctypes.data)
    return y


def ffn(wg: np.ndarray, wu: np.ndarray, wd: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The decode-layer FFN in FP32, Wd (silu(Wg x) * (Wu x)) (cpu_llm.cpp:907-913),
    through the function the oracle's own decode step calls."""
    wg, wu, wd, x = (np.ascontiguousarray(a, dtype=np.float32) for a in (wg, wu, wd, x))
    f, h = wg.shape
    assert wu.shape == (f, h) and wd.shape == (h, f) and x.shape == (h,)
    out = np.empty(h, dtype=np.float32)
    lib().oracle_ffn(wg.ctypes.data, wu.ctypes.data, wd.ctypes.data, x.ctypes.data, h, f, out.ctypes.data)
    return out


def generate(model, prompt, max_new_tokens: int, stop_token_ids=(), logits_sink=None):
    """chat.cpp:831-878 generate(): prefill, then emit/decode up to the limit."""
    if len(prompt) == 0:
        raise ValueError("Generation requires at least one initial token")
    if max_new_tokens == 0:
        raise ValueError("Generation requires max_new_tokens > 0")
    if len(prompt) >= model.max_sequence:
        raise ValueError("Initial token sequence leaves no room for generated tokens")
    limit = min(max_new_tokens, model.max_sequence - len(prompt))
    model.reset()
    V = model.config["vocabulary_size"]
    logits = np.empty(V, dtype=np.float32) if logits_sink is not None else None
    nxt = model.prefill(prompt, logits)
    if logits_sink is not None:
        logits_sink(logits.copy())
    out = []
    for step in range(limit):
        if nxt in stop_token_ids:
            break
        out.append(nxt)
        if step + 1 >= limit:
            break
        nxt = model.decode(nxt, logits)
        if logits_sink is not None:
            logits_sink(logits.copy())
    return out


def run_reference(gguf_path, prompt, tokens: int, max_sequence: int = 0,
                  logits_path=None, timeout: float = 3600) -> dict:
    """Runs the compiled reference CPULLM (oracle/_ref/ref_cpullm)."""
    if not REF_BIN.exists():
        raise FileNotFoundError(f"{REF_BIN} not built (needs the reference sources)")
    cmd = [str(REF_BIN), str(gguf_path), "--prompt", ",".join(str(int(t)) for t in prompt),
           "--tokens", str(tokens)]
    if max_sequence:
        cmd += ["--max-sequence", str(max_sequence)]
    if logits_path:
        cmd += ["--logits", str(logits_path)]
    out = subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=timeout)
    return json.loads(out.stdout)
