"""Locating and loading the in-tree native libraries.

The product library (``libhipllm.so``: HIP kernels, the HipLLM runtime and
its C ABI) and the host-only tools library (``libhipllm_tools.so``) are built
in-tree by ``myllm_amd.build`` into ``myllm_amd/lib``. Nothing here falls back
to another implementation: a missing library is an error.
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_DIR = pathlib.Path(__file__).resolve().parent / "lib"
HIPLLM_LIB = LIB_DIR / "libhipllm.so"
TOOLS_LIB = LIB_DIR / "libhipllm_tools.so"

_cache: dict[str, ctypes.CDLL] = {}


class NativeLibraryMissing(RuntimeError):
    """Raised when an in-tree native library has not been built."""


def _load(path: pathlib.Path) -> ctypes.CDLL:
    key = str(path)
    if key in _cache:
        return _cache[key]
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path} is missing; build it with `python -m myllm_amd.build` "
            "(or __graft_entry__.build())")
    lib = ctypes.CDLL(key, mode=ctypes.RTLD_GLOBAL)
    _cache[key] = lib
    return lib


def tools() -> ctypes.CDLL:
    lib = _load(TOOLS_LIB)
    if not getattr(lib, "_hipllm_typed", False):
        c = ctypes
        lib.hipllm_tools_row_bytes.restype = c.c_size_t
        lib.hipllm_tools_row_bytes.argtypes = [c.c_uint32, c.c_size_t]
        lib.hipllm_tools_quantize_rows.restype = c.c_int
        lib.hipllm_tools_quantize_rows.argtypes = [
            c.c_uint32, c.c_void_p, c.c_size_t, c.c_size_t, c.c_void_p, c.c_uint32]
        lib.hipllm_tools_fill_normal.restype = None
        lib.hipllm_tools_fill_normal.argtypes = [
            c.c_uint64, c.c_uint64, c.c_uint64, c.c_size_t, c.c_float, c.c_void_p]
        lib.hipllm_tools_fill_uniform_int.restype = None
        lib.hipllm_tools_fill_uniform_int.argtypes = [
            c.c_uint64, c.c_uint64, c.c_uint64, c.c_size_t, c.c_uint32, c.c_void_p]
        lib.hipllm_tools_write_qwen2.restype = c.c_int
        lib.hipllm_tools_write_qwen2.argtypes = [
            c.c_char_p, c.c_void_p, c.c_char_p, c.c_size_t]
        lib.hipllm_tools_write_qwen35moe.restype = c.c_int
        lib.hipllm_tools_write_qwen35moe.argtypes = [
            c.c_char_p, c.c_void_p, c.c_char_p, c.c_size_t]
        lib._hipllm_typed = True
    return lib


def hipllm() -> ctypes.CDLL:
    return _load(HIPLLM_LIB)
