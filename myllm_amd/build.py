"""In-tree build of the native libraries.

* ``myllm_amd/lib/libhipllm.so``: HIP kernels for gfx950 + the HipLLM runtime
  + the C ABI (include/hipllm.h), compiled with hipcc.
* ``myllm_amd/lib/hipllm_chat``: the chat command (a ``main`` over
  ``hipllm_chat_main``), linked to libhipllm.so with an ``$ORIGIN`` rpath.
* ``myllm_amd/lib/libhipllm_tools.so``: host-only synthetic-input tools
  (include/hipllm_tools.h), compiled with g++.
* ``oracle/``: the CPU oracle and, when the reference sources are present,
  oracle/_ref (via ``make -C oracle``); test infrastructure, built here so one
  command prepares everything.

Every call recompiles (no staleness checks). Usage: ``python -m myllm_amd.build``.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"

ARCH = os.environ.get("HIPLLM_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 ops stay disabled for device code: the compiler would otherwise
# form v_pk_{add,mul,fma}_f32 from scalar float code.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-pthread"]

HIP_SOURCES = [
    "kernels/dequant.hip",
    "kernels/gemv.hip",
    "kernels/ops.hip",
    "kernels/prefill.hip",
    "kernels/moe.hip",
    "runtime/gguf_reader.cpp",
    "runtime/hip_llm.cpp",
    "runtime/hip_moe.cpp",
    "runtime/profile.cpp",
    "runtime/tokenizer.cpp",
    "runtime/hip_chat.cpp",
    "runtime/capi.cpp",
]
TOOLS_SOURCES = ["tools/quants.cpp", "tools/synth_gguf.cpp", "tools/tools_capi.cpp"]


def _run(cmd, cwd=None):
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "warning: feature flag")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}\n{res.stdout}")
    return err


def build_hipllm(jobs: int) -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    srcs = [s for s in HIP_SOURCES if (CSRC / s).exists()]

    def compile_one(src):
        obj = OBJ / (src.replace("/", "_") + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, srcs))
    out = LIB / "libhipllm.so"
    tmp = LIB / "libhipllm.so.tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    build_chat(out)
    return out


def build_chat(libhipllm: pathlib.Path) -> pathlib.Path:
    """The chat command, linked to libhipllm.so beside it."""
    out = LIB / "hipllm_chat"
    tmp = LIB / "hipllm_chat.tmp"
    _run([HIPCC, "-O2", "-std=c++17", str(CSRC / "runtime" / "chat_main.cpp"), f"-L{libhipllm.parent}", "-lhipllm",
          "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_tools() -> pathlib.Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libhipllm_tools.so"
    tmp = LIB / "libhipllm_tools.so.tmp"
    cxx = shutil.which("g++") or "c++"
    _run([cxx, *HOST_FLAGS, "-shared", *[str(CSRC / s) for s in TOOLS_SOURCES], "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_oracle() -> None:
    _run(["make", "-B", "-C", str(ROOT / "oracle"), "-j4"])


def build_all(jobs: int | None = None, oracle: bool = True) -> None:
    jobs = jobs or min(8, os.cpu_count() or 1)
    build_tools()
    build_hipllm(jobs)
    if oracle:
        build_oracle()


if __name__ == "__main__":
    build_all(oracle="--no-oracle" not in sys.argv)
    print("built:", ", ".join(p.name for p in sorted(LIB.glob("*.so"))))
