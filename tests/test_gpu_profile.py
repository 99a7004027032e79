"""enable_profiling on the GPU: the reference's operator table and its
command / kernel / operation sidecars (profiler.cpp:127-174, 619-632), filled
from HIP events, for both backends, with and without per-launch timing."""

from __future__ import annotations

import csv

import pytest

from myllm_amd import synth
from myllm_amd.hipllm import HipLLM, generate

pytestmark = pytest.mark.gpu


def read(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def profile_run(path, tmp_path, detailed, tokens=4, prompt=None):
    csv_path = tmp_path / "llm_profile.csv"
    with HipLLM(path, 64) as m:
        m.enable_profiling(csv_path, detailed)
        out = generate(m, prompt or [1, 2, 3, 4, 5], tokens)
        m.disable_profiling()
    stem = tmp_path / "llm_profile"
    return out, read(csv_path), read(f"{stem}_metal_commands.csv"), read(f"{stem}_metal_kernels.csv"), \
        read(f"{stem}_metal_ops.csv")


@pytest.mark.parametrize("detailed", [False, True])
def test_dense_profile_tables(cuda, golden_model, tmp_path, detailed):
    path, g = golden_model("tiny")
    out, table, commands, kernels, ops = profile_run(path, tmp_path, detailed)
    forwards = len(out)  # prefill + (tokens - 1) decodes
    assert len(out) == 4
    per = [r for r in table if r["record_type"] in ("forward_total", "forward_stage")]
    assert len(per) == 2 * forwards
    stages = [r["stage"] for r in per if r["record_type"] == "forward_stage"]
    assert stages == ["prefill.gpu_resident"] + ["decode.gpu_resident"] * (forwards - 1)
    assert [int(r["sequence_tokens"]) for r in per if r["record_type"] == "forward_total"] == \
        [5] + list(range(6, 5 + forwards))
    for r in per:
        assert float(r["time_ms"]) > 0 and int(r["flops"]) > 0 and int(r["read_bytes"]) > 0
    glob = {r["stage"]: r for r in table if r["record_type"] == "global"}
    assert set(glob) == {"forward.total", "prefill.gpu_resident", "decode.gpu_resident"}
    assert int(glob["forward.total"]["calls"]) == forwards
    # Decode logical flops grow with the keys attended.
    dec = [int(r["flops"]) for r in per if r["record_type"] == "forward_total"][1:]
    assert dec == sorted(dec) and dec[0] < dec[-1]
    assert len(commands) == forwards
    for c in commands:
        assert int(c["kernel_count"]) > 0 and int(c["threadgroups"]) > 0 and float(c["gpu_duration_ms"]) > 0
        assert c["counter_requested"] == ("1" if detailed else "0")
    if detailed:
        assert len(kernels) > 0
        assert {k["operation"] for k in kernels} >= {"embedding", "argmax", "RoPE/KV write + attention"}
        assert all(float(k["gpu_duration_us"]) >= 0 and int(k["threadgroups"]) > 0 for k in kernels)
        total = sum(int(o["calls"]) for o in ops)
        assert total == len(kernels)
    else:
        assert kernels == [] and ops == []


def test_moe_profile_stage_names(cuda, tmp_path):
    path = synth.write_qwen35moe(tmp_path / "moe.gguf", synth.MOE_SHAPES["moe-tiny"], seed=3)
    out, table, commands, kernels, ops = profile_run(path, tmp_path, True, tokens=3)
    stages = [r["stage"] for r in table if r["record_type"] == "forward_stage"]
    assert stages == ["prefill.gpu_moe", "decode.gpu_moe", "decode.gpu_moe"]
    assert len(commands) == 3 and all(int(c["kernel_count"]) > 0 for c in commands)
    assert len(kernels) > 0 and len(ops) > 0
