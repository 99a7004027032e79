"""Writes the golden fixtures from the reference's own CPULLM.

Run in a container that holds the reference sources (``make -C oracle`` builds
oracle/_ref/ref_cpullm from them first). For each model the synthetic GGUF is
regenerated from its seed, its SHA-256 is recorded (so a later run can prove it
fed the same bytes), and the reference's greedy tokens and logits are stored:

* ``tiny_golden.npz``: 2-layer model using every block type (Q8_0 embedding,
  Q4_K attention Q/K/V and FFN gate/up, Q5_0 attention output, Q6_K ffn_down
  and output); 16-token prompt, 32 greedy tokens, the full logits of all 32
  steps.
* ``qwen2.5-0.5b_golden.npz``: the Qwen2.5-0.5B-shaped Q4_K_M model; 16-token
  prompt, 32 greedy tokens, and the top-64 (index, logit) pairs of every step.
* ``qwen2.5-7b_golden.npz``: the Qwen2.5-7B-shaped Q4_K_M model (28 layers,
  hidden 3584, FFN 18944); 8-token prompt, 16 greedy tokens, top-64 pairs of
  every step. Bounded so the reference's single-threaded CPULLM finishes in
  minutes (it holds about 35 GB of FP32 weights and file image).

Usage: python tests/golden/make_golden.py [--only tiny|qwen2.5-0.5b|qwen2.5-7b]
"""

from __future__ import annotations

import argparse
import pathlib
import sys
import tempfile

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from myllm_amd import synth  # noqa: E402

HERE = pathlib.Path(__file__).resolve().parent

CASES = {
    "tiny": dict(shape="tiny", types="all", seed=1, prompt_seed=7, prompt_len=16,
                 tokens=32, max_sequence=0, full_logits=True),
    "qwen2.5-0.5b": dict(shape="qwen2.5-0.5b", types="q4_k_m", seed=0, prompt_seed=0,
                         prompt_len=16, tokens=32, max_sequence=64, full_logits=False),
    "qwen2.5-7b": dict(shape="qwen2.5-7b", types="q4_k_m", seed=0, prompt_seed=3,
                       prompt_len=8, tokens=16, max_sequence=32, full_logits=False),
}


def model_path(case: str, directory) -> pathlib.Path:
    c = CASES[case]
    shape = synth.SHAPES[c["shape"]]
    types = synth.tiny_all_types() if c["types"] == "all" else synth.q4_k_m_types(shape)
    return synth.write_qwen2(pathlib.Path(directory) / f"{case}.gguf", shape, types, seed=c["seed"])


def prompt_ids(case: str) -> np.ndarray:
    c = CASES[case]
    return synth.uniform_ids(c["prompt_len"], synth.SHAPES[c["shape"]].vocab, seed=c["prompt_seed"])


def make(case: str) -> None:
    c = CASES[case]
    with tempfile.TemporaryDirectory() as tmp:
        path = model_path(case, tmp)
        sha = synth.file_sha256(path)
        prompt = prompt_ids(case)
        logits_file = pathlib.Path(tmp) / "logits.bin"
        res = oracle.run_reference(path, prompt, c["tokens"], c["max_sequence"], logits_file)
        if res["tokens"] != res["recomposed_tokens"]:
            raise SystemExit("reference CPULLM and the recomposed forward disagree")
        V = synth.SHAPES[c["shape"]].vocab
        logits = np.fromfile(logits_file, dtype=np.float32).reshape(-1, V)
        out = dict(prompt=prompt, tokens=np.asarray(res["tokens"], dtype=np.int32),
                   gguf_sha256=np.asarray(sha), seed=np.asarray(c["seed"]),
                   max_sequence=np.asarray(c["max_sequence"]))
        if c["full_logits"]:
            out["logits"] = logits
        else:
            top = np.argsort(-logits, axis=1, kind="stable")[:, :64].astype(np.int32)
            out["top_index"] = top
            out["top_logit"] = np.take_along_axis(logits, top, axis=1)
        np.savez_compressed(HERE / f"{case}_golden.npz", **out)
        print(case, sha, res["tokens"][:8], "...")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=sorted(CASES))
    args = ap.parse_args()
    for name in CASES:
        if args.only == name or (args.only is None and name != "qwen2.5-7b"):
            make(name)
