"""Known-answer tests for the GGUF block formats and the synthetic inputs.

The oracle's dequantizer (a restatement of model.cpp:500-683) must reproduce
closed-form values of hand-built blocks (tests/blocks.py) exactly, and its
binary16 conversion must follow IEEE 754 for subnormals, infinities, signed
zero and NaN. The quantizers that make synthetic inputs are checked for the
properties any GGML quantizer has (round trip within half a quantization
step), not for byte equality with a particular ggml release.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from myllm_amd import synth
from tests import blocks


@pytest.mark.parametrize("case", range(4))
def test_dequant_known_answers(case):
    qtype, data, cols, expected = blocks.kat_rows()[case]
    got = oracle.dequant_rows(qtype, np.frombuffer(data, dtype=np.uint8)[None, :], cols)[0]
    assert np.array_equal(got.astype(np.float64), expected)


@pytest.mark.parametrize("bits,value", [
    (0x0000, 0.0), (0x8000, -0.0), (0x0001, 2.0 ** -24), (0x03FF, 1023 * 2.0 ** -24),
    (0x0400, 2.0 ** -14), (0x3C00, 1.0), (0xC000, -2.0), (0x7BFF, 65504.0),
    (0x7C00, math.inf), (0xFC00, -math.inf),
])
def test_half_to_float(bits, value):
    got = oracle.lib().oracle_half_to_float(bits)
    assert got == value and math.copysign(1.0, got) == math.copysign(1.0, value)


def test_half_nan():
    assert math.isnan(oracle.lib().oracle_half_to_float(0x7E00))
    assert math.isnan(oracle.lib().oracle_half_to_float(0xFD01))


@pytest.mark.parametrize("qtype,cols,block,step,rel", [
    (synth.Q8_0, 256, 32, 1 / 254, 0.008), (synth.Q5_0, 256, 32, 1 / 31, 0.06),
    (synth.Q4_K, 512, 32, 1 / 15, 0.09), (synth.Q6_K, 512, 16, 1 / 63, 0.025),
])
def test_quantizer_round_trip(qtype, cols, block, step, rel):
    w = synth.normal(64 * cols, seed=5, stddev=0.02).reshape(64, cols)
    q = synth.quantize(w, qtype)
    assert q.shape == (64, synth.row_bytes(qtype, cols))
    back = oracle.dequant_rows(qtype, q, cols)
    # Per element, the error stays within one quantization step of the
    # group's range (half a step for the symmetric formats).
    g = w.reshape(64, -1, block)
    span = g.max(axis=2, keepdims=True) - np.minimum(0, g.min(axis=2, keepdims=True))
    err = np.abs(back - w).reshape(64, -1, block)
    assert np.all(err <= span * step * 1.01 + 1e-7)
    assert np.linalg.norm(back - w) / np.linalg.norm(w) < rel


def test_random_source_is_deterministic_and_normal():
    a = synth.normal(100000, seed=11, stddev=2.0)
    b = synth.normal(100000, seed=11, stddev=2.0)
    assert np.array_equal(a, b)
    # Any slice can be generated on its own.
    assert np.array_equal(synth.normal(10, seed=11, stddev=2.0, first=500), a[500:510])
    assert abs(a.mean()) < 0.03 and abs(a.std() - 2.0) < 0.03
    ids = synth.uniform_ids(50000, 1000, seed=2)
    assert ids.min() >= 0 and ids.max() < 1000 and abs(ids.mean() - 499.5) < 10


def test_row_bytes():
    assert synth.row_bytes(synth.Q4_K, 3584) == 2016
    assert synth.row_bytes(synth.Q6_K, 18944) == 15540
    assert synth.row_bytes(synth.Q8_0, 896) == 952
    assert synth.row_bytes(synth.Q5_0, 896) == 616
    with pytest.raises(ValueError):
        synth.row_bytes(synth.Q4_K, 896)
