"""CPU checks of the XGroup activation format the integer GEMV multiplies.

The GPU side (common.h xgroup_encode, gemv.hip dot3 / dot3_value) is tested
against the same definition in test_gpu_kernels.py; here the definition
itself is pinned: encoding error bounds, digit ranges, exactness of the
digit dot products and the int32 headroom the narrow (Q4_K) combine relies
on.
"""

from __future__ import annotations

import numpy as np

from tests import xgroup


def _values(seed, n=4096):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=n).astype(np.float32) * np.float32(3.0) ** rng.normal(scale=4.0, size=n).astype(np.float32)
    x[16:32] = 0.0
    x[100] = np.float32(-7e30)
    return x


def test_encode_meets_definition():
    for seed in range(4):
        x = _values(seed)
        xgroup.check(xgroup.encode(x), x)


def test_extreme_digits_round_trip():
    # +-QMAX, one unit, and the balanced-digit carry cases.
    v = np.array([1.0, -1.0, 0.5, -0.5, 1 / 8355711, -1 / 8355711, 128 / 8355711, -128 / 8355711,
                  255 / 8355711, 256 / 8355711, 32767 / 8355711, 32768 / 8355711, -65535 / 8355711,
                  0.999999, -0.999999, 0.0], dtype=np.float32)
    g = xgroup.decode(xgroup.encode(v))
    assert g["q"][0][0] == 8355711 and g["q"][0][1] == -8355711
    assert np.all(np.abs(g["s"][:, 2]) <= 127) and np.all(np.abs(g["s"]) <= 128)
    xgroup.check(xgroup.encode(v), v)


def test_digit_dots_are_exact_and_fit_int32():
    rng = np.random.default_rng(5)
    x = _values(9, 16 * 64)
    g = xgroup.decode(xgroup.encode(x))
    s = g["s"]  # [groups, 3, 16]
    for lo, hi, narrow in ((0, 15, True), (0, 63, False), (-128, 127, False), (0, 31, False)):
        q = rng.integers(lo, hi + 1, size=(s.shape[0], 16))
        a = (q[:, None, :] * s).sum(axis=2)  # per-digit sums, as v_dot4 chains produce them
        assert np.all(np.abs(a) < 2**31)
        exact = (q * g["q"]).sum(axis=1)
        if narrow:
            # (a0 + (a1 << 8)) + (a2 << 16) evaluated in int32 must not wrap.
            bound = 16 * 15 * (127 * 65536 + 128 * 256 + 128)
            assert bound < 2**31
            assert np.all(a[:, 0] + a[:, 1] * 256 + a[:, 2] * 65536 == exact)
        else:
            lo_part = a[:, 0] + a[:, 1] * 256
            assert np.all(np.abs(lo_part) < 2**31)
            assert np.all(lo_part + a[:, 2] * 65536 == exact)
    # The GEMV value e * sum(q * q_x) is the dot with the encoded input.
    q = rng.integers(0, 16, size=(s.shape[0], 16))
    ref = (q * x.reshape(-1, 16).astype(np.float64)).sum(axis=1)
    got = g["e"].astype(np.float64) * (q * g["q"]).sum(axis=1)
    # Per value |x - e q_x| <= 4 e = 4 max|x| / 8355711 (the group's largest magnitude).
    scale = np.abs(q).sum(axis=1) * np.abs(x.reshape(-1, 16)).max(axis=1).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 4.0 / 8355711 * scale + 1e-30)
