"""The XGroup activation format of the integer GEMV path, restated in numpy.

Definition (the kernels' common.h): every 16 consecutive values v of a GEMV
input become one 64-byte group

    s0[16], s1[16], s2[16]   signed-byte digits of q = s2 * 65536 + s1 * 256 + s0
    float32 sum              the FP32 sum of the 16 values
    float32 e                scale, e = max|v| / 8355711 (0 for an all-zero group)
    8 bytes padding

with q = round(v / e), |q| <= 8355711 (0x7f7f7f, the largest magnitude whose
balanced base-256 digits all fit a signed byte: s0, s1 in [-128, 127], s2 in
[-127, 127]), so |v - e q| is a few e, i.e. about 2^-23 of the group's
largest magnitude.

``decode`` reads groups written by the GPU; ``check`` asserts that groups
encode given FP32 values under that definition; ``encode`` builds groups on
the CPU (used to test the format's arithmetic without a GPU).
"""

from __future__ import annotations

import numpy as np

QMAX = 8355711
GROUP_BYTES = 64


def decode(raw) -> dict:
    """raw: bytes-like / uint8 array / torch tensor holding whole groups."""
    if hasattr(raw, "cpu"):
        raw = raw.cpu().numpy()
    b = np.ascontiguousarray(np.asarray(raw)).view(np.uint8).reshape(-1, GROUP_BYTES)
    s = b[:, :48].view(np.int8).reshape(-1, 3, 16).astype(np.int64)
    meta = b[:, 48:56].copy().view(np.float32).reshape(-1, 2)
    q = s[:, 2] * 65536 + s[:, 1] * 256 + s[:, 0]
    return {"s": s, "q": q, "sum": meta[:, 0], "e": meta[:, 1],
            "values": q.astype(np.float64) * meta[:, 1:2].astype(np.float64)}


def check(raw, values, groups: int | None = None) -> None:
    """Assert that the first ``groups`` groups of raw encode ``values``."""
    v = np.asarray(values, dtype=np.float32).reshape(-1, 16)
    if groups is not None:
        v = v[:groups]
    g = decode(raw)
    n = v.shape[0]
    s, q, e, total = g["s"][:n], g["q"][:n], g["e"][:n].astype(np.float64), g["sum"][:n].astype(np.float64)
    amax = np.abs(v).max(axis=1).astype(np.float64)
    assert np.all((s[:, :2] >= -128) & (s[:, :2] <= 127)), "low digit outside a signed byte"
    assert np.all(np.abs(s[:, 2]) <= 127), "high digit outside [-127, 127]"
    assert np.all(np.abs(q) <= QMAX)
    assert np.allclose(e, amax / QMAX, rtol=1e-6, atol=0.0), "scale e != max|v| / 8355711"
    err = np.abs(g["values"][:n] - v.astype(np.float64))
    assert np.all(err <= 4.0 * e[:, None] + 1e-37), f"value error {float((err / np.maximum(e[:, None], 1e-37)).max())} e"
    ref = v.astype(np.float64).sum(axis=1)
    mag = np.abs(v.astype(np.float64)).sum(axis=1)
    assert np.all(np.abs(total - ref) <= 1e-6 * mag + 1e-30), "group sum"


def encode(values) -> np.ndarray:
    """CPU restatement of the encoder: float32 values (multiple of 16) -> uint8 groups."""
    v = np.asarray(values, dtype=np.float32).reshape(-1, 16)
    amax = np.abs(v).max(axis=1)
    e = np.where(amax > 0, amax / np.float32(QMAX), np.float32(0)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(QMAX) / np.where(amax > 0, amax, 1), np.float32(0)).astype(np.float32)
    q = np.clip(np.rint(v * inv[:, None]), -QMAX, QMAX).astype(np.int64)
    d0 = ((q & 0xFF) ^ 0x80) - 0x80
    r = (q - d0) >> 8
    d1 = ((r & 0xFF) ^ 0x80) - 0x80
    d2 = (r - d1) >> 8
    out = np.zeros((v.shape[0], GROUP_BYTES), dtype=np.uint8)
    out[:, 0:16] = d0.astype(np.int8).view(np.uint8)
    out[:, 16:32] = d1.astype(np.int8).view(np.uint8)
    out[:, 32:48] = d2.astype(np.int8).view(np.uint8)
    meta = np.stack([v.sum(axis=1, dtype=np.float32), e], axis=1).astype(np.float32)
    out[:, 48:56] = meta.view(np.uint8).reshape(-1, 8)
    return out.reshape(-1)


def buffer(torch, k: int, device, rows: int = 1):
    """Device buffer for rows x (k / 16) groups (4 k bytes per row)."""
    return torch.empty(rows * k, dtype=torch.float32, device=device)
