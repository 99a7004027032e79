"""hipllm_gemv_noalloc: the decode GEMV without a workspace or any allocation.

Called through the C ABI and compared with hipllm_gemv (caller workspace) on
the same inputs, bit for bit, on two calls in a row, the second smaller than
the first (the shared static scratch keeps the first call's contents, which
the second must not read). Also: k past the scratch's 65536 values is
rejected with HIPLLM_LENGTH_ERROR before anything is launched.
"""

from __future__ import annotations

import numpy as np
import pytest

from myllm_amd import synth
from myllm_amd.hipllm import LengthError, kernels
from tests.test_gpu_kernels import dev_bytes, random_rows

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _pair(cuda, qtype, n, k, seed, bias):
    w = random_rows(qtype, n, k, seed)
    dw = dev_bytes(w, cuda)
    x = torch.from_numpy(synth.normal(k, seed + 1)).to(cuda)
    b = torch.from_numpy(synth.normal(n, seed + 2)).to(cuda) if bias else None
    ws = torch.empty(kernels.gemv_workspace_bytes(k), dtype=torch.uint8, device=cuda)
    y_ws = torch.full((n,), float("nan"), device=cuda)
    y_na = torch.full((n,), float("nan"), device=cuda)
    kernels.gemv(qtype, dw, w.shape[1], x, b, y_ws, n, k, ws)
    kernels.gemv_noalloc(qtype, dw, w.shape[1], x, b, y_na, n, k)
    torch.cuda.synchronize()
    return y_ws.cpu().numpy(), y_na.cpu().numpy()


def test_gemv_noalloc_matches_workspace_entry(cuda):
    # A large call (Qwen2.5-7B down shape: k = 18944), then a smaller one.
    for qtype, n, k, seed, bias in ((synth.Q4_K, 3584, 18944, 5, False), (synth.Q6_K, 300, 1024, 9, True),
                                    (synth.Q8_0, 64, 256, 13, False)):
        a, b = _pair(cuda, qtype, n, k, seed, bias)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qtype, n, k)


def test_gemv_noalloc_rejects_k_past_scratch(cuda):
    w = torch.zeros(16, dtype=torch.uint8, device=cuda)
    x = torch.zeros(16, device=cuda)
    y = torch.zeros(1, device=cuda)
    with pytest.raises(LengthError, match="65536"):
        kernels.gemv_noalloc(synth.Q4_K, w, 144 * 257, x, None, y, 1, 65536 + 256)
