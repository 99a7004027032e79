"""Kernel parity on the GPU, called through the C ABI (libhipllm.so).

Bars (from the project's correctness contract):
* dequantization, embedding gather, RMSNorm and RoPE: bit-exact against the
  CPU oracle (the restatement of CPULLM, itself pinned to the reference's
  golden vectors);
* GEMV: rel_err = max|y - ref| / max|ref| <= 1e-3, ref = float64 product of
  the FP32-dequantized weights and the FP32 input (the GEMV reads the input in
  its XGroup form, 24-bit fixed point per 16 values, see tests/xgroup.py);
* producers of GEMV inputs write that form: checked against its definition;
* attention, SwiGLU: same rel_err bound against float64;
* argmax: exact index, ties to the lower index.
Device weight buffers get 256 bytes of tail padding, as the runtime's arena
does, because realigned dword loads may read past the last block.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import oracle
from myllm_amd import synth
from myllm_amd.hipllm import kernels
from tests import blocks, xgroup

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

PAD = 256


def dev_bytes(arr: np.ndarray, cuda):
    flat = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    buf = torch.zeros(flat.size + PAD, dtype=torch.uint8, device=cuda)
    buf[: flat.size] = torch.from_numpy(flat.copy()).to(cuda)
    return buf


def rel_err(y, ref) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def random_rows(qtype, rows, cols, seed):
    if qtype == synth.F32:
        return synth.normal(rows * cols, seed, stddev=0.02).reshape(rows, cols).view(np.uint8).reshape(rows, -1)
    if qtype == synth.F16:
        return synth.normal(rows * cols, seed, stddev=0.02).reshape(rows, cols).astype(np.float16).view(
            np.uint8).reshape(rows, -1)
    return synth.random_quantized(rows, cols, qtype, seed)


# ------------------------------------------------------------- dequant
DEQ_SHAPES = [
    (synth.Q4_K, 7, 512), (synth.Q4_K, 3, 3584), (synth.Q6_K, 5, 4864), (synth.Q6_K, 3, 512),
    (synth.Q8_0, 9, 96), (synth.Q8_0, 4, 896), (synth.Q5_0, 6, 96), (synth.Q5_0, 3, 896),
    (synth.F16, 4, 256), (synth.F32, 3, 64),
]


@pytest.mark.parametrize("qtype,rows,cols", DEQ_SHAPES)
def test_dequant_bit_exact(cuda, qtype, rows, cols):
    w = random_rows(qtype, rows, cols, seed=rows * 100 + cols)
    dw = dev_bytes(w, cuda)
    out = torch.empty(rows * cols, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(qtype, dw, w.shape[1], rows, cols, out)
    got = out.cpu().numpy().reshape(rows, cols)
    ref = oracle.dequant_rows(qtype, w, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("case", range(4))
def test_dequant_known_answers(cuda, case):
    qtype, data, cols, expected = blocks.kat_rows()[case]
    w = np.frombuffer(data, dtype=np.uint8)[None, :]
    out = torch.empty(cols, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(qtype, dev_bytes(w, cuda), w.shape[1], 1, cols, out)
    assert np.array_equal(out.cpu().numpy().astype(np.float64), expected)


def test_dequant_special_halves(cuda):
    # Q8_0 blocks whose scale is a subnormal, infinite or NaN binary16.
    qs = np.arange(1, 33, dtype=np.int8)
    data = b"".join(blocks.f16(b) + qs.tobytes() for b in (0x0001, 0x03FF, 0x7C00, 0xFC00, 0x8000, 0x7E00))
    w = np.frombuffer(data, dtype=np.uint8)[None, :]
    out = torch.empty(192, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(synth.Q8_0, dev_bytes(w, cuda), w.shape[1], 1, 192, out)
    got = out.cpu().numpy()
    ref = oracle.dequant_rows(synth.Q8_0, w, 192)[0]
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))


# ------------------------------------------------------------- GEMV
def gemv_case(cuda, qtype, n, k, seed, bias=False, residual=False, tiling=0):
    w = random_rows(qtype, n, k, seed)
    x = synth.normal(k, seed + 1)
    dw = dev_bytes(w, cuda)
    dx = torch.from_numpy(x).to(cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(dx, xq, k)
    b = synth.normal(n, seed + 2) if bias else None
    r = synth.normal(n, seed + 3) if residual else None
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_prepped(qtype, dw, w.shape[1], dx, xq, None if b is None else torch.from_numpy(b).to(cuda),
                         None if r is None else torch.from_numpy(r).to(cuda), y, n, k, tiling)
    # Reference: float64 over the FP32 dequantized weights (GPU dequant is
    # bit-exact to the oracle, checked above).
    wf = torch.empty(n * k, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(qtype, dw, w.shape[1], n, k, wf)
    ref = (wf.view(n, k).double() @ dx.double()).cpu().numpy()
    if b is not None:
        ref = ref + b
    if r is not None:
        ref = ref + r
    return y.cpu().numpy(), ref


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K, synth.Q8_0, synth.Q5_0, synth.F16, synth.F32])
@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (130, 1024), (333, 2816)])
def test_gemv_small(cuda, qtype, n, k):
    y, ref = gemv_case(cuda, qtype, n, k, seed=n + k)
    assert rel_err(y, ref) <= 1e-3


@pytest.mark.parametrize("qtype", [synth.Q5_0, synth.Q8_0])
@pytest.mark.parametrize("k", [32, 64 * 3, 800, 896])
def test_gemv_ragged_two_byte_aligned_blocks(cuda, qtype, k):
    # 34- and 22-byte blocks: every odd block starts at a 2-byte offset. A
    # unit is 4 blocks: k = 32, 192 and 800 leave a last unit of 1, 2 and 1
    # blocks (lanes past the row must contribute nothing).
    y, ref = gemv_case(cuda, qtype, 77, k, seed=3 + k)
    assert rel_err(y, ref) <= 1e-3


def test_prep_x_encodes_xgroups(cuda):
    # Magnitudes spanning many binades, exact zeros, a zero group and a
    # group with one huge outlier.
    k = 4096
    x = synth.normal(k, 5) * np.float32(3.0) ** synth.normal(k, 6, stddev=4.0).astype(np.float32)
    x[16:32] = 0.0
    x[40] = 0.0
    x[64:80] *= np.float32(1e-20)
    x[96] = np.float32(3e30)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(torch.from_numpy(x.astype(np.float32)).to(cuda), xq, k)
    xgroup.check(xq, x)
    got = xgroup.decode(xq)
    assert np.all(got["q"][1] == 0) and got["e"][1] == 0.0


TILINGS = [108, 116, 132, 202, 204, 208, 216, 232, 401, 402, 404, 408, 416, 432, 802, 804, 808, 816, 832]
SWIGLU_TILINGS = [202, 204, 401, 402, 404, 408, 802, 804, 808, 816]


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K, synth.Q8_0, synth.Q5_0, synth.F16, synth.F32])
@pytest.mark.parametrize("tiling", TILINGS)
def test_gemv_tilings_agree(cuda, qtype, tiling):
    # 1001 rows: no tiling divides it, so every one has a partial last block.
    y, ref = gemv_case(cuda, qtype, 1001, 2048, seed=7, bias=True, residual=True, tiling=tiling)
    assert rel_err(y, ref) <= 1e-3


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K, synth.Q8_0])
@pytest.mark.parametrize("tiling", [116, 216, 232, 416])
@pytest.mark.parametrize("k", [4864, 18944])
def test_gemv_wave_split_tilings(cuda, qtype, tiling, k):
    # OPR 16 / 32: a row group spans 2 / 4 waves whose partials meet in LDS;
    # 19 and 74 super-blocks split unevenly over the octets.
    y, ref = gemv_case(cuda, qtype, 1001, k, seed=tiling, bias=True, residual=True, tiling=tiling)
    assert rel_err(y, ref) <= 1e-3


@pytest.mark.parametrize("tiling", [12, 28, 2412, 103, 1616])
def test_gemv_rejects_unknown_tilings(cuda, tiling):
    with pytest.raises(ValueError):
        gemv_case(cuda, synth.Q4_K, 64, 1024, seed=1, tiling=tiling)


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K])
@pytest.mark.parametrize("n,k", [(18944, 3584), (3584, 18944), (4608, 3584)])
def test_gemv_qwen7b_shapes(cuda, qtype, n, k):
    y, ref = gemv_case(cuda, qtype, n, k, seed=11)
    assert rel_err(y, ref) <= 1e-3


def test_gemv_qwen05b_q6k_down(cuda):
    # K = 4864: Q6_K rows of 3990 bytes, so rows alternate 4- and 2-byte alignment.
    y, ref = gemv_case(cuda, synth.Q6_K, 896, 4864, seed=5, residual=True)
    assert rel_err(y, ref) <= 1e-3


def test_gemv_public_entry_with_workspace(cuda):
    n, k = 300, 1024
    w = random_rows(synth.Q4_K, n, k, 21)
    x = synth.normal(k, 22)
    dw, dx = dev_bytes(w, cuda), torch.from_numpy(x).to(cuda)
    ws = torch.empty(kernels.gemv_workspace_bytes(k), dtype=torch.uint8, device=cuda)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv(synth.Q4_K, dw, w.shape[1], dx, None, y, n, k, ws)
    ref = oracle.dequant_rows(synth.Q4_K, w, k).astype(np.float64) @ x.astype(np.float64)
    assert rel_err(y.cpu().numpy(), ref) <= 1e-3


def swiglu_case(cuda, qtype, n, k, tiling=0, with_yq=True):
    wg, wu = random_rows(qtype, n, k, 31), random_rows(qtype, n, k, 32)
    x = synth.normal(k, 33)
    dx = torch.from_numpy(x).to(cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(dx, xq, k)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, n, cuda) if with_yq else None
    kernels.gemv_swiglu(qtype, dev_bytes(wg, cuda), dev_bytes(wu, cuda), wg.shape[1], dx, xq, y, yq, n, k, tiling)
    g = oracle.dequant_rows(qtype, wg, k).astype(np.float64) @ x
    u = oracle.dequant_rows(qtype, wu, k).astype(np.float64) @ x
    ref = g / (1 + np.exp(-g)) * u
    got = y.cpu().numpy()
    assert rel_err(got, ref) <= 1e-3
    if with_yq:
        xgroup.check(yq, got)


@pytest.mark.parametrize("qtype,n,k", [(synth.Q4_K, 4864, 1024), (synth.Q4_K, 2048, 3584),
                                        (synth.Q4_K, 18944, 3584), (synth.Q6_K, 1040, 5120),
                                        (synth.Q5_0, 480, 896), (synth.Q8_0, 512, 2048)])
def test_gemv_swiglu(cuda, qtype, n, k):
    swiglu_case(cuda, qtype, n, k)


@pytest.mark.parametrize("tiling", TILINGS)
@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K])
def test_gemv_swiglu_tilings(cuda, qtype, tiling):
    # 1040 rows: a partial last block for every rows-per-block choice. The
    # XGroup output needs blocks owning whole 16-groups (SWIGLU_TILINGS); the
    # other tilings reject it and compute y alone.
    if tiling in SWIGLU_TILINGS:
        swiglu_case(cuda, qtype, 1040, 2048, tiling)
    else:
        with pytest.raises(ValueError):
            swiglu_case(cuda, qtype, 1040, 2048, tiling)
        swiglu_case(cuda, qtype, 1040, 2048, tiling, with_yq=False)


# ------------------------------------------------------------- norm prologue
@pytest.mark.parametrize("tiling", [0, 208, 216, 408, 416])
@pytest.mark.parametrize("qtype,n,k", [(synth.Q4_K, 4608, 3584), (synth.Q6_K, 1040, 5120), (synth.Q8_0, 1152, 896),
                                        (synth.Q5_0, 300, 896)])
def test_gemv_norm_matches_rmsnorm_then_gemv(cuda, qtype, n, k, tiling):
    # The norm in the GEMV's prologue against hipllm_rmsnorm followed by the
    # GEMV on its XGroup output (bias and residual included): the same
    # arithmetic in two separately compiled kernels (FMA contraction may round
    # differently), so within 1e-6.
    w = random_rows(qtype, n, k, 81)
    dw = dev_bytes(w, cuda)
    x = torch.from_numpy(synth.normal(k, 82, stddev=3.0)).to(cuda)
    g = torch.from_numpy(synth.normal(k, 83, stddev=0.5) + 1.0).to(cuda)
    b = torch.from_numpy(synth.normal(n, 84)).to(cuda)
    r = torch.from_numpy(synth.normal(n, 85)).to(cuda)
    y1 = torch.empty(n, dtype=torch.float32, device=cuda)
    y2 = torch.empty(n, dtype=torch.float32, device=cuda)
    xn = torch.empty(k, dtype=torch.float32, device=cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.rmsnorm(x, g, xn, xq, 1, k, 1e-6)
    kernels.gemv_prepped(qtype, dw, w.shape[1], xn, xq, b, r, y1, n, k, tiling)
    kernels.gemv_norm(qtype, dw, w.shape[1], x, g, 1e-6, b, r, y2, n, k, tiling)
    got, ref = y2.cpu().numpy(), y1.cpu().numpy()
    print("max rel diff", rel_err(got, ref))
    assert rel_err(got, ref) <= 1e-6


@pytest.mark.parametrize("tiling", [204, 408])
@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K, synth.Q8_0])
def test_gemv_swiglu_norm_matches_rmsnorm_then_swiglu(cuda, qtype, tiling):
    n, k = 1040, 3584 if qtype != synth.Q8_0 else 896
    wg, wu = random_rows(qtype, n, k, 86), random_rows(qtype, n, k, 87)
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    x = torch.from_numpy(synth.normal(k, 88, stddev=2.0)).to(cuda)
    g = torch.from_numpy(synth.normal(k, 89, stddev=0.5) + 1.0).to(cuda)
    xn = torch.empty(k, dtype=torch.float32, device=cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.rmsnorm(x, g, xn, xq, 1, k, 1e-6)
    outs = []
    for fused in (False, True):
        y = torch.empty(n, dtype=torch.float32, device=cuda)
        yq = xgroup.buffer(torch, n, cuda)
        if fused:
            kernels.gemv_swiglu_norm(qtype, dg, du, wg.shape[1], x, g, 1e-6, y, yq, n, k, tiling)
        else:
            kernels.gemv_swiglu(qtype, dg, du, wg.shape[1], xn, xq, y, yq, n, k, tiling)
        outs.append((y.cpu().numpy(), yq.cpu().numpy()))
    print("max rel diff", rel_err(outs[1][0], outs[0][0]))
    assert rel_err(outs[1][0], outs[0][0]) <= 1e-6
    xgroup.check(outs[1][1], outs[1][0])


MULTI_CASES = {
    # DeltaNet decode shape: QKV, z, alpha/beta (F32) of one normalised row
    "deltanet": (2048, [(synth.Q6_K, 0, 1000), (synth.Q4_K, 0, 520), (synth.F32, 0, 64)]),
    # attention: Q/gate with bias and residual, packed K/V
    "attention": (1024, [(synth.Q4_K, 0, 777), (synth.Q8_0, 0, 256)]),
    # router (E + 1 rows) and shared gate/up + SwiGLU with its XGroup form
    "router": (2048, [(synth.F32, 0, 257), (synth.Q8_0, 1, 512)]),
    # SwiGLU of every quantized type, ragged Q5_0 rows (27 blocks)
    "swiglu": (768, [(synth.Q4_K, 1, 48), (synth.Q6_K, 1, 32), (synth.Q5_0, 0, 100)]),
    "ragged": (864, [(synth.Q8_0, 1, 64), (synth.Q5_0, 0, 33)]),
    # mode 2 here: SwiGLU without the XGroup output (4-row blocks), ragged row counts
    "swiglu_fp32": (1024, [(synth.F32, 0, 257), (synth.Q8_0, 2, 510), (synth.Q6_K, 2, 37)]),
    "swiglu_fp32_q4": (512, [(synth.Q4_K, 2, 130), (synth.Q5_0, 2, 64)]),
}


@pytest.mark.parametrize("case", sorted(MULTI_CASES))
def test_gemv_multi_norm_matches_rmsnorm_then_gemvs(cuda, case):
    # Every job of the grouped launch against hipllm_rmsnorm followed by the
    # single GEMV (tiling 208 / 132) or SwiGLU GEMV (204, 108) on its output:
    # the same arithmetic in separately compiled kernels, so within 1e-6;
    # the stored norm and its XGroup form bit for bit.
    k, specs = MULTI_CASES[case]
    x = torch.from_numpy(synth.normal(k, 91, stddev=3.0)).to(cuda)
    g = torch.from_numpy(synth.normal(k, 92, stddev=0.5) + 1.0).to(cuda)
    xn = torch.empty(k, dtype=torch.float32, device=cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.rmsnorm(x, g, xn, xq, 1, k, 1e-6)
    jobs, refs = [], []
    for i, (qtype, mode, n) in enumerate(specs):
        w = random_rows(qtype, n, k, 100 + i)
        dw = dev_bytes(w, cuda)
        rb = w.shape[1]
        y = torch.full((n,), float("nan"), device=cuda)
        yref = torch.empty(n, device=cuda)
        j = dict(type=qtype, mode=min(mode, 1), w=dw, row_bytes=rb, y=y, n=n)
        if mode >= 1:
            du = dev_bytes(random_rows(qtype, n, k, 200 + i), cuda)
            j["w2"] = du
            yq = xgroup.buffer(torch, n, cuda) if n % 16 == 0 and mode == 1 else None
            j["yq"] = yq
            kernels.gemv_swiglu(qtype, dw, du, rb, xn, xq, yref, None, n, k, 204 if mode == 1 else 108)
        else:
            b = torch.from_numpy(synth.normal(n, 300 + i)).to(cuda) if i == 0 else None
            r = torch.from_numpy(synth.normal(n, 400 + i)).to(cuda) if i == 0 else None
            j["bias"], j["residual"] = b, r
            kernels.gemv_prepped(qtype, dw, rb, xn, xq, b, r, yref, n, k, 132 if qtype == synth.F32 else 208)
        jobs.append(j)
        refs.append(yref)
    norm = torch.empty(k, device=cuda)
    normq = xgroup.buffer(torch, k, cuda)
    kernels.gemv_multi_norm(jobs, x, g, 1e-6, k, norm, normq)
    assert torch.equal(norm.view(torch.int32), xn.view(torch.int32))
    assert torch.equal(normq.view(torch.int32), xq.view(torch.int32))
    for j, yref in zip(jobs, refs):
        got, ref = j["y"].cpu().numpy(), yref.cpu().numpy()
        print(case, j["type"], j["mode"], "max rel diff", rel_err(got, ref))
        assert rel_err(got, ref) <= 1e-6
        if j.get("yq") is not None:
            xgroup.check(j["yq"], got)


def test_gemv_multi_norm_rejects_bad_arguments(cuda):
    k = 256
    w = torch.zeros(1024 * 64, dtype=torch.uint8, device=cuda)
    x = torch.ones(9216, device=cuda)
    y = torch.zeros(64, device=cuda)
    ok = dict(type=synth.Q8_0, mode=0, w=w, row_bytes=272, y=y, n=16)
    kernels.gemv_multi_norm([ok], x, x, 1e-6, k)  # valid
    torch.cuda.synchronize()
    bad_jobs = [
        [ok] * 4,                                                    # at most 3 jobs
        [dict(ok, type=synth.F16, row_bytes=512)],                   # no F16 form
        [dict(ok, type=synth.F32, row_bytes=1024, mode=1, w2=w)],    # F32 only in mode 0
        [dict(ok, mode=1)],                                          # SwiGLU without W2
        [dict(ok, mode=1, w2=w, yq=y, n=20)],                        # XGroup output needs n % 16 == 0
        [dict(ok, yq=y)],                                            # XGroup output only in mode 1
        [dict(ok, reserved=1)],
        [dict(ok, row_bytes=100)],                                   # rows shorter than k
    ]
    for jobs in bad_jobs:
        with pytest.raises(ValueError):
            kernels.gemv_multi_norm(jobs, x, x, 1e-6, k)
    with pytest.raises(ValueError):  # k beyond the 8192-value prologue
        kernels.gemv_multi_norm([dict(ok, row_bytes=9792)], x, x, 1e-6, 9216)
    with pytest.raises(ValueError):  # eps must be positive
        kernels.gemv_multi_norm([ok], x, x, 0.0, k)


@pytest.mark.parametrize("qtype,n,k", [(synth.Q8_0, 2048, 512), (synth.Q4_K, 300, 768), (synth.Q6_K, 64, 2048)])
def test_gemv_norm_without_gain_encodes_x(cuda, qtype, n, k):
    # gamma = None: the prologue only encodes x, against hipllm_prep_x then
    # the GEMV (separately compiled, so within 1e-6).
    w = random_rows(qtype, n, k, 93)
    dw = dev_bytes(w, cuda)
    x = torch.from_numpy(synth.normal(k, 94, stddev=2.0)).to(cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(x, xq, k)
    y1 = torch.empty(n, device=cuda)
    y2 = torch.empty(n, device=cuda)
    kernels.gemv_prepped(qtype, dw, w.shape[1], x, xq, None, None, y1, n, k, 208)
    kernels.gemv_norm(qtype, dw, w.shape[1], x, None, 0.0, None, None, y2, n, k, 208)
    assert rel_err(y2.cpu().numpy(), y1.cpu().numpy()) <= 1e-6


def test_gemv_norm_rejects_bad_arguments(cuda):
    w = torch.zeros(144 * 40, dtype=torch.uint8, device=cuda)
    x = torch.zeros(9216, device=cuda)
    y = torch.zeros(4, device=cuda)
    with pytest.raises(ValueError):  # k beyond the 8192-value LDS prologue
        kernels.gemv_norm(synth.Q4_K, w, 144 * 36, x, x, 1e-6, None, None, y, 4, 9216)
    with pytest.raises(ValueError):  # float weights have no norm form
        kernels.gemv_norm(synth.F32, w, 1024, x, x, 1e-6, None, None, y, 4, 256)
    with pytest.raises(ValueError):  # unknown norm tiling
        kernels.gemv_norm(synth.Q4_K, w, 144, x, x, 1e-6, None, None, y, 4, 256, 432)
    for code in (100, 7, 1416):  # malformed codes are rejected before any use
        with pytest.raises(ValueError):
            kernels.gemv_norm(synth.Q4_K, w, 144, x, x, 1e-6, None, None, y, 4, 256, code)


# ------------------------------------------------------------- small ops
@pytest.mark.parametrize("rows,cols", [(1, 896), (5, 3584), (3, 5120)])
def test_rmsnorm_bit_exact(cuda, rows, cols):
    x = synth.normal(rows * cols, 41, stddev=3.0).reshape(rows, cols)
    g = synth.normal(cols, 42, stddev=0.5) + 1.0
    y = torch.empty(rows * cols, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, cols, cuda, rows)
    kernels.rmsnorm(torch.from_numpy(x).to(cuda), torch.from_numpy(g).to(cuda), y, yq, rows, cols, 1e-6)
    ref = x.copy()
    for r in range(rows):
        oracle.lib().oracle_rmsnorm(ref[r].ctypes.data, g.ctypes.data, cols, ctypes.c_float(1e-6))
    got = y.cpu().numpy().reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    xgroup.check(yq, got)


def _libm():
    m = ctypes.CDLL("libm.so.6")
    for f in ("cosf", "sinf"):
        getattr(m, f).restype = ctypes.c_float
        getattr(m, f).argtypes = [ctypes.c_float]
    m.powf.restype = ctypes.c_float
    m.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return m


@pytest.mark.parametrize("hq,hkv,d,pos0,rows", [(14, 2, 64, 0, 1), (14, 2, 64, 37, 3), (40, 8, 128, 4000, 2)])
def test_rope_kv_bit_exact(cuda, hq, hkv, d, pos0, rows):
    theta = 1e6
    m = _libm()
    half = d // 2
    npos = pos0 + rows
    # Same float32 expressions as CPULLM's Vector::rope (cpu_llm.cpp:218-224).
    freq = [m.powf(theta, float(np.float32(-2.0) * np.float32(p) / np.float32(d))) for p in range(half)]
    table = np.empty((npos, half, 2), dtype=np.float32)
    for pos in range(pos0, npos):
        for p in range(half):
            ang = float(np.float32(pos) * np.float32(freq[p]))
            table[pos, p] = (m.cosf(ang), m.sinf(ang))
    stride = (hq + 2 * hkv) * d
    qkv = synth.normal(rows * stride, 51).reshape(rows, stride)
    dq = torch.from_numpy(qkv.copy()).to(cuda)
    kc = torch.zeros(npos * hkv * d, dtype=torch.float32, device=cuda)
    vc = torch.zeros_like(kc)
    kernels.rope_kv(dq, torch.from_numpy(table).to(cuda), d, hq, hkv, d, pos0, rows, stride, kc, vc)
    ref = qkv.copy()
    for r in range(rows):
        for h in range(hq + hkv):
            seg = np.ascontiguousarray(ref[r, h * d:(h + 1) * d])
            oracle.lib().oracle_rope(seg.ctypes.data, d, pos0 + r, ctypes.c_float(theta), d)
            ref[r, h * d:(h + 1) * d] = seg
    got = dq.cpu().numpy().reshape(rows, stride)
    assert np.array_equal(got[:, : (hq + hkv) * d].view(np.uint32), ref[:, : (hq + hkv) * d].view(np.uint32))
    kv = hkv * d
    kcache = kc.cpu().numpy().reshape(npos, kv)
    vcache = vc.cpu().numpy().reshape(npos, kv)
    assert np.array_equal(kcache[pos0:], got[:, hq * d: hq * d + kv])
    assert np.array_equal(vcache[pos0:], qkv[:, hq * d + kv:])


@pytest.mark.parametrize("length", [1, 7, 255, 256, 257, 1000, 4096, 5000])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (40, 8, 128)])
def test_attention_decode(cuda, length, hq, hkv, d):
    kv = hkv * d
    q = synth.normal(hq * d, 61)
    k = synth.normal(length * kv, 62).reshape(length, kv)
    v = synth.normal(length * kv, 63).reshape(length, kv)
    scale = np.float32(1.0) / np.float32(math.sqrt(d))
    out = torch.empty(hq * d, dtype=torch.float32, device=cuda)
    outq = xgroup.buffer(torch, hq * d, cuda)
    scratch = torch.empty(kernels.attn_decode_scratch_floats(hq, d, length), dtype=torch.float32, device=cuda)
    kernels.attn_decode(torch.from_numpy(q).to(cuda), torch.from_numpy(k).to(cuda), torch.from_numpy(v).to(cuda),
                        out, outq, scratch, hq, hkv, d, length, float(scale))
    ref = np.empty(hq * d)
    for h in range(hq):
        g = h // (hq // hkv)
        s = k[:, g * d:(g + 1) * d].astype(np.float64) @ q[h * d:(h + 1) * d] * float(scale)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h * d:(h + 1) * d] = p @ v[:, g * d:(g + 1) * d]
    got = out.cpu().numpy()
    assert rel_err(got, ref) <= 1e-5
    xgroup.check(outq, got)


@pytest.mark.parametrize("hq,hkv,d,rot,pos", [(14, 2, 64, 64, 0), (14, 2, 64, 64, 130), (40, 8, 128, 128, 257),
                                               (16, 2, 256, 64, 70)])
def test_attention_decode_rope_matches_two_steps(cuda, hq, hkv, d, rot, pos):
    # The fused decode step (RoPE + cache write inside the attention blocks)
    # against hipllm_rope_kv followed by hipllm_attn_decode: same bits for
    # the output, its XGroup form and the cache row; the raw row untouched.
    rng = np.random.default_rng(pos + d)
    kv = hkv * d
    cap = pos + 3
    stride = (hq + 2 * hkv) * d
    qkv = rng.normal(size=stride).astype(np.float32)
    ang = rng.uniform(-3.0, 3.0, size=(cap, rot // 2)).astype(np.float32)
    table = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
    kc0 = rng.normal(size=(cap, kv)).astype(np.float32)
    vc0 = rng.normal(size=(cap, kv)).astype(np.float32)
    dtab = torch.from_numpy(table).to(cuda)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(d)))
    outs = []
    for fused in (False, True):
        dq = torch.from_numpy(qkv.copy()).to(cuda)
        kc = torch.from_numpy(kc0.copy()).to(cuda)
        vc = torch.from_numpy(vc0.copy()).to(cuda)
        out = torch.empty(hq * d, dtype=torch.float32, device=cuda)
        outq = xgroup.buffer(torch, hq * d, cuda)
        scratch = torch.empty(kernels.attn_decode_scratch_floats(hq, d, pos + 1), dtype=torch.float32, device=cuda)
        if fused:
            kernels.attn_decode_rope(dq, dtab, rot, kc, vc, out, outq, scratch, hq, hkv, d, pos, scale)
            assert np.array_equal(dq.cpu().numpy(), qkv)
        else:
            kernels.rope_kv(dq, dtab, rot, hq, hkv, d, pos, 1, stride, kc, vc)
            kernels.attn_decode(dq, kc, vc, out, outq, scratch, hq, hkv, d, pos + 1, scale)
        outs.append((out.cpu().numpy(), outq.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()))
    (o1, q1, k1, v1), (o2, q2, k2, v2) = outs
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(q1.view(np.uint32), q2.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    assert not np.array_equal(k2[pos], kc0[pos])


@pytest.mark.parametrize("hq,hkv,d,rot,pos", [(16, 2, 256, 64, 70), (16, 2, 256, 64, 0), (14, 2, 64, 64, 130)])
def test_attention_decode_rope_gated_matches_gate_kernel(cuda, hq, hkv, d, rot, pos):
    # The output gate in the merge against the fused step followed by the
    # gate kernel (gate_mul): same bits for the gated output and its XGroup
    # form.
    rng = np.random.default_rng(pos + 3 * d)
    kv = hkv * d
    cap = pos + 3
    stride = (hq + 2 * hkv) * d
    qkv = rng.normal(size=stride).astype(np.float32)
    gate = (rng.normal(size=hq * d) * 3.0).astype(np.float32)
    ang = rng.uniform(-3.0, 3.0, size=(cap, rot // 2)).astype(np.float32)
    table = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
    kc0 = rng.normal(size=(cap, kv)).astype(np.float32)
    vc0 = rng.normal(size=(cap, kv)).astype(np.float32)
    dtab = torch.from_numpy(table).to(cuda)
    dgate = torch.from_numpy(gate).to(cuda)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(d)))
    outs = []
    for fused in (False, True):
        dq = torch.from_numpy(qkv.copy()).to(cuda)
        kc = torch.from_numpy(kc0.copy()).to(cuda)
        vc = torch.from_numpy(vc0.copy()).to(cuda)
        out = torch.empty(hq * d, dtype=torch.float32, device=cuda)
        outq = xgroup.buffer(torch, hq * d, cuda)
        scratch = torch.empty(kernels.attn_decode_scratch_floats(hq, d, pos + 1), dtype=torch.float32, device=cuda)
        if fused:
            kernels.attn_decode_rope_gated(dq, dtab, rot, kc, vc, dgate, out, outq, scratch, hq, hkv, d, pos, scale)
        else:
            att = torch.empty(hq * d, dtype=torch.float32, device=cuda)
            kernels.attn_decode_rope(dq, dtab, rot, kc, vc, att, None, scratch, hq, hkv, d, pos, scale)
            kernels.gate_mul(att, dgate, out, outq, hq * d)
        outs.append((out.cpu().numpy(), outq.cpu().numpy()))
    (o1, q1), (o2, q2) = outs
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(q1.view(np.uint32), q2.view(np.uint32))


@pytest.mark.parametrize("hq,hkv,d,length", [(14, 2, 64, 1), (14, 2, 64, 37), (14, 2, 64, 130),
                                              (40, 8, 128, 257), (16, 2, 256, 70)])
def test_attention_ignores_cache_rows_past_length(cuda, hq, hkv, d, length):
    # Cache rows at or past the length are not part of the result, whatever
    # bits they hold: with NaN / Inf there the decode (plain and fused RoPE +
    # cache write) and prefill attention outputs equal, bit for bit, those
    # with zeros there. A read of such a row weighted by p = 0 would turn
    # NaN into NaN and fail this.
    rng = np.random.default_rng(length + d)
    kv = hkv * d
    cap = length + 70  # the last chunk has unused rows, and a whole chunk follows
    stride = (hq + 2 * hkv) * d
    k0 = rng.normal(size=(cap, kv)).astype(np.float32)
    v0 = rng.normal(size=(cap, kv)).astype(np.float32)
    qkv = rng.normal(size=stride).astype(np.float32)
    rows_p = min(length, 5)
    qp = rng.normal(size=(rows_p, hq * d)).astype(np.float32)
    ang = rng.uniform(-3.0, 3.0, size=(cap, d // 2)).astype(np.float32)
    dtab = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)).to(cuda)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(d)))

    def run(fill):
        kc0, vc0 = k0.copy(), v0.copy()
        kc0[length:] = fill
        vc0[length:] = fill
        res = []
        for mode in ("decode", "fused", "prefill"):
            kc = torch.from_numpy(kc0.copy()).to(cuda)
            vc = torch.from_numpy(vc0.copy()).to(cuda)
            scratch = torch.empty(kernels.attn_decode_scratch_floats(hq, d, cap), dtype=torch.float32, device=cuda)
            if mode == "decode":
                out = torch.empty(hq * d, dtype=torch.float32, device=cuda)
                kernels.attn_decode(torch.from_numpy(qkv).to(cuda), kc, vc, out, None, scratch, hq, hkv, d, length,
                                    scale)
            elif mode == "fused":
                out = torch.empty(hq * d, dtype=torch.float32, device=cuda)
                # The step writes row length - 1 itself; rows past it stay poisoned.
                kernels.attn_decode_rope(torch.from_numpy(qkv).to(cuda), dtab, d, kc, vc, out, None, scratch, hq, hkv,
                                         d, length - 1, scale)
            else:
                out = torch.empty(rows_p * hq * d, dtype=torch.float32, device=cuda)
                pos0 = length - rows_p
                kernels.attn_prefill(torch.from_numpy(qp).to(cuda), hq * d, kc, vc, out, hq * d, rows_p, hq, hkv, d,
                                     pos0, scale)
            res.append(out.cpu().numpy())
        return res

    clean = run(0.0)
    for fill in (np.nan, np.inf, -np.inf):
        for a, b in zip(run(fill), clean):
            assert np.isfinite(b).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), fill


@pytest.mark.parametrize("n", [1, 100, 2048, 2049, 151936])
def test_argmax(cuda, n):
    x = synth.normal(n, 71 + n)
    for case in range(3):
        if case == 1 and n > 1:  # tie: the lower index wins
            i, j = n // 3, n - 1
            x[i] = x[j] = x.max() + 1
        if case == 2:
            x[:] = -np.inf
            x[n // 2] = 0.0
        scratch = torch.empty(kernels.argmax_scratch_bytes(n), dtype=torch.uint8, device=cuda)
        out = torch.empty(1, dtype=torch.int32, device=cuda)
        kernels.argmax(torch.from_numpy(x).to(cuda), n, out, scratch)
        assert int(out.item()) == oracle.lib().oracle_argmax(x.ctypes.data, n)


def test_embed_bit_exact(cuda):
    vocab, cols = 300, 896
    table = random_rows(synth.Q8_0, vocab, cols, 81)
    ids = np.array([0, 299, 17, 17, -1, 300], dtype=np.int32)
    out = torch.empty(len(ids) * cols, dtype=torch.float32, device=cuda)
    kernels.embed(synth.Q8_0, dev_bytes(table, cuda), table.shape[1], torch.from_numpy(ids).to(cuda), len(ids),
                  vocab, cols, out)
    got = out.cpu().numpy().reshape(len(ids), cols)
    ref = oracle.dequant_rows(synth.Q8_0, table, cols)
    for r, t in enumerate(ids):
        expect = ref[t] if 0 <= t < vocab else np.zeros(cols, dtype=np.float32)
        assert np.array_equal(got[r].view(np.uint32), expect.view(np.uint32))


def test_swiglu_elementwise(cuda):
    n = 4864
    g, u = synth.normal(n, 91, stddev=4.0), synth.normal(n, 92)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, n, cuda)
    kernels.swiglu(torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda), y, yq, n)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert rel_err(y.cpu().numpy(), ref) <= 1e-6
    xgroup.check(yq, y.cpu().numpy())


def test_launchers_reject_bad_arguments(cuda):
    from myllm_amd.hipllm import lib
    y = torch.empty(16, dtype=torch.float32, device=cuda)
    w = torch.zeros(1024, dtype=torch.uint8, device=cuda)
    with pytest.raises(ValueError):
        kernels.gemv_prepped(synth.Q4_K, w, 144, y, y, None, None, y, 4, 100)  # k not block aligned
    with pytest.raises(ValueError):
        kernels.gemv_prepped(99, w, 144, y, y, None, None, y, 4, 256)  # unknown type
    with pytest.raises(ValueError):
        kernels.rmsnorm(y, y, y, None, 1, 16, 0.0)  # eps must be positive
    assert lib().hipllm_version()

