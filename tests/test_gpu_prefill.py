"""Prefill matmul parity on the GPU (fp16 MFMA over native GGUF weights).

Two references per case, both float64 over the bit-exact FP32 dequantized
weights:
* the contract: against the FP32 operands, max|Y - ref| / max|ref| <= 2e-2
  (the fp16 operands land near 1e-3);
* the kernel's own arithmetic: against the same product with X given as its
  scaled fp16 rows (checked bit for bit against numpy's round-to-nearest-even
  conversion of the row scaled by the power of two its largest magnitude
  fixes) and W rounded to fp16, within 1e-4 -- what is left is FP32
  accumulation order, so a wrong operand layout, k map, scale index or tile
  edge fails here even when it would hide inside the 2e-2 bound.
"""

from __future__ import annotations

import pytest

import numpy as np

from myllm_amd import synth
from myllm_amd.hipllm import kernels, lib
from tests.test_gpu_kernels import dev_bytes, random_rows, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_K, synth.Q6_K, synth.Q8_0, synth.Q5_0, synth.F16, synth.F32]


def f16_rows_ref(x: np.ndarray):
    """The scaled fp16 operand rows: per row 2^e with max|x| / 2^e in
    [2^13, 2^14) (NaN left out of the maximum; e = 0 for a zero row or one
    holding an Inf; e clamped to [-126, 127]), xh = fp16(x / 2^e)."""
    x = np.asarray(x, dtype=np.float32)
    xh = np.empty(x.shape, dtype=np.float16)
    scale = np.ones(x.shape[0], dtype=np.float32)
    for r in range(x.shape[0]):
        a = np.abs(x[r])
        mx = np.nanmax(a) if not np.isnan(a).all() else 0.0
        e = 0
        if 0 < mx < np.inf:
            e = min(127, max(-126, int(np.frexp(mx)[1]) - 14))
        xh[r] = (x[r] * np.float32(2.0 ** -e)).astype(np.float16)
        scale[r] = np.float32(2.0 ** e)
    return xh, scale


def to_f16(x, cuda):
    """hipllm_to_f16 of the device rows x, checked against f16_rows_ref."""
    m, k = x.shape
    xh = torch.empty(m, k, dtype=torch.float16, device=cuda)
    xs = torch.empty(m, dtype=torch.float32, device=cuda)
    kernels.to_f16(x, k, xh, xs, m, k)
    rh, rs = f16_rows_ref(x.cpu().numpy())
    assert np.array_equal(xh.cpu().numpy().view(np.uint16), rh.view(np.uint16)), "fp16 rows"
    assert np.array_equal(xs.cpu().numpy(), rs), "row scales"
    return xh, xs


def gemm_case(cuda, qtype, m, n, k, seed, tile=-1, bias=False, residual=False, splits=0, in_place=False):
    w = random_rows(qtype, n, k, seed)
    dw = dev_bytes(w, cuda)
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    # Rows of different magnitudes (the scale follows each row).
    x = (x * torch.exp2(torch.randint(-12, 13, (m, 1), generator=g).float())).to(cuda)
    xh, xs = to_f16(x, cuda)
    b = torch.randn(n, generator=g).to(cuda) if bias else None
    r = torch.randn(m, n, generator=g).to(cuda) if residual else None
    y = r.clone() if in_place else torch.empty(m, n, dtype=torch.float32, device=cuda)
    kernels.gemm_mfma(qtype, dw, w.shape[1], xh, xs, b, y if in_place else r, y, m, n, k, tile, splits=splits)
    wf = torch.empty(n, k, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(qtype, dw, w.shape[1], n, k, wf)
    ref = x.double() @ wf.double().T
    ref_b = (xh.double() * xs.double()[:, None]) @ wf.to(torch.float16).double().T
    for extra in (b, r):
        if extra is not None:
            ref = ref + extra.double()
            ref_b = ref_b + extra.double()
    # Relative to each row's own magnitude (rows differ by up to 2^24).
    ref, ref_b, y = (t.double().cpu().numpy() for t in (ref, ref_b, y))
    norm = np.abs(ref).max(axis=1, keepdims=True)
    return y / norm, ref / norm, ref_b / norm


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6])
def test_gemm_types_and_tiles_ragged(cuda, qtype, tile):
    # m = 77, n = 333: partial tiles on both axes; k = 512: four 128-steps
    # (both halves of a K-quant super-block).
    y, ref, ref_b = gemm_case(cuda, qtype, 77, 333, 512, seed=qtype * 10 + tile, tile=tile, bias=True,
                              residual=True)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 10])
@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K, synth.Q8_0])
def test_gemm_k_splits(cuda, qtype, splits):
    # k = 1280: ten 128-steps, split 1, 2, 3 (4 + 4 + 2), 7 (2 x 5, so 5
    # splits) and 10 ways; partial tiles, bias and residual on every split.
    for tile in (1, 4):
        y, ref, ref_b = gemm_case(cuda, qtype, 45, 300, 1280, seed=splits, tile=tile, bias=True, residual=True,
                                  splits=splits)
        assert rel_err(y, ref) <= 2e-2
        assert rel_err(y, ref_b) <= 1e-4
    y, ref, ref_b = gemm_case(cuda, qtype, 300, 200, 1280, seed=splits, tile=5, bias=True, residual=True,
                              splits=splits)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


@pytest.mark.parametrize("tile", [1, 4])
def test_gemm_k_split_is_deterministic(cuda, tile):
    """The K split's partial sums are added in split order by one reduce
    launch, not by atomics: repeated runs give the same bits."""
    first = gemm_case(cuda, synth.Q4_K, 45, 300, 1280, seed=5, tile=tile, bias=True, residual=True, splits=7)[0]
    for _ in range(4):
        again = gemm_case(cuda, synth.Q4_K, 45, 300, 1280, seed=5, tile=tile, bias=True, residual=True, splits=7)[0]
        assert np.array_equal(first, again)


def test_gemm_split_workspace_rules(cuda):
    """An explicit split without room for its partial planes is rejected;
    the default split without workspace runs unsplit (same bits as splits=1)."""
    qtype, m, n, k = synth.Q4_K, 40, 256, 1536
    w = random_rows(qtype, n, k, 9)
    dw = dev_bytes(w, cuda)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(9)).to(cuda)
    xh, xs = to_f16(x, cuda)
    need = lib().hipllm_gemm_mfma_workspace_bytes(m, n, k, -1, 0)
    assert need == lib().hipllm_gemm_mfma_workspace_bytes(m, n, k, -1, 0) > 0  # this shape splits by default
    assert lib().hipllm_gemm_mfma_workspace_bytes(m, n, k, -1, 1) == 0
    y1 = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma(qtype, dw, w.shape[1], xh, xs, None, None, y1, m, n, k, splits=1)
    y0 = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma(qtype, dw, w.shape[1], xh, xs, None, None, y0, m, n, k,
                      workspace=torch.empty(0, dtype=torch.uint8, device=cuda))
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
    need4 = lib().hipllm_gemm_mfma_workspace_bytes(m, n, k, -1, 4)
    assert need4 == 4 * m * n * 4
    short = torch.empty(need4 - 16, dtype=torch.uint8, device=cuda)
    with pytest.raises(ValueError):
        kernels.gemm_mfma(qtype, dw, w.shape[1], xh, xs, None, None, y0, m, n, k, splits=4, workspace=short)
    yd = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma(qtype, dw, w.shape[1], xh, xs, None, None, yd, m, n, k)  # default split, full workspace
    assert rel_err(yd.cpu().numpy(), y1.cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("splits", [1, 4])
def test_gemm_in_place_residual(cuda, splits):
    # y aliases residual (the decoder's hidden-state update), with and without a K split.
    y, ref, ref_b = gemm_case(cuda, synth.Q4_K, 33, 256, 1024, seed=8, tile=0, bias=True, residual=True,
                              splits=splits, in_place=True)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


@pytest.mark.parametrize("qtype", TYPES)
def test_gemm_small_m(cuda, qtype):
    y, ref, ref_b = gemm_case(cuda, qtype, 1, 260, 1024, seed=3)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


@pytest.mark.parametrize("m", [64, 512, 2048])
def test_gemm_qwen7b_prefill_shape_q4k(cuda, m):
    # M x K=3584 x N=18944 with Q4_K weights (the prefill matmul microbench).
    y, ref, ref_b = gemm_case(cuda, synth.Q4_K, m, 18944, 3584, seed=m)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


def test_gemm_qwen7b_down_shape_q6k(cuda):
    y, ref, ref_b = gemm_case(cuda, synth.Q6_K, 512, 3584, 18944, seed=5)
    assert rel_err(y, ref) <= 2e-2
    assert rel_err(y, ref_b) <= 1e-4


def test_gemm_fp32_entry_with_workspace(cuda):
    m, n, k = 40, 300, 896
    w = random_rows(synth.Q5_0, n, k, 9)
    dw = dev_bytes(w, cuda)
    x = torch.randn(m, k + 8, device=cuda)  # ldx > k
    ws = torch.empty(kernels.gemm_workspace_bytes(m, k), dtype=torch.uint8, device=cuda)
    y = torch.empty(m, n, device=cuda)
    kernels.gemm(synth.Q5_0, dw, w.shape[1], x, k + 8, None, y, m, n, k, ws)
    wf = torch.empty(n, k, dtype=torch.float32, device=cuda)
    kernels.dequant_rows(synth.Q5_0, dw, w.shape[1], n, k, wf)
    ref = x[:, :k].double() @ wf.double().T
    assert rel_err(y.double().cpu().numpy(), ref.cpu().numpy()) <= 2e-2


def test_to_f16_special_rows(cuda):
    # Zero rows, a row at the FP32 maximum, tiny rows (subnormal fp16 after
    # scaling only far below the row's largest value), and Inf / NaN rows
    # (scale 1: the non-finite values pass through).
    k = 64
    x = np.zeros((7, k), dtype=np.float32)
    x[6] = np.linspace(-2e-37, 2e-37, k, dtype=np.float32)  # e clamped at -126
    x[1] = np.linspace(-3.4e38, 3.4e38, k, dtype=np.float32)
    x[2] = np.linspace(-1e-30, 1e-30, k, dtype=np.float32)
    x[2, 0] = 1e-38
    x[3] = 1.0
    x[3, 5] = np.inf
    x[4] = 2.0
    x[4, 9] = np.nan
    x[5] = np.linspace(-70000.0, 65504.0 * 4, k, dtype=np.float32)
    xh, xs = to_f16(torch.from_numpy(x).to(cuda), cuda)
    assert xs[0].item() == 1.0 and xs[3].item() == 1.0 and xs[4].item() != 1.0
    assert torch.isnan(xh[4, 9]) and torch.isinf(xh[3, 5]) and xs[6].item() == 2.0 ** -126
    assert torch.isfinite(xh[1]).all() and torch.isfinite(xh[5]).all()


def test_gemm_rejects_bad_arguments(cuda):
    w = torch.zeros(144 * 4 + 256, dtype=torch.uint8, device=cuda)
    xh = torch.zeros(2, 256, dtype=torch.float16, device=cuda)
    xs = torch.ones(2, device=cuda)
    y = torch.zeros(2, 2, device=cuda)
    with pytest.raises(ValueError):
        kernels.gemm_mfma(synth.Q4_K, w, 144, xh, xs, None, None, y, 2, 2, 192)  # k % 128 != 0
    with pytest.raises(ValueError):
        kernels.gemm_mfma(synth.Q4_K, w, 144, xh, xs, None, None, y, 2, 2, 256, 8)  # unknown tile
    with pytest.raises(ValueError):
        kernels.gemm_mfma(99, w, 144, xh, xs, None, None, y, 2, 2, 256)  # unknown type
    with pytest.raises(ValueError):
        kernels.gemm_mfma(synth.Q4_K, w, 144, xh, xs, None, None, y, 2, 2, 256, 0, splits=-1)
    with pytest.raises(ValueError):
        kernels.gemm_mfma(synth.Q4_K, w, 144, xh, xs, None, None, y, 2, 2, 256, 0, splits=1025)
    with pytest.raises(ValueError):
        kernels.gemm_mfma(synth.Q4_K, w, 144, xh, None, None, None, y, 2, 2, 256)  # no row scales


@pytest.mark.parametrize("qtype,m,n,k", [(synth.Q4_K, 128, 4864, 1024), (synth.Q6_K, 45, 1280, 512),
                                         (synth.Q8_0, 300, 512, 1024), (synth.Q4_K, 1100, 256, 512),
                                         (synth.Q4_K, 512, 6144, 512), (synth.Q5_0, 64, 512, 256)])
def test_gemm_swiglu_matches_two_matmuls_and_swiglu(cuda, qtype, m, n, k):
    """Gate / up matmuls with their SwiGLU in one reduce launch against two
    hipllm_gemm_mfma calls (default tile and K split) and hipllm_swiglu: the
    same bits, split (few tiles) and unsplit (many rows)."""
    wg, wu = random_rows(qtype, n, k, 91), random_rows(qtype, n, k, 92)
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    g = torch.Generator(device="cpu").manual_seed(93)
    x = torch.randn(m, k, generator=g).to(cuda)
    xh, xs = to_f16(x, cuda)
    y = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma_swiglu(qtype, dg, du, wg.shape[1], xh, xs, y, m, n, k)
    ga = torch.empty(m, n, device=cuda)
    ua = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma(qtype, dg, wg.shape[1], xh, xs, None, None, ga, m, n, k)
    kernels.gemm_mfma(qtype, du, wu.shape[1], xh, xs, None, None, ua, m, n, k)
    ref = torch.empty(m, n, device=cuda)
    kernels.swiglu(ga, ua, ref, None, m * n)
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))


@pytest.mark.parametrize("qtype,m,n,k", [(synth.Q4_K, 128, 18944, 512), (synth.Q6_K, 45, 1280, 512),
                                         (synth.Q8_0, 64, 512, 1024), (synth.Q4_K, 300, 32768, 256),
                                         (synth.Q4_K, 1100, 256, 512)])
def test_gemm_swiglu_f16_matches_swiglu_then_f16(cuda, qtype, m, n, k):
    """The SwiGLU rows written as fp16 operand rows in the reduce launch
    against the FP32 form followed by hipllm_to_f16: the same fp16 bits and
    row scales (n up to the 32768 limit, split and unsplit)."""
    wg, wu = random_rows(qtype, n, k, 94), random_rows(qtype, n, k, 95)
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    g = torch.Generator(device="cpu").manual_seed(96)
    x = torch.randn(m, k, generator=g).to(cuda)
    xh, xs = to_f16(x, cuda)
    yh = torch.empty(m, n, dtype=torch.float16, device=cuda)
    ys = torch.empty(m, device=cuda)
    kernels.gemm_mfma_swiglu_f16(qtype, dg, du, wg.shape[1], xh, xs, yh, ys, m, n, k)
    y = torch.empty(m, n, device=cuda)
    kernels.gemm_mfma_swiglu(qtype, dg, du, wg.shape[1], xh, xs, y, m, n, k)
    rh, rs = to_f16(y, cuda)
    assert torch.equal(yh.view(torch.int16), rh.view(torch.int16))
    assert torch.equal(ys.view(torch.int32), rs.view(torch.int32))


def test_gemm_swiglu_f16_rejects_bad_shapes(cuda):
    w = torch.zeros(144 * 64, dtype=torch.uint8, device=cuda)
    xh = torch.zeros(2, 256, dtype=torch.float16, device=cuda)
    xs = torch.ones(2, device=cuda)
    yh = torch.zeros(2, 32776, dtype=torch.float16, device=cuda)
    ys = torch.zeros(2, device=cuda)
    with pytest.raises(ValueError):  # n % 8
        kernels.gemm_mfma_swiglu_f16(synth.Q4_K, w, w, 144, xh, xs, yh, ys, 2, 20, 256)
    with pytest.raises(ValueError):  # n beyond 32768
        kernels.gemm_mfma_swiglu_f16(synth.Q4_K, w, w, 144, xh, xs, yh, ys, 2, 32776, 256)


def test_gemm_swiglu_rejects_bad_arguments(cuda):
    w = torch.zeros(144 * 64, dtype=torch.uint8, device=cuda)
    xh = torch.zeros(2, 256, dtype=torch.float16, device=cuda)
    xs = torch.ones(2, device=cuda)
    y = torch.zeros(2, 16, device=cuda)
    small = torch.zeros(16, dtype=torch.uint8, device=cuda)
    with pytest.raises(ValueError):
        kernels.gemm_mfma_swiglu(synth.F32, w, w, 144, xh, xs, y, 2, 16, 256)  # quantized weights only
    with pytest.raises(ValueError):
        kernels.gemm_mfma_swiglu(synth.Q4_K, w, w, 144, xh, xs, y, 2, 16, 192)  # k % 128
    with pytest.raises(ValueError):
        kernels.gemm_mfma_swiglu(synth.Q4_K, w, w, 144, xh, xs, y, 2, 16, 256, workspace=small)  # workspace too small


@pytest.mark.parametrize("rows,cols", [(1, 896), (7, 3584), (130, 5120), (3, 8192)])
def test_rmsnorm_f16_matches_norm_then_f16(cuda, rows, cols):
    """RMSNorm and the fp16 operand form in one launch against hipllm_rmsnorm
    followed by hipllm_to_f16: normalised rows, fp16 values and row scales
    bit for bit (rows of very different magnitudes, one all zero)."""
    g = torch.Generator(device="cpu").manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g) * torch.exp2(torch.randint(-20, 21, (rows, 1), generator=g).float())
    if rows > 2:
        x[1] = 0.0
    x = x.to(cuda)
    gamma = torch.randn(cols, generator=g).to(cuda)
    norm = torch.empty(rows, cols, device=cuda)
    xh = torch.empty(rows, cols, dtype=torch.float16, device=cuda)
    xs = torch.empty(rows, device=cuda)
    kernels.rmsnorm_f16(x, gamma, norm, xh, xs, rows, cols, 1e-6)
    norm_r = torch.empty(rows, cols, device=cuda)
    xh_r = torch.empty(rows, cols, dtype=torch.float16, device=cuda)
    xs_r = torch.empty(rows, device=cuda)
    kernels.rmsnorm(x, gamma, norm_r, None, rows, cols, 1e-6)
    kernels.to_f16(norm_r, cols, xh_r, xs_r, rows, cols)
    assert torch.equal(norm.view(torch.int32), norm_r.view(torch.int32))
    assert torch.equal(xh.view(torch.int16), xh_r.view(torch.int16))
    assert torch.equal(xs.view(torch.int32), xs_r.view(torch.int32))
