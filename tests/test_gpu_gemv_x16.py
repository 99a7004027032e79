"""The x16 tile-packed Q4_K / Q6_K forms and the int8-MFMA decode GEMV over
them.

* Packing: the device packer's bytes against a numpy restatement of each
  layout (tile T, unit u at (T * units + u) * 16 B; Q4_K: the 16 rows'
  headers, then for lane l = 16 s + r the quant bytes [16 s, +16) of row r,
  then its bytes [64 + 16 s, +16); Q6_K: for lane l the ql bytes
  [64 (s >> 1) + 16 (s & 1), +16), then ql [64 (s >> 1) + 32 + 16 (s & 1),
  +16), then qh [32 (s >> 1) + 16 (s & 1), +16), then the 16 rows' scale
  bytes and their d); rows past n are zero.
* Product: against float64 over the oracle's bit-exact CPU dequantization of
  the same GGUF rows (oracle.dequant_rows restates model.cpp:616-683), for
  ragged row counts, every launch shape, bias and residual, short and long
  rows; and against the vector GEMV on the GGUF rows, which computes the
  same exact integer digit sums (only the FP32 summation order differs).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from myllm_amd import synth
from myllm_amd.hipllm import kernels
from tests import xgroup
from tests.test_gpu_kernels import dev_bytes, random_rows, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SHAPES = [1104, 1108, 1116, 2104, 2108, 2116]
TYPES = [synth.Q4_K, synth.Q6_K]
PLAIN_TYPES = TYPES + [synth.Q8_0]  # Q8_0 copies serve plain products only
BLOCK = {synth.Q4_K: 144, synth.Q6_K: 210, synth.Q8_0: 272}


def pack_ref(qtype: int, w: np.ndarray, n: int, k: int) -> np.ndarray:
    """numpy restatement of the x16 layout from GGUF rows [n, row_bytes]."""
    B = BLOCK[qtype]
    units = k // 256
    tiles = (n + 15) // 16
    rows = np.zeros((tiles * 16, units, B), dtype=np.uint8)
    rows[:n] = w[:, : units * B].reshape(n, units, B)
    out = np.empty((tiles, units, 16 * B), dtype=np.uint8)
    for t in range(tiles):
        blk = rows[16 * t: 16 * t + 16]  # [16, units, B]

        def lanes(offset_of_s):
            # lane l = 16 s + r: 16 bytes at offset_of_s(s) of row r -> [units, 1024]
            sl = np.stack([blk[:, :, offset_of_s(s): offset_of_s(s) + 16] for s in range(4)])  # [4, 16, units, 16]
            return sl.transpose(2, 0, 1, 3).reshape(units, 1024)

        if qtype == synth.Q8_0:
            # MFMA i, lane 16 s + r: block 2 i + (s >> 1), quants 16 (s & 1) on; then
            # per row its d values, half 4 p + i = block 2 i + p.
            for i in range(4):
                out[t, :, 1024 * i:1024 * (i + 1)] = lanes(lambda s, i=i: 34 * (2 * i + (s >> 1)) + 2 + 16 * (s & 1))
            d = np.stack([blk[:, :, 34 * (2 * (h & 3) + (h >> 2)):34 * (2 * (h & 3) + (h >> 2)) + 2] for h in range(8)],
                         axis=2)  # [16, units, 8, 2]
            out[t, :, 4096:4352] = d.reshape(16, units, 16).transpose(1, 0, 2).reshape(units, 256)
        elif qtype == synth.Q4_K:
            out[t, :, :256] = blk[:, :, :16].transpose(1, 0, 2).reshape(units, 256)
            out[t, :, 256:1280] = lanes(lambda s: 16 + 16 * s)
            out[t, :, 1280:2304] = lanes(lambda s: 80 + 16 * s)
        else:
            out[t, :, 0:1024] = lanes(lambda s: 64 * (s >> 1) + 16 * (s & 1))
            out[t, :, 1024:2048] = lanes(lambda s: 64 * (s >> 1) + 32 + 16 * (s & 1))
            out[t, :, 2048:3072] = lanes(lambda s: 128 + 32 * (s >> 1) + 16 * (s & 1))
            out[t, :, 3072:3328] = blk[:, :, 192:208].transpose(1, 0, 2).reshape(units, 256)
            out[t, :, 3328:3360] = blk[:, :, 208:210].transpose(1, 0, 2).reshape(units, 32)
    return out.reshape(-1)


def packed_case(cuda, qtype, n, k, seed, bias=False, residual=False, waves=0):
    w = random_rows(qtype, n, k, seed)
    dw = dev_bytes(w, cuda)
    packed = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(qtype, dw, w.shape[1], n, k, packed)
    x = synth.normal(k, seed + 1)
    dx = torch.from_numpy(x).to(cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(dx, xq, k)
    b = synth.normal(n, seed + 2) if bias else None
    r = synth.normal(n, seed + 3) if residual else None
    db = None if b is None else torch.from_numpy(b).to(cuda)
    dr = None if r is None else torch.from_numpy(r).to(cuda)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_x16(qtype, packed, xq, db, dr, y, n, k, waves)
    yv = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_prepped(qtype, dw, w.shape[1], dx, xq, db, dr, yv, n, k, 0)
    wf = oracle.dequant_rows(qtype, w, k).astype(np.float64)
    ref = wf @ x.astype(np.float64)
    for extra in (b, r):
        if extra is not None:
            ref = ref + extra
    return y.cpu().numpy(), yv.cpu().numpy(), ref, w, packed


@pytest.mark.parametrize("qtype", PLAIN_TYPES)
@pytest.mark.parametrize("n,k", [(1, 256), (16, 512), (37, 3584), (333, 2816), (1001, 1024)])
def test_pack_layout(cuda, qtype, n, k):
    w = random_rows(qtype, n, k, n + k)
    packed = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    assert packed.numel() == (n + 15) // 16 * 16 * (k // 256) * BLOCK[qtype]
    kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], n, k, packed)
    assert np.array_equal(packed.cpu().numpy(), pack_ref(qtype, w, n, k))


def test_pack_layout_q6k_odd_row_alignment(cuda):
    """Q6_K rows of an odd unit count start 2-byte aligned (210 = 2 * 105):
    rows taken from a buffer offset by 2 bytes pack the same."""
    n, k = 21, 3 * 256
    w = random_rows(synth.Q6_K, n, k, 5)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device=cuda)
    buf[2: 2 + w.size] = torch.from_numpy(w.reshape(-1)).to(cuda)
    packed = torch.empty(kernels.x16_bytes(synth.Q6_K, n, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(synth.Q6_K, buf[2:], w.shape[1], n, k, packed)
    assert np.array_equal(packed.cpu().numpy(), pack_ref(synth.Q6_K, w, n, k))


@pytest.mark.parametrize("qtype", PLAIN_TYPES)
@pytest.mark.parametrize("n,k", [(1, 256), (16, 256), (37, 512), (333, 2816), (1001, 3584), (130, 18944)])
def test_gemv_x16_matches_oracle_and_vector_path(cuda, qtype, n, k):
    y, yv, ref, _, _ = packed_case(cuda, qtype, n, k, seed=7 * n + k, bias=True, residual=True)
    assert rel_err(y, ref) <= 1e-5
    assert rel_err(y, yv) <= 1e-6


@pytest.mark.parametrize("qtype", PLAIN_TYPES)
@pytest.mark.parametrize("waves", SHAPES)
def test_gemv_x16_launch_shapes(cuda, qtype, waves):
    # 7 units: fewer than some shapes' waves (idle waves), more than others'
    # (several units per wave, ring refills); 45 rows: a partial tile, and
    # for two tiles per block a partial tile pair.
    y, yv, ref, _, _ = packed_case(cuda, qtype, 45, 7 * 256, seed=waves, residual=True, waves=waves)
    assert rel_err(y, ref) <= 1e-5
    assert rel_err(y, yv) <= 1e-6


@pytest.mark.parametrize("qtype", PLAIN_TYPES)
def test_gemv_x16_deterministic_and_long_rows(cuda, qtype):
    # 159 units (ten per wave at 16 waves per block): every shape reduces in a
    # fixed order, so repeated launches give the same bits.
    n, k = 64, 159 * 256
    y, yv, ref, _, _ = packed_case(cuda, qtype, n, k, seed=11, waves=1116)
    assert rel_err(y, ref) <= 1e-5
    y2, _, _, _, _ = packed_case(cuda, qtype, n, k, seed=11, waves=1116)
    assert np.array_equal(y.view(np.int32), y2.view(np.int32))


@pytest.mark.parametrize("qtype", PLAIN_TYPES)
def test_gemv_x16_nan_input_propagates(cuda, qtype):
    # A non-finite activation makes its XGroup's e NaN: the rows that read the
    # group are NaN, as FP32 arithmetic would make them.
    n, k = 32, 512
    w = random_rows(qtype, n, k, 3)
    packed = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], n, k, packed)
    x = torch.from_numpy(synth.normal(k, 4)).to(cuda)
    x[100] = float("nan")
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(x, xq, k)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_x16(qtype, packed, xq, None, None, y, n, k, 0)
    assert torch.isnan(y).all()


def test_gemv_x16_rejects_bad_arguments(cuda):
    n, k = 16, 256
    packed = torch.zeros(kernels.x16_bytes(synth.Q4_K, n, k) + 16, dtype=torch.uint8, device=cuda)
    xq = xgroup.buffer(torch, k, cuda)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    assert kernels.x16_bytes(synth.Q4_K, n, 300) == 0
    assert kernels.x16_bytes(synth.Q5_0, n, 256) == 0
    with pytest.raises(ValueError):
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n, 300, 0)  # k % 256
    with pytest.raises(ValueError):
        kernels.gemv_x16(synth.Q5_0, packed, xq, None, None, y, n, k, 0)  # not a packed type
    with pytest.raises(ValueError):
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n, k, 1103)  # unknown launch shape
    with pytest.raises(ValueError):
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n, k, 1204)  # two units in flight: not offered
    with pytest.raises(ValueError):
        kernels.gemv_x16(synth.Q4_K, packed[8:], xq, None, None, y, n, k, 0)  # misaligned weights
    w = torch.zeros(n * 210 + 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(ValueError):
        kernels.pack_x16(synth.Q4_K, w, 150, n, k, packed)  # Q4_K row_bytes % 16
    with pytest.raises(ValueError):
        kernels.pack_x16(synth.Q4_K, w, 144, n, 200, packed)  # k % 256
    with pytest.raises(ValueError):
        kernels.pack_x16(synth.Q6_K, w[1:], 210, n, k, packed)  # Q6_K rows must be 2-byte aligned
    with pytest.raises(ValueError):
        kernels.pack_x16(synth.Q6_K, w, 209, n, k, packed)  # row shorter than its blocks


def silu_mul_ref(g, u):
    """Sign-branched SiLU(g) * u in float64 (cpu_llm.cpp:188-202)."""
    g = np.asarray(g, dtype=np.float64)
    sig = np.where(g >= 0, 1.0 / (1.0 + np.exp(-np.abs(g))), np.exp(-np.abs(g)) / (1.0 + np.exp(-np.abs(g))))
    return g * sig * np.asarray(u, dtype=np.float64)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k,waves", [(16, 256, 0), (64, 512, 1108), (1040, 3584, 0), (4864, 1024, 0),
                                       (320, 2048, 2104), (48, 18944, 1116), (13824, 1280, 0)])
def test_gemv_x16_swiglu(cuda, qtype, n, k, waves):
    wg = random_rows(qtype, n, k, n + 1)
    wu = random_rows(qtype, n, k, n + 2)
    pg = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    pu = torch.empty_like(pg)
    kernels.pack_x16(qtype, dev_bytes(wg, cuda), wg.shape[1], n, k, pg)
    kernels.pack_x16(qtype, dev_bytes(wu, cuda), wu.shape[1], n, k, pu)
    x = synth.normal(k, n + 3)
    dx = torch.from_numpy(x).to(cuda)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(dx, xq, k)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, n, cuda)
    kernels.gemv_x16_swiglu(qtype, pg, pu, xq, y, yq, n, k, waves)
    g = oracle.dequant_rows(qtype, wg, k).astype(np.float64) @ x.astype(np.float64)
    u = oracle.dequant_rows(qtype, wu, k).astype(np.float64) @ x.astype(np.float64)
    ref = silu_mul_ref(g, u)
    yv = y.cpu().numpy()
    assert rel_err(yv, ref) <= 1e-5
    xgroup.check(yq, yv)
    # The same pair through the vector path on the GGUF rows.
    yv2 = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_swiglu(qtype, dev_bytes(wg, cuda), dev_bytes(wu, cuda), wg.shape[1], dx, xq, yv2, None, n, k, 0)
    assert rel_err(yv, yv2.cpu().numpy()) <= 1e-6
    # Without the XGroup output, and the output rows reject a ragged n.
    kernels.gemv_x16_swiglu(qtype, pg, pu, xq, y, None, n, k, waves)
    assert np.array_equal(y.cpu().numpy().view(np.int32), yv.view(np.int32))
    if n > 16:
        with pytest.raises(ValueError):
            kernels.gemv_x16_swiglu(qtype, pg, pu, xq, y, yq, n - 1, k, waves)


def rms_inv(x: np.ndarray, eps: float) -> np.float32:
    """1 / sqrt(mean(x^2) + eps) as the reference's RMSNorm forms it (double
    sum of squares, FP32 mean, eps and root; cpu_llm.cpp:143-166)."""
    ss = float(np.sum(x.astype(np.float64) ** 2))
    ms = np.float32(ss / x.size)
    return np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)


def tile_sumsq(v: np.ndarray) -> np.ndarray:
    """Per-16-value double sums of squares, each summed in value order."""
    out = np.zeros(v.size // 16)
    for t in range(out.size):
        acc = 0.0
        for x in v[16 * t: 16 * t + 16].astype(np.float64):
            acc += x * x
        out[t] = acc
    return out


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k,waves", [(48, 256, 0), (4608, 3584, 0), (300, 5120, 2108), (1001, 2048, 1104)])
def test_gemv_x16_norm_before_product(cuda, qtype, n, k, waves):
    """W rmsnorm(x) from the XGroup form of x * gamma and the per-16 sums of
    squares of x, against float64 over the oracle's weights and the
    reference's normalised row."""
    w = random_rows(qtype, n, k, n + k)
    packed = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], n, k, packed)
    x = (3.0 * synth.normal(k, n)).astype(np.float32)
    gamma = (1.0 + 0.3 * synth.normal(k, n + 1)).astype(np.float32)
    eps = 1e-6
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(torch.from_numpy(x * gamma).to(cuda), xq, k)
    ssq = torch.from_numpy(tile_sumsq(x)).to(cuda)
    b = synth.normal(n, n + 2)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_x16(qtype, packed, xq, torch.from_numpy(b).to(cuda), None, y, n, k, waves,
                     norm={"sumsq_in": ssq, "eps": eps})
    xn = x * (rms_inv(x, eps) * gamma)  # the reference's normalised row (FP32)
    ref = oracle.dequant_rows(qtype, w, k).astype(np.float64) @ xn.astype(np.float64) + b
    assert rel_err(y.cpu().numpy(), ref) <= 1e-5
    # The SwiGLU pair with the same norm.
    wu = random_rows(qtype, n, k, n + k + 1)
    pu = torch.empty_like(packed)
    kernels.pack_x16(qtype, dev_bytes(wu, cuda), wu.shape[1], n, k, pu)
    if n % 16 == 0:
        ys = torch.empty(n, dtype=torch.float32, device=cuda)
        yq = xgroup.buffer(torch, n, cuda)
        kernels.gemv_x16_swiglu(qtype, packed, pu, xq, ys, yq, n, k, 0, norm={"sumsq_in": ssq, "eps": eps})
        g = oracle.dequant_rows(qtype, w, k).astype(np.float64) @ xn.astype(np.float64)
        u = oracle.dequant_rows(qtype, wu, k).astype(np.float64) @ xn.astype(np.float64)
        assert rel_err(ys.cpu().numpy(), silu_mul_ref(g, u)) <= 1e-5
        xgroup.check(yq, ys.cpu().numpy())


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k,waves", [(3584, 18944, 0), (3584, 3584, 0), (64, 512, 2104), (5120, 13824, 0)])
def test_gemv_x16_norm_after_product(cuda, qtype, n, k, waves):
    """y is the plain GEMV's, bit for bit; the norm data is the XGroup form of
    y * gamma and the per-16 double sums of squares of y in row order; a
    consumer applying it equals the consumer of the standalone RMSNorm."""
    w = random_rows(qtype, n, k, n + 3 * k)
    packed = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], n, k, packed)
    x = synth.normal(k, 5)
    xq = xgroup.buffer(torch, k, cuda)
    kernels.prep_x(torch.from_numpy(x).to(cuda), xq, k)
    res = torch.from_numpy(synth.normal(n, 6)).to(cuda)
    gamma = torch.from_numpy((1.0 + 0.3 * synth.normal(n, 7)).astype(np.float32)).to(cuda)
    y0 = torch.empty(n, dtype=torch.float32, device=cuda)
    kernels.gemv_x16(qtype, packed, xq, None, res, y0, n, k, waves)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, n, cuda)
    ssq = torch.empty(n // 16, dtype=torch.float64, device=cuda)
    kernels.gemv_x16(qtype, packed, xq, None, res, y, n, k, waves,
                     norm={"gamma_out": gamma, "yq_out": yq, "sumsq_out": ssq})
    yv = y.cpu().numpy()
    assert np.array_equal(yv.view(np.int32), y0.cpu().numpy().view(np.int32))
    xgroup.check(yq, yv * gamma.cpu().numpy())
    assert np.array_equal(ssq.cpu().numpy(), tile_sumsq(yv))
    if n <= 8192 and n % 256 == 0:
        # Consumer: n rows of the next matrix read the norm data ...
        m = 256
        w2 = random_rows(synth.Q4_K, m, n, 9)
        p2 = torch.empty(kernels.x16_bytes(synth.Q4_K, m, n), dtype=torch.uint8, device=cuda)
        kernels.pack_x16(synth.Q4_K, dev_bytes(w2, cuda), w2.shape[1], m, n, p2)
        z = torch.empty(m, dtype=torch.float32, device=cuda)
        kernels.gemv_x16(synth.Q4_K, p2, yq, None, None, z, m, n, 0, norm={"sumsq_in": ssq, "eps": 1e-6})
        # ... against the standalone RMSNorm's XGroup output.
        nq = xgroup.buffer(torch, n, cuda)
        nf = torch.empty(n, dtype=torch.float32, device=cuda)
        kernels.rmsnorm(y, gamma, nf, nq, 1, n, 1e-6)
        z0 = torch.empty(m, dtype=torch.float32, device=cuda)
        kernels.gemv_x16(synth.Q4_K, p2, nq, None, None, z0, m, n, 0)
        assert rel_err(z.cpu().numpy(), z0.cpu().numpy()) <= 2e-6


def test_gemv_x16_norm_rejects_bad_combinations(cuda):
    n, k = 32, 256
    packed = torch.zeros(kernels.x16_bytes(synth.Q4_K, n, k), dtype=torch.uint8, device=cuda)
    xq = xgroup.buffer(torch, k, cuda)
    y = torch.empty(n, dtype=torch.float32, device=cuda)
    ssq = torch.zeros(64, dtype=torch.float64, device=cuda)
    gamma = torch.ones(n, dtype=torch.float32, device=cuda)
    yq = xgroup.buffer(torch, n, cuda)
    with pytest.raises(ValueError):  # both forms at once
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n, k, 0,
                         norm={"sumsq_in": ssq, "gamma_out": gamma, "yq_out": yq, "sumsq_out": ssq})
    with pytest.raises(ValueError):  # output form without its buffers
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n, k, 0, norm={"gamma_out": gamma})
    with pytest.raises(ValueError):  # output form with a ragged tile
        kernels.gemv_x16(synth.Q4_K, packed, xq, None, None, y, n - 1, k, 0,
                         norm={"gamma_out": gamma, "yq_out": yq, "sumsq_out": ssq})
    with pytest.raises(ValueError):  # the SwiGLU pair takes no output form
        kernels.gemv_x16_swiglu(synth.Q4_K, packed, packed, xq, y, None, n, k, 0,
                                norm={"gamma_out": gamma, "yq_out": yq, "sumsq_out": ssq})
    big = 9216
    pb = torch.zeros(kernels.x16_bytes(synth.Q4_K, 16, big), dtype=torch.uint8, device=cuda)
    xb = xgroup.buffer(torch, big, cuda)
    with pytest.raises(ValueError):  # input form beyond 8192 values
        kernels.gemv_x16(synth.Q4_K, pb, xb, None, None, y, 16, big, 0, norm={"sumsq_in": ssq})


@pytest.mark.parametrize("src", ["raw row", "norm data"])
@pytest.mark.parametrize("ta,tb,na,nb,k,ksize", [(synth.Q6_K, synth.Q4_K, 96, 64, 2048, 4),
                                                (synth.Q4_K, synth.Q6_K, 40, 37, 512, 3),
                                                (synth.Q4_K, synth.Q8_0, 64, 48, 768, 0)])
def test_pair_norm_conv_matches_float64(cuda, ta, tb, na, nb, k, ksize, src):
    """Two GEMVs of one row in one launch, each block normalising the raw row
    itself (or taking the norm from a producer's data: the XGroup form of
    x * gamma and per-16 double sums of squares), job A with the causal
    conv + SiLU epilogue (history shifted by one row), against float64 over
    the oracle's dequantization; two calls in a row, so the second reads the
    history the first wrote."""
    wa, wb = random_rows(ta, na, k, 61), random_rows(tb, nb, k, 62)
    pa = torch.empty(kernels.x16_bytes(ta, na, k), dtype=torch.uint8, device=cuda)
    pb = torch.empty(kernels.x16_bytes(tb, nb, k), dtype=torch.uint8, device=cuda)
    kernels.pack_x16(ta, dev_bytes(wa, cuda), wa.shape[1], na, k, pa)
    kernels.pack_x16(tb, dev_bytes(wb, cuda), wb.shape[1], nb, k, pb)
    fa = oracle.dequant_rows(ta, wa, k).astype(np.float64)
    fb = oracle.dequant_rows(tb, wb, k).astype(np.float64)
    rng = np.random.default_rng(63)
    gamma = rng.normal(size=k).astype(np.float32)
    conv = rng.normal(scale=0.5, size=(na, max(ksize, 1))).astype(np.float32)
    hist = rng.normal(size=(max(ksize - 1, 1), na)).astype(np.float32)
    dconv = torch.from_numpy(conv).to(cuda) if ksize else None
    dhist = torch.from_numpy(hist.copy()).to(cuda) if ksize else None
    for call in range(2):
        x = rng.normal(size=k).astype(np.float32)
        ya = torch.empty(na, device=cuda)
        yb = torch.empty(nb, device=cuda)
        xq = ss = None
        if src == "norm data":
            xq = xgroup.buffer(torch, k, cuda)
            kernels.prep_x(torch.from_numpy(x * gamma).to(cuda), xq, k)
            xd = x.astype(np.float64).reshape(-1, 16)
            ss = torch.from_numpy((xd * xd).sum(axis=1)).to(cuda)
        kernels.gemv_x16_pair(ta, pa, na, ya, tb, pb, nb, yb, k, torch.from_numpy(x).to(cuda),
                              torch.from_numpy(gamma).to(cuda), 1e-6, dconv, dhist, ksize, xq=xq, sumsq=ss)
        xs = x.astype(np.float64)
        n = xs / np.sqrt(np.mean(xs * xs) + 1e-6) * gamma
        pre = fa @ n
        assert rel_err(yb.cpu().numpy(), fb @ n) <= 1e-3, call
        if not ksize:
            assert rel_err(ya.cpu().numpy(), pre) <= 1e-3, call
            continue
        win = np.concatenate([hist.astype(np.float64), pre[None, :]])  # [ksize, na]
        o = np.einsum("jc,cj->c", win, conv.astype(np.float64))
        assert rel_err(ya.cpu().numpy(), o / (1.0 + np.exp(-o))) <= 1e-3, call
        got_hist = dhist.cpu().numpy()
        np.testing.assert_array_equal(got_hist[:-1], hist[1:])
        assert rel_err(got_hist[-1], pre) <= 1e-3, call
        hist = got_hist.copy()


def test_pair_rejects_bad_arguments(cuda):
    w = torch.zeros(kernels.x16_bytes(synth.Q4_K, 16, 512), dtype=torch.uint8, device=cuda)
    v = torch.zeros(512, device=cuda)
    ok = (synth.Q4_K, w, 16, v, synth.Q4_K, w, 16, v, 512, v, v, 1e-6)
    kernels.gemv_x16_pair(*ok)
    for i, bad in ((0, synth.Q8_0), (8, 320), (11, 0.0)):
        args = list(ok)
        args[i] = bad
        with pytest.raises(ValueError):
            kernels.gemv_x16_pair(*args)
    with pytest.raises(ValueError):  # conv without a history
        kernels.gemv_x16_pair(*ok, conv_w=v, history=None, ksize=4)
    with pytest.raises(ValueError):  # ksize beyond the epilogue's four taps
        kernels.gemv_x16_pair(*ok, conv_w=v, history=v, ksize=5)
