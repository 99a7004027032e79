"""qwen35moe parity on the GPU: every HipMoeLLM kernel against the float64
host reference (oracle/moe_ref.py, itself pinned by tests/test_moe_ref.py),
then whole models through the C ABI handle API.

Bars: router ids exact (ties to the lower id) and weights <= 1e-5; FP32
kernels <= 1e-4 relative to float64 (GEMVs <= 1e-3, the FP32 GEMV bound);
end to end: identical greedy tokens, identical expert routes at every layer
and step, logits within max|l - ref| / max|ref| <= 1e-3.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import oracle
from myllm_amd import synth
from myllm_amd.hipllm import HipLLM, LengthError, generate, kernels
from oracle import moe_ref
from tests import xgroup
from tests.test_gpu_kernels import dev_bytes, random_rows, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def t32(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(cuda)


# ------------------------------------------------------------ router
def test_router_topk_ties_and_weights(cuda):
    rng = np.random.default_rng(0)
    T, E, k = 6, 256, 8
    logits = rng.normal(size=(T, E + 1)).astype(np.float32)
    logits[1, [3, 9, 200]] = 5.0          # a three-way tie at the top
    logits[2, :] = 0.5                    # all equal: ids 0..7
    logits[3, [10, 11]] = logits[3].max() + 1.0
    ids = torch.empty(T, k, dtype=torch.int32, device=cuda)
    w = torch.empty(T, k, device=cuda)
    kernels.router_topk(t32(logits, cuda), E + 1, T, E, k, ids, w)
    for t in range(T):
        p = moe_ref.softmax(logits[t, :E].astype(np.float64))
        ri, rv = moe_ref.topk_insertion(p, k)
        assert ids[t].cpu().numpy().tolist() == ri.tolist(), t
        assert rel_err(w[t].cpu().numpy(), moe_ref.renorm(rv)) <= 1e-5
    assert ids[2].cpu().numpy().tolist() == list(range(8))


# ------------------------------------------------------------ batched / expert GEMV
@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q6_K])
def test_expert_gemv_routed(cuda, qtype):
    E, n, kdim, T, routes = 8, 96, 512, 3, 4
    w = random_rows(qtype, E * n, kdim, 41)
    dw = dev_bytes(w, cuda)
    rb = w.shape[1]
    wf = torch.empty(E * n, kdim, device=cuda)
    kernels.dequant_rows(qtype, dw, rb, E * n, kdim, wf)
    wf = wf.double().cpu().numpy().reshape(E, n, kdim)
    ids_np = np.array([[5, 0, 7, 2], [1, 1, 3, 6], [7, 4, 0, 5]], dtype=np.int32)
    # x per token (x_routed = False) and per route (x_routed = True)
    for routed in (False, True):
        rows = T * routes if routed else T
        x = synth.normal(rows * kdim, 42 + routed).reshape(rows, kdim)
        dx = t32(x, cuda)
        xs = torch.empty(rows, kdim, device=cuda)  # XGroup rows, kdim / 16 groups each
        for r in range(rows):
            kernels.prep_x(dx[r], xs[r], kdim)
        y = torch.empty(T * routes, n, device=cuda)
        kernels.gemv_batched(qtype, dw, None, rb, dx, xs, None, None, y, None, n, kdim, T * routes,
                             ids=torch.from_numpy(ids_np.reshape(-1).copy()).to(cuda), experts=E, routes=routes,
                             expert_stride=n * rb, x_routed=routed, ldx=kdim, ldy=n)
        got = y.double().cpu().numpy()
        for j in range(T * routes):
            e = ids_np.reshape(-1)[j]
            xr = x[j] if routed else x[j // routes]
            assert rel_err(got[j], wf[e] @ xr.astype(np.float64)) <= 1e-3, (routed, j)


@pytest.mark.parametrize("qtype", [synth.Q4_K, synth.Q8_0, synth.F32])
def test_batched_rows_and_swiglu(cuda, qtype):
    T, n, kdim = 5, 128, 512
    wg, wu = random_rows(qtype, n, kdim, 51), random_rows(qtype, n, kdim, 52)
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    rb = wg.shape[1]
    x = synth.normal(T * kdim, 53).reshape(T, kdim)
    dx = t32(x, cuda)
    xs = torch.empty(T, kdim, device=cuda)  # XGroup rows
    for r in range(T):
        kernels.prep_x(dx[r], xs[r], kdim)
    res = synth.normal(T * n, 54).reshape(T, n)
    y = torch.empty(T, n, device=cuda)
    kernels.gemv_batched(qtype, dg, None, rb, dx, xs, None, t32(res, cuda), y, None, n, kdim, T)
    G = torch.empty(n, kdim, device=cuda)
    U = torch.empty(n, kdim, device=cuda)
    kernels.dequant_rows(qtype, dg, rb, n, kdim, G)
    kernels.dequant_rows(qtype, du, rb, n, kdim, U)
    G, U = G.double().cpu().numpy(), U.double().cpu().numpy()
    ref = x.astype(np.float64) @ G.T + res
    assert rel_err(y.cpu().numpy(), ref) <= 1e-3
    yq = torch.empty(T, n, device=cuda)
    kernels.gemv_batched(qtype, dg, du, rb, dx, xs, None, None, y, yq, n, kdim, T)
    g, u = x.astype(np.float64) @ G.T, x.astype(np.float64) @ U.T
    ref = moe_ref.silu(g) * u
    got = y.double().cpu().numpy()
    assert rel_err(got, ref) <= 1e-3
    xgroup.check(yq, y.cpu().numpy())


# ------------------------------------------------------------ DeltaNet pieces
@pytest.mark.parametrize("qtype,E,K,T,n,kdim", [(synth.Q4_K, 256, 8, 1, 64, 512), (synth.Q8_0, 64, 4, 3, 32, 256),
                                                 (synth.Q6_K, 16, 2, 2, 48, 256)])
def test_gemv_routed_swiglu_matches_topk_then_batched(cuda, qtype, E, K, T, n, kdim):
    """Routing in the expert gate/up prologue against router_topk followed by
    the batched SwiGLU GEMV with those ids: the same ids and weights bit for
    bit, outputs within 1e-6 (separately compiled), XGroup form of the output."""
    rng = np.random.default_rng(31)
    wg = random_rows(qtype, E * n, kdim, 51)
    wu = random_rows(qtype, E * n, kdim, 52)
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    rb = wg.shape[1]
    x = synth.normal(T * kdim, 53).reshape(T, kdim)
    dx = t32(x, cuda)
    xs = torch.empty(T, kdim, device=cuda)
    for t in range(T):
        kernels.prep_x(dx[t], xs[t], kdim)
    logits = rng.normal(size=(T, E + 1)).astype(np.float32)
    logits[0, [3, 7]] = logits[0].max() + 1.0  # a tie at the top of token 0
    dl = t32(logits, cuda)
    ids_ref = torch.empty(T, K, dtype=torch.int32, device=cuda)
    w_ref = torch.empty(T, K, device=cuda)
    kernels.router_topk(dl, E + 1, T, E, K, ids_ref, w_ref)
    y_ref = torch.empty(T * K, n, device=cuda)
    yq_ref = xgroup.buffer(torch, n, cuda, T * K)
    kernels.gemv_batched(qtype, dg, du, rb, dx, xs, None, None, y_ref, yq_ref, n, kdim, T * K, ids=ids_ref.view(-1),
                         experts=E, routes=K, expert_stride=n * rb, x_routed=False, ldx=kdim, ldy=n)
    ids = torch.full((T, K), -1, dtype=torch.int32, device=cuda)
    wts = torch.empty(T, K, device=cuda)
    y = torch.empty(T * K, n, device=cuda)
    yq = xgroup.buffer(torch, n, cuda, T * K)
    kernels.gemv_routed_swiglu(qtype, dg, du, rb, dx, xs, kdim, y, yq, n, kdim, T, dl, E + 1, E, K, n * rb, ids, wts)
    assert torch.equal(ids, ids_ref)
    assert torch.equal(wts.view(torch.int32), w_ref.view(torch.int32))
    got, ref = y.cpu().numpy(), y_ref.cpu().numpy()
    assert rel_err(got, ref) <= 1e-6
    for v in range(T * K):
        xgroup.check(yq[v * n:(v + 1) * n], got[v])


@pytest.mark.parametrize("qtype,E,K,n,kdim,waves", [(synth.Q4_K, 256, 8, 64, 512, 0), (synth.Q6_K, 16, 2, 48, 768, 1104),
                                                    (synth.Q4_K, 32, 4, 512, 2048, 2108)])
def test_gemv_x16_routed_matches_vector_routes(cuda, qtype, E, K, n, kdim, waves):
    """The x16 routed expert GEMVs of one token against the vector ones on
    the GGUF rows: gate / up with the top-k in the kernel (ids and weights bit
    for bit, outputs within 1e-6, XGroup form of the output), then down by
    those ids from the routed SwiGLU outputs (within 1e-6)."""
    rng = np.random.default_rng(E + n)
    wg = random_rows(qtype, E * n, kdim, 61)
    wu = random_rows(qtype, E * n, kdim, 62)
    wd = random_rows(qtype, E * kdim, n, 63) if n % 256 == 0 else None
    dg, du = dev_bytes(wg, cuda), dev_bytes(wu, cuda)
    rb = wg.shape[1]

    def pack(w, rows, cols):
        p = torch.empty(kernels.x16_bytes(qtype, rows, cols), dtype=torch.uint8, device=cuda)
        kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], rows, cols, p)
        return p

    pg, pu = pack(wg, E * n, kdim), pack(wu, E * n, kdim)
    x = synth.normal(kdim, 64)
    dx = t32(x, cuda)
    xq = xgroup.buffer(torch, kdim, cuda)
    kernels.prep_x(dx, xq, kdim)
    logits = rng.normal(size=E).astype(np.float32)
    logits[[1, 5]] = logits.max() + 1.0  # a tie at the top
    dl = t32(logits, cuda)
    ids_ref = torch.empty(K, dtype=torch.int32, device=cuda)
    w_ref = torch.empty(K, device=cuda)
    y_ref = torch.empty(K, n, device=cuda)
    yq_ref = xgroup.buffer(torch, n, cuda, K)
    kernels.gemv_routed_swiglu(qtype, dg, du, rb, dx, xq, kdim, y_ref, yq_ref, n, kdim, 1, dl, E, E, K, n * rb,
                               ids_ref, w_ref)
    ids = torch.full((K,), -1, dtype=torch.int32, device=cuda)
    wts = torch.empty(K, device=cuda)
    y = torch.empty(K, n, device=cuda)
    yq = xgroup.buffer(torch, n, cuda, K)
    kernels.gemv_x16_routed(qtype, pg, pu, xq, kdim, False, y, yq, n, n, kdim, E, K, logits=dl, ids_out=ids,
                            weights_out=wts, waves=waves)
    assert torch.equal(ids, ids_ref)
    assert torch.equal(wts.view(torch.int32), w_ref.view(torch.int32))
    got = y.cpu().numpy()
    assert rel_err(got, y_ref.cpu().numpy()) <= 1e-6
    for v in range(K):
        xgroup.check(yq[v * n:(v + 1) * n], got[v])
    if wd is None:
        return
    pd = pack(wd, E * kdim, n)
    dd = dev_bytes(wd, cuda)
    d_ref = torch.empty(K, kdim, device=cuda)
    kernels.gemv_batched(qtype, dd, None, wd.shape[1], y, yq, None, None, d_ref, None, kdim, n, K, ids=ids,
                         experts=E, routes=K, expert_stride=kdim * wd.shape[1], x_routed=True, ldx=n, ldy=kdim)
    d = torch.empty(K, kdim, device=cuda)
    kernels.gemv_x16_routed(qtype, pd, None, yq, n, True, d, None, kdim, kdim, n, E, K, ids=ids)
    assert rel_err(d.cpu().numpy(), d_ref.cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("qr,qs,E,K,n,ff,ffs", [(synth.Q6_K, synth.Q8_0, 32, 8, 256, 512, 512),
                                                 (synth.Q4_K, synth.Q6_K, 16, 3, 64, 256, 768),
                                                 (synth.Q6_K, synth.Q4_K, 8, 1, 48, 1024, 256)])
def test_gemv_x16_moe_down_matches_down_and_combine(cuda, qr, qs, E, K, n, ff, ffs):
    """Routed down + shared down + combine in one launch against the routed
    x16 down launch followed by the shared down with the combine in its
    epilogue (vector GEMV on the GGUF rows), and against float64 over the
    oracle's dequantization; repeated ids included."""
    rng = np.random.default_rng(K + n)
    wd = random_rows(qr, E * n, ff, 71)
    ws = random_rows(qs, n, ffs, 72)

    def pack(t, w, rows, cols):
        p = torch.empty(kernels.x16_bytes(t, rows, cols), dtype=torch.uint8, device=cuda)
        kernels.pack_x16(t, dev_bytes(w, cuda), w.shape[1], rows, cols, p)
        return p

    pd, ps = pack(qr, wd, E * n, ff), pack(qs, ws, n, ffs)
    ids_np = rng.integers(0, E, size=K).astype(np.int32)
    if K > 2:
        ids_np[2] = ids_np[0]
    ids = torch.from_numpy(ids_np).to(cuda)
    act = rng.normal(size=(K, ff)).astype(np.float32)
    actq = xgroup.buffer(torch, ff, cuda, K)
    dact = t32(act, cuda)
    for j in range(K):
        kernels.prep_x(dact[j], actq[j * ff:(j + 1) * ff], ff)
    sx = rng.normal(size=ffs).astype(np.float32)
    wts = rng.random(K).astype(np.float32)
    sg = np.array([0.7], dtype=np.float32)
    res = rng.normal(size=n).astype(np.float32)
    y = torch.empty(n, device=cuda)
    gam = rng.normal(size=n).astype(np.float32)
    yq_out = xgroup.buffer(torch, n, cuda)
    ss_out = torch.empty(n // 16, dtype=torch.float64, device=cuda)
    kernels.gemv_x16_moe_down(qr, pd, ids, E, actq, ff, ff, qs, ps, t32(sx, cuda), ffs, t32(wts, cuda), t32(sg, cuda),
                              t32(res, cuda), y, n, K,
                              norm_out={"gamma_out": t32(gam, cuda), "yq_out": yq_out, "sumsq_out": ss_out})
    down = torch.empty(K, n, device=cuda)
    kernels.gemv_x16_routed(qr, pd, None, actq, ff, True, down, None, n, n, ff, E, K, ids=ids)
    y_ref = torch.empty(n, device=cuda)
    kernels.gemv_moe_combine(qs, dev_bytes(ws, cuda), ws.shape[1], t32(sx, cuda), t32(res, cuda), down,
                             t32(wts, cuda), t32(sg, cuda), K, y_ref, n, ffs)
    got = y.cpu().numpy()
    assert rel_err(got, y_ref.cpu().numpy()) <= 1e-5
    # The next norm's data: XGroup form of y * gamma, per-16 double sums of squares.
    xgroup.check(yq_out, got * gam)
    gd = got.astype(np.float64).reshape(-1, 16)
    np.testing.assert_allclose(ss_out.cpu().numpy(), (gd * gd).sum(axis=1), rtol=1e-13)
    fd = oracle.dequant_rows(qr, wd, ff).astype(np.float64).reshape(E, n, ff)
    fs = oracle.dequant_rows(qs, ws, ffs).astype(np.float64)
    routed = sum(float(wts[j]) * (fd[ids_np[j]] @ act[j].astype(np.float64)) for j in range(K))
    ref = res + routed + (fs @ sx.astype(np.float64)) / (1.0 + math.exp(-0.7))
    assert rel_err(got, ref) <= 1e-4


def test_gemv_x16_moe_down_rejects_bad_arguments(cuda):
    z = torch.zeros(1 << 16, dtype=torch.uint8, device=cuda)
    f = torch.zeros(4096, device=cuda)
    ids = torch.zeros(8, dtype=torch.int32, device=cuda)
    ok = [synth.Q6_K, z, ids, 4, f, 256, 256, synth.Q8_0, z, f, 256, f, f, f, f, 32, 2]
    kernels.gemv_x16_moe_down(*ok)
    for i, bad in ((0, synth.Q8_0), (7, synth.Q5_0), (6, 320), (10, 2304), (15, 40), (16, 9), (16, 0)):
        args = list(ok)
        args[i] = bad
        with pytest.raises((ValueError, OverflowError)):
            kernels.gemv_x16_moe_down(*args)


@pytest.mark.parametrize("qtype,E,K,T,n,kdim", [(synth.Q4_K, 32, 8, 5, 64, 512), (synth.Q6_K, 8, 4, 9, 48, 768),
                                                 (synth.Q4_K, 64, 8, 12, 512, 2048)])
def test_gemv_x16_grouped_matches_batched(cuda, qtype, E, K, T, n, kdim):
    """Expert-grouped x16 products of a prompt (groups of at most four
    vectors) against the batched vector GEMV by the same ids on the GGUF rows:
    gate / up with SwiGLU (outputs within 1e-6, XGroup form), then down from
    the routed SwiGLU outputs (within 1e-6)."""
    rng = np.random.default_rng(T + n)
    wg, wu = random_rows(qtype, E * n, kdim, 81), random_rows(qtype, E * n, kdim, 82)
    wd = random_rows(qtype, E * kdim, n, 83) if n % 256 == 0 else None

    def pack(w, rows, cols):
        p = torch.empty(kernels.x16_bytes(qtype, rows, cols), dtype=torch.uint8, device=cuda)
        kernels.pack_x16(qtype, dev_bytes(w, cuda), w.shape[1], rows, cols, p)
        return p

    pg, pu = pack(wg, E * n, kdim), pack(wu, E * n, kdim)
    x = rng.normal(size=(T, kdim)).astype(np.float32)
    dx = t32(x, cuda)
    xq = xgroup.buffer(torch, kdim, cuda, T)
    for t in range(T):
        kernels.prep_x(dx[t], xq[t * kdim:(t + 1) * kdim], kdim)
    ids_np = rng.integers(0, E, size=(T, K)).astype(np.int32)
    ids_np[1, :] = ids_np[0, :]  # experts shared by two tokens
    ids = torch.from_numpy(ids_np.reshape(-1).copy()).to(cuda)
    nv = T * K
    mg = kernels.route_groups_max(nv, E, 4)
    order = torch.empty(nv, dtype=torch.int32, device=cuda)
    groups = torch.empty(2 * mg, dtype=torch.int32, device=cuda)
    ngroups = torch.empty(1, dtype=torch.int32, device=cuda)
    kernels.route_groups(ids, nv, E, 4, order, groups, ngroups)
    y = torch.empty(nv, n, device=cuda)
    yq = xgroup.buffer(torch, n, cuda, nv)
    kernels.gemv_x16_grouped(qtype, pg, pu, xq, kdim, False, K, y, yq, n, n, kdim, E, order, groups, ngroups, mg)
    y_ref = torch.empty(nv, n, device=cuda)
    yq_ref = xgroup.buffer(torch, n, cuda, nv)
    kernels.gemv_batched(qtype, dev_bytes(wg, cuda), dev_bytes(wu, cuda), wg.shape[1], dx, xq, None, None, y_ref,
                         yq_ref, n, kdim, nv, ids=ids, experts=E, routes=K, expert_stride=n * wg.shape[1],
                         x_routed=False, ldx=kdim, ldy=n)
    got = y.cpu().numpy()
    assert rel_err(got, y_ref.cpu().numpy()) <= 1e-6
    for v in range(nv):
        xgroup.check(yq[v * n:(v + 1) * n], got[v])
    if wd is None:
        return
    pd = pack(wd, E * kdim, n)
    d = torch.empty(nv, kdim, device=cuda)
    kernels.gemv_x16_grouped(qtype, pd, None, yq, n, True, K, d, None, kdim, kdim, n, E, order, groups, ngroups, mg)
    d_ref = torch.empty(nv, kdim, device=cuda)
    kernels.gemv_batched(qtype, dev_bytes(wd, cuda), None, wd.shape[1], y, yq, None, None, d_ref, None, kdim, n, nv,
                         ids=ids, experts=E, routes=K, expert_stride=kdim * wd.shape[1], x_routed=True, ldx=n,
                         ldy=kdim)
    assert rel_err(d.cpu().numpy(), d_ref.cpu().numpy()) <= 1e-6


def test_gemv_routed_swiglu_rejects_bad_arguments(cuda):
    w = torch.zeros(272 * 64, dtype=torch.uint8, device=cuda)
    x = torch.zeros(256, device=cuda)
    y = torch.zeros(64, device=cuda)
    ids = torch.zeros(8, dtype=torch.int32, device=cuda)
    wts = torch.zeros(8, device=cuda)
    ok = dict(E=4, K=2, n=16, ld=5)

    def call(qtype=synth.Q8_0, **kw):
        a = {**ok, **kw}
        kernels.gemv_routed_swiglu(qtype, w, w, 272, x, x, 256, y, None, a["n"], 256, 1, x, a["ld"], a["E"], a["K"],
                                   a["n"] * 272, ids, wts)

    call()  # valid: equal logits route to experts 0 and 1 with weight 1/2
    torch.cuda.synchronize()
    assert ids[:2].cpu().numpy().tolist() == [0, 1]
    assert wts[:2].cpu().numpy().tolist() == [0.5, 0.5]
    with pytest.raises(LengthError):  # one wave holds at most 256 logits
        call(E=257, ld=257)
    for bad in (dict(K=9, E=16, ld=16), dict(K=5), dict(ld=3)):
        with pytest.raises(ValueError):
            call(**bad)
    with pytest.raises(ValueError):  # quantized weights only
        call(qtype=synth.F32)


@pytest.mark.parametrize("qtype,H,FFs,K", [(synth.Q8_0, 2048, 512, 8), (synth.Q4_K, 512, 768, 4)])
def test_gemv_moe_combine_matches_down_then_combine(cuda, qtype, H, FFs, K):
    """The combine in the shared down projection's epilogue against the down
    GEMV (same tiling, encode prologue) followed by moe_combine: within 1e-6
    (separately compiled), and against float64 within 1e-4."""
    rng = np.random.default_rng(33)
    wd = random_rows(qtype, H, FFs, 61)
    dw = dev_bytes(wd, cuda)
    rb = wd.shape[1]
    act = synth.normal(FFs, 62, stddev=0.5)
    res = rng.normal(size=H).astype(np.float32)
    down = rng.normal(size=(K, H)).astype(np.float32)
    wts = rng.uniform(size=K).astype(np.float32)
    wts /= wts.sum()
    sg = np.array([0.3, 0.0], dtype=np.float32)
    dact, dres, ddown, dwts, dsg = (t32(a, cuda) for a in (act, res, down, wts, sg))
    sh = torch.empty(H, device=cuda)
    kernels.gemv_norm(qtype, dw, rb, dact, None, 0.0, None, None, sh, H, FFs)
    ref = torch.empty(H, device=cuda)
    kernels.moe_combine(dres, ddown, dwts, sh, dsg, 1, ref, 1, H, K)
    out = torch.empty(H, device=cuda)
    kernels.gemv_moe_combine(qtype, dw, rb, dact, dres, ddown, dwts, dsg, K, out, H, FFs)
    got = out.cpu().numpy()
    assert rel_err(got, ref.cpu().numpy()) <= 1e-6
    wf = torch.empty(H, FFs, device=cuda)
    kernels.dequant_rows(qtype, dw, rb, H, FFs, wf)
    shared = wf.double().cpu().numpy() @ act.astype(np.float64)
    exact = res + wts.astype(np.float64) @ down + moe_ref.sigmoid(np.float64(sg[0])) * shared
    assert rel_err(got, exact) <= 1e-4


def test_gemv_moe_combine_rejects_bad_arguments(cuda):
    w = torch.zeros(34 * 16 * 64, dtype=torch.uint8, device=cuda)
    x = torch.zeros(9 * 512, device=cuda)
    with pytest.raises(ValueError):  # the epilogue holds at most 8 routes
        kernels.gemv_moe_combine(synth.Q8_0, w, 34 * 16, x, x, x, x, x, 9, x, 64, 512)
    with pytest.raises(ValueError):  # quantized weights only
        kernels.gemv_moe_combine(synth.F32, w, 2048, x, x, x, x, x, 8, x, 64, 512)
    with pytest.raises(ValueError):  # the prologue holds at most 8192 inputs
        kernels.gemv_moe_combine(synth.Q8_0, w, 34 * 16 * 20, x, x, x, x, x, 8, x, 1, 10240)


@pytest.mark.parametrize("n,E,vmax", [(512, 256, 64), (37, 8, 4), (16384, 256, 64), (1, 1, 64), (600, 8, 64),
                                      (3000, 1024, 4), (70, 100, 3)])
def test_route_groups(cuda, n, E, vmax):
    """The vectors sorted by expert (in any order inside one expert), cut
    into groups of at most vmax vectors of one expert, in expert order."""
    rng = np.random.default_rng(n + E)
    ids = rng.integers(0, E, size=n).astype(np.int32)
    if n > 4:
        ids[3] = E + 5   # out of range: the last expert, as the GEMVs clamp it
    cl = np.minimum(ids, E - 1)
    mg = kernels.route_groups_max(n, E, vmax)
    order = torch.full((n,), -1, dtype=torch.int32, device=cuda)
    groups = torch.full((2 * mg,), -1, dtype=torch.int32, device=cuda)
    ng = torch.zeros(1, dtype=torch.int32, device=cuda)
    kernels.route_groups(torch.from_numpy(ids).to(cuda), n, E, vmax, order, groups, ng)
    o = order.cpu().numpy()
    np.testing.assert_array_equal(np.sort(o), np.arange(n))            # a permutation
    np.testing.assert_array_equal(cl[o], np.sort(cl, kind="stable"))  # grouped by expert, in expert order
    counts = np.bincount(cl, minlength=E)
    expect, start = [], 0
    for e in range(E):
        for q in range(0, counts[e], vmax):
            expect.append((start + q, e | (min(vmax, counts[e] - q) << 16)))
        start += counts[e]
    ngroups = int(ng.item())
    assert ngroups == len(expect) <= mg
    np.testing.assert_array_equal(groups.cpu().numpy()[: 2 * ngroups].reshape(-1, 2),
                                  np.array(expect, dtype=np.int64).reshape(-1, 2))


@pytest.mark.parametrize("qtype,T,routed", [(synth.Q4_K, 40, False), (synth.Q6_K, 150, False),
                                            (synth.Q8_0, 30, True)])
def test_gemm_gather_matches_f16_operand_reference(cuda, qtype, T, routed):
    """Routed expert products as gathered fp16 matmuls against float64
    products of the fp16 operands (the scaled rows of hipllm_to_f16, the
    fp16-rounded weights; <= 1e-4), with experts holding more than one
    64-vector group (T = 150: about 75 vectors each) and rows of different
    magnitudes (the scale of each gathered row follows its source row)."""
    E, K, N, H = 8, 4, 256, 512
    rng = np.random.default_rng(T)
    w = random_rows(qtype, E * N, H, 81)
    dw = dev_bytes(w, cuda)
    rb = w.shape[1]
    nv = T * K
    xrows = nv if routed else T
    x = synth.normal(xrows * H, 82).reshape(xrows, H) * np.exp2(rng.integers(-10, 11, size=(xrows, 1)))
    x = torch.from_numpy(x.astype(np.float32)).to(cuda)
    xb = torch.empty(xrows, H, dtype=torch.float16, device=cuda)
    xs = torch.empty(xrows, dtype=torch.float32, device=cuda)
    kernels.to_f16(x, H, xb, xs, xrows, H)
    ids = torch.from_numpy(rng.integers(0, E, size=nv).astype(np.int32)).to(cuda)
    mg = kernels.route_groups_max(nv, E, 64)
    order = torch.empty(nv, dtype=torch.int32, device=cuda)
    groups = torch.empty(2 * mg, dtype=torch.int32, device=cuda)
    ng = torch.zeros(1, dtype=torch.int32, device=cuda)
    kernels.route_groups(ids, nv, E, 64, order, groups, ng)
    y = torch.full((nv, N), float("nan"), device=cuda)
    kernels.gemm_gather(qtype, dw, rb, xb, xs, y, N, H, N, order, groups, ng, mg, N * rb, K, routed)
    wf = torch.empty(E * N, H, device=cuda)
    kernels.dequant_rows(qtype, dw, rb, E * N, H, wf)
    wb = wf.to(torch.float16).double().reshape(E, N, H)
    xd = xb.double() * xs.double()[:, None]
    idn = ids.cpu().numpy()
    ref = torch.stack([wb[idn[j]] @ xd[j if routed else j // K] for j in range(nv)])
    got = y.double()
    err = ((got - ref).abs().max(dim=1).values / ref.abs().max(dim=1).values).max().item()
    print("max rel err", err)
    assert err <= 1e-4


def test_gemm_gather_rejects_bad_arguments(cuda):
    w = torch.zeros(144 * 64, dtype=torch.uint8, device=cuda)
    xb = torch.zeros(64, 256, dtype=torch.float16, device=cuda)
    xs = torch.ones(64, device=cuda)
    y = torch.zeros(64, device=cuda)
    i = torch.zeros(16, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError):  # k a multiple of 128
        kernels.gemm_gather(synth.Q8_0, w, 68, xb, xs, y, 4, 64, 4, i, i, i, 4, 4 * 68, 1, False)
    with pytest.raises(LengthError):  # one launch row per group
        kernels.gemm_gather(synth.Q4_K, w, 144, xb, xs, y, 4, 256, 4, i, i, i, 70000, 4 * 144, 1, False)
    with pytest.raises(ValueError):  # experts closer than their rows
        kernels.gemm_gather(synth.Q4_K, w, 144, xb, xs, y, 4, 256, 4, i, i, i, 4, 144, 1, False)
    with pytest.raises(ValueError):  # no row scales
        kernels.gemm_gather(synth.Q4_K, w, 144, xb, None, y, 4, 256, 4, i, i, i, 4, 4 * 144, 1, False)
    with pytest.raises(LengthError):
        kernels.route_groups(i, 16385, 8, 64, i, i, i)


@pytest.mark.parametrize("m,n,k", [(64, 257, 2048), (5, 33, 100), (512, 257, 2048), (1, 1, 1)])
def test_matmul_f32_matches_float64(cuda, m, n, k):
    rng = np.random.default_rng(m + n + k)
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = (rng.normal(size=(n, k)) / math.sqrt(k)).astype(np.float32)
    dx, dw = t32(x, cuda), t32(w, cuda)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    sf = kernels.matmul_f32_scratch_floats(m, n, k)
    results = []
    # with the K split (scratch for the partial sums) and without it
    for scratch in (torch.empty(max(sf, 1), device=cuda), None):
        y = torch.full((m, n + 3), float("nan"), device=cuda)
        kernels.matmul_f32(dx, k, dw, k, y, n + 3, m, n, k, scratch)
        got = y[:, :n].cpu().numpy()
        assert rel_err(got, ref) <= 1e-5
        assert np.isnan(y[:, n:].cpu().numpy()).all()  # columns past n untouched
        y2 = torch.empty(m, n + 3, device=cuda)
        kernels.matmul_f32(dx, k, dw, k, y2, n + 3, m, n, k, scratch)
        assert torch.equal(y[:, :n].view(torch.int32), y2[:, :n].view(torch.int32))  # fixed summation order
        results.append(got)


def test_gdn_gates(cuda):
    rng = np.random.default_rng(3)
    T, Hv = 4, 32
    ab = rng.normal(scale=5.0, size=(T, 2 * Hv)).astype(np.float32)
    ab[0, :4] = [25.0, -25.0, 20.5, -19.5]  # softplus branches
    dt = rng.normal(size=Hv).astype(np.float32)
    a = -np.abs(rng.normal(size=Hv)).astype(np.float32)
    decay, beta = torch.empty(T, Hv, device=cuda), torch.empty(T, Hv, device=cuda)
    dab = t32(ab, cuda)
    kernels.gdn_gates(dab, dab[:, Hv:], 2 * Hv, t32(dt, cuda), t32(a, cuda), decay, beta, T, Hv)
    ref_d = np.exp(moe_ref.softplus(ab[:, :Hv].astype(np.float64) + dt) * a)
    ref_b = moe_ref.sigmoid(ab[:, Hv:])
    assert rel_err(decay.cpu().numpy(), ref_d) <= 1e-5
    assert rel_err(beta.cpu().numpy(), ref_b) <= 1e-5


@pytest.mark.parametrize("ksize,T", [(2, 7), (4, 7), (4, 2), (4, 1), (4, 64), (9, 70), (4, 33)])
def test_conv1d_silu_and_history(cuda, ksize, T):
    # Prompts shorter than the history (T < ksize - 1 shifts old rows), one
    # chunk, several chunks with a ragged last one.
    rng = np.random.default_rng(4)
    C = 300
    x = rng.normal(size=(T, C)).astype(np.float32)
    hist = rng.normal(size=(ksize - 1, C)).astype(np.float32)
    w = rng.normal(size=(C, ksize)).astype(np.float32)
    dh = t32(hist, cuda)
    out = torch.empty(T, C, device=cuda)
    kernels.conv1d_silu(t32(x, cuda), C, dh, t32(w, cuda), out, C, T, C, ksize)
    h = hist.astype(np.float64)
    ref = np.empty((T, C))
    for t in range(T):
        o, h = moe_ref.conv_step(h, x[t].astype(np.float64), w.astype(np.float64))
        ref[t] = moe_ref.silu(o)
    assert rel_err(out.cpu().numpy(), ref) <= 1e-5
    np.testing.assert_array_equal(dh.cpu().numpy(), h.astype(np.float32))


def test_l2norm_heads(cuda):
    rng = np.random.default_rng(5)
    T, heads, d, ld = 3, 6, 128, 900
    x = rng.normal(size=(T, ld)).astype(np.float32)
    dx = t32(x, cuda)
    kernels.l2norm_heads(dx, ld, T, heads, d, 1e-6)
    got = dx.cpu().numpy()
    ref = moe_ref.l2norm(x[:, :heads * d].reshape(T, heads, d), 1e-6).reshape(T, -1)
    assert rel_err(got[:, :heads * d], ref) <= 1e-5
    np.testing.assert_array_equal(got[:, heads * d:], x[:, heads * d:])


# pad: extra columns per row, so that odd row strides take the scalar-load form.
@pytest.mark.parametrize("d,Hv,G,T,pad", [(128, 32, 16, 9, 0), (64, 4, 2, 9, 0), (128, 32, 16, 300, 0),
                                          (64, 4, 2, 33, 1), (128, 6, 3, 17, 3)])
def test_gdn_scan_matches_float64_steps(cuda, d, Hv, G, T, pad):
    rng = np.random.default_rng(6)
    qk = rng.normal(size=(T, 2, G, d))
    qk = qk / np.linalg.norm(qk, axis=-1, keepdims=True)
    v = rng.normal(size=(T, Hv, d))
    decay = rng.uniform(0.3, 1.0, size=(T, Hv))
    beta = rng.uniform(0.0, 1.0, size=(T, Hv))
    S0 = rng.normal(scale=0.1, size=(Hv, d, d))
    ldqk = 2 * G * d + Hv * d + pad
    buf = np.concatenate([qk.reshape(T, -1), v.reshape(T, -1), rng.normal(size=(T, pad))], axis=1)
    dbuf = t32(buf, cuda)
    state = t32(S0, cuda)
    out = torch.empty(T, Hv * d, device=cuda)
    kernels.gdn_scan(dbuf, dbuf[:, G * d:], ldqk, dbuf[:, 2 * G * d:], ldqk, t32(decay, cuda), t32(beta, cuda),
                     state, out, Hv * d, T, Hv, G, d)
    S = S0.astype(np.float32).astype(np.float64)
    ref = np.empty((T, Hv, d))
    f = lambda a: a.astype(np.float32).astype(np.float64)
    for t in range(T):
        S, ref[t] = moe_ref.gdn_step(S, f(qk[t, 0]), f(qk[t, 1]), f(v[t]), f(decay[t]), f(beta[t]), G)
    assert rel_err(out.cpu().numpy(), ref.reshape(T, -1)) <= 1e-4
    assert rel_err(state.cpu().numpy(), S) <= 1e-4


@pytest.mark.parametrize("d,Hv,G,T,pad", [(128, 32, 16, 1, 0), (128, 32, 16, 64, 0), (128, 32, 16, 100, 0),
                                          (128, 32, 16, 512, 0), (128, 32, 16, 2048, 0), (64, 4, 2, 130, 1),
                                          (128, 6, 3, 70, 3)])
def test_gdn_scan_chunked_matches_float64_steps(cuda, d, Hv, G, T, pad):
    # The chunk-parallel scan against the oracle's serial float64 steps
    # (prompt lengths of 1, 64, 100, 512 and 2048 tokens at the 35B-A3B
    # DeltaNet shape, ragged last chunks, a nonzero starting state), and
    # against the GPU serial scan on the same inputs.
    rng = np.random.default_rng(60 + T)
    qk = rng.normal(size=(T, 2, G, d))
    qk = qk / np.linalg.norm(qk, axis=-1, keepdims=True)
    v = rng.normal(size=(T, Hv, d))
    decay = rng.uniform(0.3, 1.0, size=(T, Hv))
    beta = rng.uniform(0.0, 1.0, size=(T, Hv))
    S0 = rng.normal(scale=0.1, size=(Hv, d, d))
    ldqk = 2 * G * d + Hv * d + pad
    buf = np.concatenate([qk.reshape(T, -1), v.reshape(T, -1), rng.normal(size=(T, pad))], axis=1)
    dbuf = t32(buf, cuda)
    dd, db = t32(decay, cuda), t32(beta, cuda)
    outs = {}
    for chunked in (True, False):
        state = t32(S0, cuda)
        out = torch.empty(T, Hv * d, device=cuda)
        if chunked:
            scratch = torch.empty(kernels.gdn_chunk_scratch_floats(T, Hv), device=cuda)
            kernels.gdn_scan_chunked(dbuf, dbuf[:, G * d:], ldqk, dbuf[:, 2 * G * d:], ldqk, dd, db, state, out,
                                     Hv * d, T, Hv, G, d, scratch)
        else:
            kernels.gdn_scan(dbuf, dbuf[:, G * d:], ldqk, dbuf[:, 2 * G * d:], ldqk, dd, db, state, out, Hv * d, T,
                             Hv, G, d)
        outs[chunked] = (out.cpu().numpy(), state.cpu().numpy())
    S = S0.astype(np.float32).astype(np.float64)
    ref = np.empty((T, Hv, d))
    f = lambda a: a.astype(np.float32).astype(np.float64)
    for t in range(T):
        S, ref[t] = moe_ref.gdn_step(S, f(qk[t, 0]), f(qk[t, 1]), f(v[t]), f(decay[t]), f(beta[t]), G)
    (oc, sc), (os_, ss) = outs[True], outs[False]
    print(f"chunked vs float64: out {rel_err(oc, ref.reshape(T, -1)):.2e} state {rel_err(sc, S):.2e}; "
          f"chunked vs serial GPU: out {rel_err(oc, os_):.2e}")
    assert rel_err(oc, ref.reshape(T, -1)) <= 1e-4
    assert rel_err(sc, S) <= 1e-4
    assert rel_err(oc, os_) <= 1e-4


def test_gdn_scan_chunked_rejects_bad_arguments(cuda):
    x = torch.zeros(64 * 512, device=cuda)
    small = torch.zeros(16, device=cuda)
    with pytest.raises(ValueError):  # scratch below hipllm_gdn_chunk_scratch_floats
        kernels.gdn_scan_chunked(x, x, 256, x, 256, x, x, x, x, 256, 64, 2, 1, 128, small)
    with pytest.raises(ValueError):  # state size 0
        kernels.gdn_scan_chunked(x, x, 256, x, 256, x, x, x, x, 256, 64, 2, 1, 0, x)


def test_gated_rmsnorm(cuda):
    rng = np.random.default_rng(7)
    T, Hv, d = 3, 8, 128
    o = rng.normal(size=(T, Hv * d)).astype(np.float32)
    z = rng.normal(size=(T, Hv * d)).astype(np.float32)
    g = rng.normal(size=d).astype(np.float32)
    y = torch.empty(T, Hv * d, device=cuda)
    yq = torch.empty(T, Hv * d, device=cuda)
    kernels.gated_rmsnorm(t32(o, cuda), Hv * d, t32(g, cuda), t32(z, cuda), Hv * d, y, yq, Hv * d, T, Hv, d, 1e-6)
    ref = (moe_ref.rmsnorm(o.reshape(T, Hv, d), g, 1e-6) * moe_ref.silu(z.reshape(T, Hv, d))).reshape(T, -1)
    got = y.cpu().numpy()
    assert rel_err(got, ref) <= 1e-5
    xgroup.check(yq, got)


@pytest.mark.parametrize("d", [64, 128])
def test_conv_l2norm_fused(cuda, d):
    # conv + SiLU + history over 5 head segments, the first 2 L2-normalised.
    rng = np.random.default_rng(14)
    T, C, ksize, nc = 6, 5 * d, 4, 2 * d
    x = rng.normal(size=(T, C)).astype(np.float32)
    hist = rng.normal(size=(ksize - 1, C)).astype(np.float32)
    w = rng.normal(size=(C, ksize)).astype(np.float32)
    dh = t32(hist, cuda)
    out = torch.empty(T, C, device=cuda)
    kernels.conv_l2norm(t32(x, cuda), C, dh, t32(w, cuda), out, C, T, C, ksize, nc, d, 1e-6)
    h = hist.astype(np.float64)
    ref = np.empty((T, C))
    for t in range(T):
        o, h = moe_ref.conv_step(h, x[t].astype(np.float64), w.astype(np.float64))
        ref[t] = moe_ref.silu(o)
    ref[:, :nc] = moe_ref.l2norm(ref[:, :nc].reshape(T, nc // d, d), 1e-6).reshape(T, nc)
    assert rel_err(out.cpu().numpy(), ref) <= 1e-5
    np.testing.assert_array_equal(dh.cpu().numpy(), h.astype(np.float32))


@pytest.mark.parametrize("d,Hv,G", [(128, 32, 16), (64, 4, 2)])
def test_gdn_scan_gated_matches_float64_steps(cuda, d, Hv, G):
    # Gates from raw alpha / beta, the recurrence and the gated RMSNorm in one
    # launch, against the float64 steps of the three.
    rng = np.random.default_rng(15)
    T = 7
    qk = rng.normal(size=(T, 2, G, d))
    qk = qk / np.linalg.norm(qk, axis=-1, keepdims=True)
    v = rng.normal(size=(T, Hv, d))
    ab = rng.normal(scale=2.0, size=(T, 2 * Hv)).astype(np.float32)
    dt = rng.normal(size=Hv).astype(np.float32)
    a = -np.abs(rng.normal(size=Hv)).astype(np.float32)
    z = rng.normal(size=(T, Hv * d)).astype(np.float32)
    gamma = rng.normal(size=d).astype(np.float32)
    S0 = rng.normal(scale=0.1, size=(Hv, d, d))
    ldqk = 2 * G * d + Hv * d
    buf = np.concatenate([qk.reshape(T, -1), v.reshape(T, -1)], axis=1)
    dbuf = t32(buf, cuda)
    dab = t32(ab, cuda)
    state = t32(S0, cuda)
    y = torch.empty(T, Hv * d, device=cuda)
    yq = torch.empty(T, Hv * d, device=cuda)
    kernels.gdn_scan_gated(dbuf, dbuf[:, G * d:], ldqk, dbuf[:, 2 * G * d:], ldqk, dab, dab[:, Hv:], 2 * Hv,
                           t32(dt, cuda), t32(a, cuda), state, t32(z, cuda), Hv * d, t32(gamma, cuda), y, yq, Hv * d,
                           T, Hv, G, d, 1e-6)
    f = lambda arr: arr.astype(np.float32).astype(np.float64)
    decay = np.exp(moe_ref.softplus(ab[:, :Hv].astype(np.float64) + dt) * a)
    beta = moe_ref.sigmoid(ab[:, Hv:].astype(np.float64))
    S = f(S0)
    ref = np.empty((T, Hv, d))
    for t in range(T):
        S, o = moe_ref.gdn_step(S, f(qk[t, 0]), f(qk[t, 1]), f(v[t]), decay[t], beta[t], G)
        ref[t] = moe_ref.rmsnorm(o, gamma, 1e-6) * moe_ref.silu(z[t].reshape(Hv, d))
    got = y.cpu().numpy()
    assert rel_err(got, ref.reshape(T, -1)) <= 1e-4
    assert rel_err(state.cpu().numpy(), S) <= 1e-4
    xgroup.check(yq, got)


@pytest.mark.parametrize("d,Hv,G,H", [(128, 32, 16, 2048), (64, 4, 2, 512), (64, 6, 3, 768)])
def test_gdn_decode_matches_float64_step(cuda, d, Hv, G, H):
    # One decode token after the projections: alpha / beta from the F32
    # projection of rmsnorm(x) * gamma, the Q / K L2 norms, gates, recurrence
    # and gated norm, against the float64 steps; three tokens in a row
    # (the state carries over).
    rng = np.random.default_rng(17)
    ab_w = rng.normal(scale=0.05, size=(2 * Hv, H)).astype(np.float32)
    xg = rng.normal(size=H).astype(np.float32)
    dt = rng.normal(size=Hv).astype(np.float32)
    a = -np.abs(rng.normal(size=Hv)).astype(np.float32)
    gamma = rng.normal(size=d).astype(np.float32)
    S0 = rng.normal(scale=0.1, size=(Hv, d, d)).astype(np.float32)
    state = t32(S0, cuda)
    S = S0.astype(np.float64)
    f = lambda arr: arr.astype(np.float32).astype(np.float64)
    for step in range(3):
        qkv = rng.normal(size=(2 * G + Hv) * d).astype(np.float32)
        x = rng.normal(size=H).astype(np.float32)
        z = rng.normal(size=Hv * d).astype(np.float32)
        y = torch.empty(Hv * d, device=cuda)
        yq = torch.empty(Hv * d, device=cuda)
        kernels.gdn_decode(t32(qkv, cuda), t32(x, cuda), t32(xg, cuda), t32(ab_w, cuda), H, t32(dt, cuda),
                           t32(a, cuda), state, t32(z, cuda), t32(gamma, cuda), y, yq, Hv, G, d, 1e-6)
        n = moe_ref.rmsnorm(x.astype(np.float64), xg, 1e-6)
        ab = ab_w.astype(np.float64) @ n
        decay = np.exp(moe_ref.softplus(ab[:Hv] + dt) * a)
        beta = moe_ref.sigmoid(ab[Hv:])
        qk = moe_ref.l2norm(qkv[:2 * G * d].astype(np.float64).reshape(2, G, d), 1e-6)
        S, o = moe_ref.gdn_step(S, qk[0], qk[1], f(qkv[2 * G * d:]).reshape(Hv, d), decay, beta, G)
        ref = moe_ref.rmsnorm(o, gamma, 1e-6) * moe_ref.silu(z.reshape(Hv, d))
        got = y.cpu().numpy()
        assert rel_err(got, ref.reshape(-1)) <= 1e-4, step
        assert rel_err(state.cpu().numpy(), S) <= 1e-4, step
        xgroup.check(yq, got)


def test_gdn_decode_rejects_bad_shapes(cuda):
    z = torch.zeros(8192, device=cuda)
    args = lambda Hv, G, d, H: (z, z, z, z, H, z, z, z, z, z, z, None, Hv, G, d, 1e-6)
    for bad in ((10, 4, 64, 512), (4, 4, 96, 512), (4, 4, 64, 0), (4, 4, 64, 4352)):
        with pytest.raises(ValueError):
            kernels.gdn_decode(*args(*bad))


# ------------------------------------------------------------ attention pieces
@pytest.mark.parametrize("hq,hkv,d,rot,pos", [(16, 2, 256, 64, 70), (16, 2, 256, 64, 128), (8, 2, 128, 128, 150),
                                              (14, 2, 64, 64, 250)])
def test_attn_decode_qgate_matches_split_and_gated_step(cuda, hq, hkv, d, rot, pos):
    """Head norms + RoPE / KV write + attention + output gate in one launch
    against split_qgate_norm followed by the gated decode step: both caches
    bit for bit, the output within 1e-6 of the largest value (the two
    kernels are compiled separately, and the compiler may fuse a multiply
    and add in one and not the other: 14 heads of 64 at 251 keys differ by a
    few ulps in one head) and its XGroup form."""
    rng = np.random.default_rng(pos + d)
    kvw = hkv * d
    cap = pos + 3
    mixed = rng.normal(size=hq * 2 * d).astype(np.float32)
    kv = rng.normal(size=2 * kvw).astype(np.float32)
    qg, kg = rng.normal(size=d).astype(np.float32), rng.normal(size=d).astype(np.float32)
    ang = rng.uniform(-3.0, 3.0, size=(cap, rot // 2)).astype(np.float32)
    table = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)).to(cuda)
    kc0 = rng.normal(size=(cap, kvw)).astype(np.float32)
    vc0 = rng.normal(size=(cap, kvw)).astype(np.float32)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(d)))
    dm, dkv, dqg, dkg = t32(mixed, cuda), t32(kv, cuda), t32(qg, cuda), t32(kg, cuda)
    outs = []
    for fused in (False, True):
        kc, vc = t32(kc0, cuda), t32(vc0, cuda)
        out = torch.empty(hq * d, device=cuda)
        outq = xgroup.buffer(torch, hq * d, cuda)
        if fused:
            kernels.attn_decode_qgate(dm, dkv, dqg, dkg, 1e-6, table, rot, kc, vc, out, outq, hq, hkv, d, pos, scale)
        else:
            ldqkv = (hq + 2 * hkv) * d
            qkv = torch.zeros(1, ldqkv, device=cuda)
            gate = torch.empty(1, hq * d, device=cuda)
            kernels.split_qgate_norm(dm, hq * 2 * d, dkv, 2 * kvw, dqg, dkg, qkv, ldqkv, gate, hq * d, 1, hq, hkv, d,
                                     1e-6)
            scratch = torch.empty(kernels.attn_decode_scratch_floats(hq, d, pos + 1), device=cuda)
            kernels.attn_decode_rope_gated(qkv, table, rot, kc, vc, gate, out, outq, scratch, hq, hkv, d, pos, scale)
        outs.append([t.cpu().numpy() for t in (out, kc, vc)])
        if fused:
            xgroup.check(outq, outs[-1][0])
    (o1, k1, v1), (o2, k2, v2) = outs
    assert np.array_equal(k1.view(np.uint32), k2.view(np.uint32))
    assert np.array_equal(v1.view(np.uint32), v2.view(np.uint32))
    assert rel_err(o2, o1) <= 1e-6


def test_attn_decode_qgate_rejects_other_lengths(cuda):
    z = torch.zeros(1 << 16, device=cuda)
    args = lambda d, pos: (z, z, z, z, 1e-6, z, 64, z, z, z, None, 16, 2, d, pos, 0.1)
    kernels.attn_decode_qgate(*args(256, 100))
    for d, pos in ((256, 10), (256, 300), (96, 100)):  # one chunk, five chunks, head size
        with pytest.raises(ValueError):
            kernels.attn_decode_qgate(*args(d, pos))


def test_split_qgate_norm_and_gate_mul(cuda):
    rng = np.random.default_rng(8)
    T, Hq, Hkv, D = 2, 4, 2, 256
    mixed = rng.normal(size=(T, Hq * 2 * D)).astype(np.float32)
    kv = rng.normal(size=(T, 2 * Hkv * D)).astype(np.float32)
    qg, kg = rng.normal(size=D).astype(np.float32), rng.normal(size=D).astype(np.float32)
    ldqkv = (Hq + 2 * Hkv) * D
    qkv = torch.zeros(T, ldqkv, device=cuda)
    gate = torch.empty(T, Hq * D, device=cuda)
    kernels.split_qgate_norm(t32(mixed, cuda), Hq * 2 * D, t32(kv, cuda), 2 * Hkv * D, t32(qg, cuda), t32(kg, cuda),
                             qkv, ldqkv, gate, Hq * D, T, Hq, Hkv, D, 1e-6)
    m = mixed.reshape(T, Hq, 2 * D).astype(np.float64)
    ref_q = moe_ref.rmsnorm(m[:, :, :D], qg, 1e-6).reshape(T, -1)
    ref_k = moe_ref.rmsnorm(kv[:, :Hkv * D].reshape(T, Hkv, D), kg, 1e-6).reshape(T, -1)
    got = qkv.cpu().numpy()
    assert rel_err(got[:, :Hq * D], ref_q) <= 1e-5
    assert rel_err(got[:, Hq * D:(Hq + Hkv) * D], ref_k) <= 1e-5
    np.testing.assert_array_equal(got[:, (Hq + Hkv) * D:], kv[:, Hkv * D:])
    np.testing.assert_array_equal(gate.cpu().numpy(), m[:, :, D:].reshape(T, -1).astype(np.float32))
    a = torch.randn(T, Hq * D, device=cuda)
    y = torch.empty_like(a)
    yq = torch.empty(T * Hq * D, device=cuda)
    kernels.gate_mul(a, gate, y, yq, T * Hq * D)
    ref = a.double().cpu().numpy() * moe_ref.sigmoid(gate.double().cpu().numpy())
    assert rel_err(y.cpu().numpy(), ref) <= 1e-5
    xgroup.check(yq, y.cpu().numpy())


def test_moe_combine(cuda):
    rng = np.random.default_rng(9)
    T, H, k, E = 3, 256, 4, 16
    res = rng.normal(size=(T, H)).astype(np.float32)
    down = rng.normal(size=(T * k, H)).astype(np.float32)
    w = rng.uniform(size=(T, k)).astype(np.float32)
    sh = rng.normal(size=(T, H)).astype(np.float32)
    rlog = rng.normal(size=(T, E + 1)).astype(np.float32)
    out = torch.empty(T, H, device=cuda)
    drlog = t32(rlog, cuda)
    kernels.moe_combine(t32(res, cuda), t32(down, cuda), t32(w, cuda), t32(sh, cuda), drlog[:, E:], E + 1, out, T,
                        H, k)
    ref = res + np.einsum("tr,trh->th", w.astype(np.float64), down.reshape(T, k, H)) + \
        sh * moe_ref.sigmoid(rlog[:, E:E + 1])
    assert rel_err(out.cpu().numpy(), ref) <= 1e-5


def _oracle_rmsnorm_rows(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    ref = np.ascontiguousarray(x, dtype=np.float32).copy()
    for r in range(ref.shape[0]):
        oracle.lib().oracle_rmsnorm(ref[r].ctypes.data, gamma.ctypes.data, ref.shape[1], ctypes.c_float(eps))
    return ref


@pytest.mark.parametrize("T,H,k", [(1, 2048, 8), (3, 256, 4), (2, 48, 2), (2, 50, 2), (1, 64, 10)])
def test_moe_combine_norm(cuda, T, H, k):
    """Combine + the next RMSNorm in one launch: the row equals the combine
    launch's, the norm equals the oracle's RMSNorm of that row bit for bit."""
    rng = np.random.default_rng(19)
    E = 16
    res = rng.normal(size=(T, H)).astype(np.float32)
    down = rng.normal(size=(T * k, H)).astype(np.float32)
    w = rng.uniform(size=(T, k)).astype(np.float32)
    sh = rng.normal(size=(T, H)).astype(np.float32)
    rlog = rng.normal(size=(T, E + 1)).astype(np.float32)
    gamma = (synth.normal(H, 7, stddev=0.5) + 1.0).astype(np.float32)
    drlog = t32(rlog, cuda)
    args = (t32(res, cuda), t32(down, cuda), t32(w, cuda), t32(sh, cuda), drlog[:, E:], E + 1)
    out_ref = torch.empty(T, H, device=cuda)
    kernels.moe_combine(*args, out_ref, T, H, k)
    out = torch.empty(T, H, device=cuda)
    norm = torch.empty(T, H, device=cuda)
    normq = xgroup.buffer(torch, H, cuda, T) if H % 16 == 0 else None
    kernels.moe_combine_norm(*args, out, t32(gamma, cuda), norm, normq, T, H, k, 1e-6)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), out_ref.cpu().numpy().view(np.uint32))
    ref = _oracle_rmsnorm_rows(got, gamma, 1e-6)
    gn = norm.cpu().numpy()
    assert np.array_equal(gn.view(np.uint32), ref.view(np.uint32))
    if normq is not None:
        for t in range(T):
            xgroup.check(normq[t * H:(t + 1) * H], gn[t])


def test_moe_combine_norm_rejects_bad_arguments(cuda):
    x = torch.zeros(64, device=cuda)
    with pytest.raises(Exception):  # eps must be positive
        kernels.moe_combine_norm(x, x, x, None, None, 0, x, x, x, None, 1, 64, 1, 0.0)
    with pytest.raises(Exception):  # XGroup output needs h % 16 == 0
        kernels.moe_combine_norm(x, x, x, None, None, 0, x, x, x, x, 1, 40, 1, 1e-6)


def test_attn_prefill_continues_a_cache(cuda):
    rng = np.random.default_rng(10)
    Hq, Hkv, D, pos0, rows = 4, 2, 256, 5, 3
    cap = pos0 + rows
    K = rng.normal(size=(cap, Hkv * D)).astype(np.float32)
    V = rng.normal(size=(cap, Hkv * D)).astype(np.float32)
    q = rng.normal(size=(rows, Hq * D)).astype(np.float32)
    out = torch.empty(rows, Hq * D, device=cuda)
    scale = 1 / math.sqrt(D)
    kernels.attn_prefill(t32(q, cuda), Hq * D, t32(K, cuda), t32(V, cuda), out, Hq * D, rows, Hq, Hkv, D, pos0, scale)
    ref = np.empty((rows, Hq * D))
    for r in range(rows):
        L = pos0 + r + 1
        for h in range(Hq):
            g = h // (Hq // Hkv)
            s = K[:L, g * D:(g + 1) * D].astype(np.float64) @ q[r, h * D:(h + 1) * D] * scale
            ref[r, h * D:(h + 1) * D] = moe_ref.softmax(s) @ V[:L, g * D:(g + 1) * D]
    assert rel_err(out.cpu().numpy(), ref) <= 1e-4


@pytest.mark.parametrize("hq,hkv,d,pos0,rows", [(28, 4, 128, 0, 37), (28, 4, 128, 3, 300), (14, 2, 64, 0, 21),
                                                (16, 2, 64, 0, 520), (16, 2, 256, 7, 45), (16, 2, 256, 0, 520),
                                                (8, 2, 96, 2, 9)])
def test_attn_prefill_tiles_match_float64(cuda, hq, hkv, d, pos0, rows):
    # Query tiles of 8 and 16 rows (the 300- and 520-row cases fill the grid
    # with 16-row tiles), ragged last tiles, a cache continued from pos0, and
    # a head size (96) the tiled form does not take. Cache rows past the
    # prompt hold NaN: the result must not read them.
    rng = np.random.default_rng(rows + d)
    cap = pos0 + rows + 20
    K = rng.normal(size=(cap, hkv * d)).astype(np.float32)
    V = rng.normal(size=(cap, hkv * d)).astype(np.float32)
    K[pos0 + rows:] = np.nan
    V[pos0 + rows:] = np.nan
    q = rng.normal(size=(rows, hq * d)).astype(np.float32)
    out = torch.empty(rows, hq * d, device=cuda)
    scale = 1 / math.sqrt(d)
    kernels.attn_prefill(t32(q, cuda), hq * d, t32(K, cuda), t32(V, cuda), out, hq * d, rows, hq, hkv, d, pos0, scale)
    L = pos0 + rows
    mask = np.arange(L)[None, :] > (pos0 + np.arange(rows))[:, None]
    ref = np.empty((rows, hq * d))
    for h in range(hq):
        g = h // (hq // hkv)
        kg = K[:L, g * d:(g + 1) * d].astype(np.float64)
        s = q[:, h * d:(h + 1) * d].astype(np.float64) @ kg.T * scale
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ref[:, h * d:(h + 1) * d] = p @ V[:L, g * d:(g + 1) * d].astype(np.float64)
    assert rel_err(out.cpu().numpy(), ref) <= 1e-4


# ------------------------------------------------------------ whole models
@pytest.fixture(scope="module")
def moe_tiny(tmp_path_factory):
    path = tmp_path_factory.mktemp("moe") / "moe-tiny.gguf"
    return synth.write_qwen35moe(path, synth.MOE_SHAPES["moe-tiny"], seed=3)


def run_pair(path, prompt, steps, max_sequence=64):
    ref = moe_ref.MoeRef(path, max_sequence)
    got_tok, ref_tok, errs, route_ok = [], [], [], []
    with HipLLM(path, max_sequence) as m:
        nxt = m.prefill(prompt)
        r = ref.prefill(prompt)
        for step in range(steps + 1):
            got_tok.append(nxt)
            ref_tok.append(r)
            lg = m.logits().astype(np.float64)
            errs.append(np.abs(lg - ref.logits).max() / np.abs(ref.logits).max())
            routes = m.routes()
            route_ok.append(all(routes[l].tolist() == ref.last_routes[l][0].tolist() for l in range(ref.L)))
            if step == steps:
                break
            nxt = m.decode(r)  # both continue from the reference's token
            r = ref.decode(r)
    return got_tok, ref_tok, np.array(errs), route_ok


def test_moe_tiny_matches_float64_reference(cuda, moe_tiny):
    prompt = synth.uniform_ids(8, 512, seed=11).tolist()
    got, ref, errs, routes = run_pair(moe_tiny, prompt, 8)
    print("max rel logit error per step:", errs.max())
    assert got == ref
    assert all(routes)
    assert errs.max() <= 1e-3


def test_moe_contract_and_stats(cuda, moe_tiny):
    with HipLLM(moe_tiny, 12) as m:
        assert m.config["architecture"] == "qwen35moe"
        assert m.uses_gpu and m.expert_cache_count == 8
        with pytest.raises(ValueError):
            m.decode(1)
        with pytest.raises(ValueError):
            m.prefill([])
        with pytest.raises(IndexError):
            m.prefill([1, 2, 512])
        with pytest.raises(LengthError):
            m.prefill(list(range(13)))
        a = generate(m, [3, 4, 5], 5)
        with pytest.raises(ValueError):
            m.prefill([1])
        b = generate(m, [3, 4, 5], 5)  # reset() zeroes the DeltaNet state
        assert a == b
        s = m.memory_stats()
        sh = synth.MOE_SHAPES["moe-tiny"]
        full = sh.layers // sh.full_attention_interval
        assert s["kv_cache_bytes"] == full * 2 * 12 * sh.kv_heads * sh.head_dim * 4
        dn = sh.layers - full
        assert s["recurrent_state_bytes"] == dn * (sh.time_step_rank * sh.state_size ** 2 +
                                                   (sh.conv_kernel - 1) * sh.qkv_width) * 4
    with pytest.raises(ValueError):
        HipLLM(moe_tiny, 12, expert_cache_count=2)  # below top-k


def test_moe_real_widths_match_float64_reference(cuda, tmp_path):
    # Qwen3.5-35B-A3B widths (2048 hidden, 256 experts top-8, 16 x 256 gated
    # attention, 32 x 128 DeltaNet), first four layers.
    shape = synth.MOE_SHAPES["qwen3.5-35b-a3b-4l"]
    path = synth.write_qwen35moe(tmp_path / "moe4l.gguf", shape, seed=5)
    prompt = synth.uniform_ids(5, shape.vocab, seed=12).tolist()
    got, ref, errs, routes = run_pair(path, prompt, 2, max_sequence=32)
    print("max rel logit error per step:", errs.max())
    assert got == ref
    assert all(routes)
    assert errs.max() <= 1e-3


def test_moe_prefill_matmul_path_real_widths(cuda, tmp_path):
    # A 20-row prompt at 35B-A3B widths takes the fp16 MFMA matmuls for the
    # dense projections (attention, DeltaNet and shared-expert projections):
    # logits within the 2e-2 prefill bar of the float64 graph, at the prompt's
    # last row and over the decode steps that follow. Every expert is routed
    # (top-8 of 8), so the graph is continuous in its inputs and fp16
    # rounding cannot flip a near-tie route (top-k is discontinuous; the
    # FP32 switch below covers the 256-expert routing).
    shape = synth.Qwen35MoeShape("moe-allroute-4l", 4, 2048, 16, 2, 256, 64, 4096, 4096, 8, 8, 512, 512, 4, 4, 128,
                                 16, 32, eos_token_id=4095)
    path = synth.write_qwen35moe(tmp_path / "moe4l-all.gguf", shape, seed=6)
    prompt = synth.uniform_ids(20, shape.vocab, seed=13).tolist()
    ref = moe_ref.MoeRef(path, 32)
    with HipLLM(path, 32) as m:
        m.prefill(prompt)
        first = m.logits().copy()
        r = ref.prefill(prompt)
        errs = []
        for step in range(3):
            lg = m.logits().astype(np.float64)
            errs.append(np.abs(lg - ref.logits).max() / np.abs(ref.logits).max())
            m.decode(r)  # both continue from the reference's token
            r = ref.decode(r)
        # K-split partial sums are added in a fixed order: a second prefill
        # of the same prompt gives the same bits.
        m.reset()
        m.prefill(prompt)
        assert np.array_equal(first.view(np.int32), m.logits().view(np.int32))
    print("max rel logit error per step:", errs)
    assert max(errs) <= 2e-2


def test_moe_fp32_prefill_switch_real_widths(cuda, tmp_path):
    # The same 20-row prompt on the 256-expert model with the matmul prefill
    # switched off: FP32 GEMVs for every row, so routes and tokens equal the
    # float64 graph's.
    shape = synth.MOE_SHAPES["qwen3.5-35b-a3b-4l"]
    path = synth.write_qwen35moe(tmp_path / "moe4l.gguf", shape, seed=6)
    prompt = synth.uniform_ids(20, shape.vocab, seed=13).tolist()
    ref = moe_ref.MoeRef(path, 32)
    with HipLLM(path, 32) as m:
        m.set_batched_prefill(False)
        got = m.prefill(prompt)
        assert got == ref.prefill(prompt)
        lg = m.logits().astype(np.float64)
        assert np.abs(lg - ref.logits).max() / np.abs(ref.logits).max() <= 1e-3
        routes = m.routes()
        assert all(routes[l].tolist() == ref.last_routes[l][0].tolist() for l in range(ref.L))


def test_moe_decode_graph_matches_eager_launches(cuda, moe_tiny):
    prompts = [synth.uniform_ids(5, 512, seed=21).tolist(), synth.uniform_ids(13, 512, seed=22).tolist()]
    out = {}
    for graphs in (True, False):
        toks, logits, routes = [], [], []
        with HipLLM(moe_tiny, 40) as m:
            m.set_decode_graphs(graphs)
            for prompt in prompts:
                m.reset()
                t = m.prefill(prompt)
                toks.append(t)
                for _ in range(8):
                    t = m.decode(t)
                    toks.append(t)
                    logits.append(m.logits())
                    routes.append(m.routes().copy())
        out[graphs] = (toks, logits, routes)
    assert out[True][0] == out[False][0]
    for a, b in zip(out[True][1], out[False][1]):
        assert np.abs(a - b).max() / np.abs(b).max() <= 1e-5
    for a, b in zip(out[True][2], out[False][2]):
        np.testing.assert_array_equal(a, b)



@pytest.mark.parametrize("prompt_len", [64, 160])
def test_moe_default_prefill_256_experts_routes_flip_only_at_near_ties(cuda, tmp_path, prompt_len):
    # The default prompt path at 35B-A3B widths (256 experts, top-8): fp16
    # MFMA dense projections feeding the FP32 router, the routed experts as
    # batched GEMVs (64 rows) or, from four routed vectors per expert, as
    # gathered fp16 matmuls (160 rows). Against the FP32 switch (whose routes
    # and tokens equal the float64 graph's, test above), layer by layer on
    # the prompt's last row:
    # * the router logits agree within the prefill bar (2e-2 of their largest);
    # * where the top-8 sets differ, every swapped pair is a near tie that
    #   the measured logit perturbation eps explains: an expert a kept by the
    #   FP32 path and dropped by fp16, and b the other way round, have FP32
    #   logits within 2 eps (a shift of at most eps each way reorders them);
    #   layers after the first flip see different inputs and are not compared;
    # * with no flip, the final logits agree within 2e-2 and the first token
    #   is the same unless the FP32 top-2 margin is inside that error.
    shape = synth.MOE_SHAPES["qwen3.5-35b-a3b-4l"]
    path = synth.write_qwen35moe(tmp_path / "moe4l.gguf", shape, seed=6)
    prompt = synth.uniform_ids(prompt_len, shape.vocab, seed=40 + prompt_len).tolist()
    res = {}
    for matmul in (True, False):
        with HipLLM(path, prompt_len + 4) as m:
            m.set_batched_prefill(matmul)
            m.set_route_probe(True)
            tok = m.prefill(prompt)
            res[matmul] = (tok, m.logits().astype(np.float64), m.routes(),
                           m.router_logits()[:, :shape.experts].astype(np.float64))
    (ta, la, ra, ga), (tb, lb, rb, gb) = res[True], res[False]
    flipped = False
    for layer in range(shape.layers):
        eps = np.abs(ga[layer] - gb[layer]).max()
        print(f"layer {layer}: router logit max diff {eps:.3e} (max |logit| {np.abs(gb[layer]).max():.3e})")
        assert eps <= 2e-2 * np.abs(gb[layer]).max()
        a_set, b_set = set(ra[layer].tolist()), set(rb[layer].tolist())
        if a_set == b_set:
            continue
        for kept in b_set - a_set:
            for taken in a_set - b_set:
                gap = gb[layer][kept] - gb[layer][taken]
                print(f"  flip: fp32 keeps {kept}, fp16 takes {taken}, fp32 logit gap {gap:.3e}")
                assert gap <= 2 * eps + 1e-6
        flipped = True
        break
    if not flipped:
        err = np.abs(la - lb).max() / np.abs(lb).max()
        top2 = np.sort(lb)[-2:]
        print(f"no route flip; logits rel err {err:.3e}, fp32 top-2 margin {top2[1] - top2[0]:.3e}")
        assert err <= 2e-2
        if top2[1] - top2[0] > 2 * np.abs(la - lb).max():
            assert ta == tb
