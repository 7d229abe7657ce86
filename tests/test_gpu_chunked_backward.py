"""The backward over row passes and vocabulary chunks: dz is staged one (pass, chunk) piece at a time within the
workspace it is given, grad_h sums the chunks in fp32, grad_W the passes. Each plan must give the oracle's gradients
(relative Frobenius error 1e-2 in 16-bit, 1e-4 in fp32), and plans of different sizes must agree with each other
to fp32 summation order (the 16-bit outputs to their own rounding). The workspace sizes are chosen from the
library's own plan query so that each case runs the chunking it names."""

import ctypes

import pytest
import torch

from octopus_amd import _lib, head_op
from octopus_amd.head_op import Post, fused_head
from oracle import head as ohead

pytestmark = pytest.mark.gpu
DEV = "cuda"
CODE = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


def _inputs(n, d, V, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype)
    W = (torch.randn(V, d, generator=g) * 0.02).to(dtype)
    y = torch.randint(0, V, (n,), generator=g)
    return h, W, y


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _workspace_for(n, d, V, code, flags, want):
    """The largest workspace (shrinking by 10% steps from the queried size) whose plan satisfies want(plan)."""
    ws = _lib.workspace_bytes(n, d, V, code, _lib.WS_BACKWARD | flags)
    while ws > (1 << 16):
        try:
            plan = _lib.bwd_plan(n, d, V, code, flags, ws)
        except ValueError:
            plan = None
        if plan is not None and want(plan):
            return ws, plan
        ws = ws * 9 // 10
    raise AssertionError("no workspace gives the wanted plan")


def _backward(h, W, y, T, g, post, cap, **kw):
    head_op.BWD_WORKSPACE_BYTES = cap
    try:
        hd = h.to(DEV).requires_grad_(True)
        Wd = W.to(DEV).requires_grad_(True)
        out = fused_head(hd, Wd, y.to(DEV), T, post, **kw)
        (out[:, 0] * g.to(DEV)).sum().backward()
        torch.cuda.synchronize()
    finally:
        head_op.BWD_WORKSPACE_BYTES = None
    return hd.grad.cpu(), Wd.grad.cpu()


# (2000, 256, 5120): grad_h reads each chunk's W rows K-major as stored; (2000, 256, 5000) and (1500, 136, 3001):
# V not a multiple of 64, so each chunk's W^T is staged (the last chunk partial, zero past V)
SHAPES = [(2000, 256, 5120), (2000, 256, 5000), (1500, 136, 3001)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_vocabulary_chunks_match_the_oracle(dtype, shape):
    n, d, V = shape
    h, W, y = _inputs(n, d, V, dtype, seed=71)
    g = torch.randn(n, generator=torch.Generator().manual_seed(72))
    code = CODE[dtype]
    ws, plan = _workspace_for(n, d, V, code, 0, lambda p: p[1] == 1 and p[3] >= 3)
    bar = 1e-4 if dtype == torch.float32 else 1e-2
    for T, post in ((1.0, Post()), (0.7, Post(0.5, 2.0, True))):
        gh_ref, gw_ref = ohead.head_backward(h, W, y, T, g, post.pre, post.post, post.tanh)
        gh, gw = _backward(h, W, y, T, g, post, ws)
        assert _rel(gh, gh_ref) <= bar and _rel(gw, gw_ref) <= bar, (plan, T, post)
        gh1, gw1 = _backward(h, W, y, T, g, post, None)  # one chunk
        if dtype == torch.float32:
            assert _rel(gh, gh1) <= 1e-5 and _rel(gw, gw1) <= 1e-5
        else:  # the chunked sums differ from the one-chunk sums in fp32 order only: at most the output's rounding
            assert _rel(gh, gh1) <= 4e-3 and _rel(gw, gw1) <= 4e-3
        # grad_W rows of each chunk come from that chunk alone: exact zeros stay exact
        assert torch.isfinite(gw).all() and torch.isfinite(gh).all()


def test_passes_and_chunks_with_compacted_rows():
    """Row passes times vocabulary chunks (grad_h only, so no grad_W partials), the rows read through the compaction
    map and the labels through idx; unscored rows get exactly zero gradient."""
    n, d, V = 3000, 256, 5120
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=73)
    mask = torch.rand(n, generator=torch.Generator().manual_seed(74)) < 0.7
    g_flat = torch.randn(n, generator=torch.Generator().manual_seed(75))
    idx, count = head_op.compact_rows(mask.to(DEV))
    sel = mask.nonzero()[:, 0]
    m = len(sel)
    ws, plan = _workspace_for(m, d, V, _lib.BF16, _lib.WS_NO_GRADW, lambda p: p[1] >= 2 and p[3] >= 2)
    head_op.BWD_WORKSPACE_BYTES = ws
    try:
        hd = h.to(DEV).requires_grad_(True)
        out = fused_head(hd, W.to(DEV), y.to(DEV), 0.7, idx=idx, count=count, labels_via_idx=True, scatter=True)
        (out[:, 0] * g_flat.to(DEV)).sum().backward()
        torch.cuda.synchronize()
    finally:
        head_op.BWD_WORKSPACE_BYTES = None
    gh_ref, _ = ohead.head_backward(h[sel], W, y[sel], 0.7, g_flat[sel], want_w=False)
    grad = hd.grad.cpu()
    assert (grad[~mask] == 0).all()
    assert _rel(grad[sel], gh_ref) <= 1e-2, plan


def test_passes_and_chunks_with_grad_w_partials():
    """More rows than one pass takes (two passes of 20,224) times vocabulary chunks, grad_W summed in fp32 across the
    passes and grad_h across the chunks: against the chunked fp32 torch reference on the GPU."""
    from tests.gpu_reference import head_fp32
    n, d, V = 40000, 128, 3000
    gen = torch.Generator(device=DEV).manual_seed(76)
    h = torch.randn(n, d, device=DEV, generator=gen).to(torch.bfloat16)
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, V, (n,), device=DEV, generator=gen)
    g = torch.randn(n, device=DEV, generator=gen)
    ws, plan = _workspace_for(n, d, V, _lib.BF16, 0, lambda p: p[1] == 2 and p[3] >= 3)
    _, _, gr, gw = head_fp32(h, W.float(), y, 0.7, g=g)
    head_op.BWD_WORKSPACE_BYTES = ws
    try:
        hd, Wd = h.clone().requires_grad_(True), W.clone().requires_grad_(True)
        out = fused_head(hd, Wd, y, 0.7)
        (out[:, 0] * g).sum().backward()
    finally:
        head_op.BWD_WORKSPACE_BYTES = None
    assert _rel(hd.grad, gr) <= 1e-2 and _rel(Wd.grad, gw) <= 1e-2, plan
    assert _rel(hd.grad[plan[0]:], gr[plan[0]:]) <= 1e-2  # the second pass's rows on their own


def test_fp8_weights_widened_chunk_by_chunk():
    """fp8 weights with a vocabulary wide enough that the forward widens them in two chunks (V d 2 bytes above
    256 MiB), and a backward to hidden over several chunks: against the oracle on the dequantised weights."""
    from octopus_amd.workloads import quantise_fp8_rows
    n, d, V = 96, 1024, 151936
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=77)
    Wq, scale = quantise_fp8_rows(W)
    W32 = Wq.float() * scale[:, None]
    g = torch.randn(n, generator=torch.Generator().manual_seed(78))
    ws, plan = _workspace_for(n, d, V, _lib.FP8E4M3, _lib.WS_NO_GRADW, lambda p: p[3] >= 3)
    head_op.BWD_WORKSPACE_BYTES = ws
    try:
        hd = h.to(DEV).requires_grad_(True)
        out = fused_head(hd, Wq.to(DEV), y.to(DEV), 1.0, w_scale=scale.to(DEV))
        (out[:, 0] * g.to(DEV)).sum().backward()
        torch.cuda.synchronize()
    finally:
        head_op.BWD_WORKSPACE_BYTES = None
    lp, ent, _ = ohead.head_forward(h, W32, y, 1.0)
    out = out.detach().cpu()
    assert (out[:, 0].double() - lp).abs().max() <= 2e-3 and (out[:, 1].double() - ent).abs().max() <= 2e-3
    gh_ref, _ = ohead.head_backward(h, W32, y, 1.0, g, want_w=False)
    assert _rel(hd.grad.cpu(), gh_ref) <= 1e-2, plan


def test_grad_w_accumulate_over_chunks_through_the_c_abi():
    """OCTO_GRADW_ACCUMULATE with a chunked plan: grad_w += each chunk's rows; grad_h in fp32 output."""
    n, d, V, T = 1000, 256, 4096, 0.8
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=79)
    g = torch.randn(n, generator=torch.Generator().manual_seed(80))
    hd, Wd, yd, gd = h.to(DEV), W.to(DEV), y.to(DEV), g.to(DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.zeros(n, 2, device=DEV)
    lse = torch.zeros(n, 2, device=DEV)
    ws = torch.empty(_lib.workspace_bytes(n, d, V, _lib.BF16, 0), dtype=torch.uint8, device=DEV)
    _lib.call("octo_head_fwd", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None, P(yd), None,
              None, n, d, V, _lib.LSE_PAIR, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse), P(out), 2, P(ws), ws.numel(), st)
    wsb_bytes, plan = _workspace_for(n, d, V, _lib.BF16, 0, lambda p: p[3] >= 4)
    wsb = torch.empty(wsb_bytes, dtype=torch.uint8, device=DEV)
    gh = torch.empty(n, d, dtype=torch.float32, device=DEV)
    base = (torch.randn(V, d, generator=torch.Generator().manual_seed(81)) * 1e-3).to(torch.float32)
    gw = base.to(DEV).clone()
    _lib.call("octo_head_bwd", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None, P(yd), None,
              None, n, d, V, _lib.LSE_PAIR | _lib.GRADW_ACCUMULATE, 1.0 / T, 1.0, 1.0, 0, P(lse), P(gd), P(gh), d,
              _lib.F32, P(gw), _lib.F32, P(wsb), wsb.numel(), st)
    torch.cuda.synchronize()
    gh_ref, gw_ref = ohead.head_backward(h, W, y, T, g)
    assert _rel(gh.cpu(), gh_ref) <= 1e-2, plan
    assert _rel(gw.cpu() - base, gw_ref) <= 1e-2, plan
