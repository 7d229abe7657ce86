"""Parity of the HIP path (through the C ABI, via octopus_amd.head_op) with the oracle.

Small shapes: every output against the fp64 oracle on the same inputs (the bf16 inputs rounded first), at
the required bars: logprob / entropy 1e-5 abs (fp32) and 2e-3 abs (bf16/f16); gradients relative
Frobenius error 1e-2 (bf16), 1e-4 (fp32); compaction and target gathers bit-exact.
Full-size configurations: all rows on the GPU, the oracle on a seeded subsample of rows, and a chunked
fp32 torch reference on the GPU for the gradients (which depend on every row)."""

import numpy as np
import pytest
import torch

from octopus_amd import head_op
from octopus_amd.head_op import Post, fused_head
from oracle import grpo as ogrpo
from oracle import head as ohead

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(n, d, V, dtype, seed=0, T_rows=None):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(T_rows or n, d, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype)
    W = (torch.randn(V, d, generator=g) * 0.02).to(dtype)  # the configurations' weight scale
    y = torch.randint(0, V, (T_rows or n,), generator=g)
    return h, W, y


def _tol(dtype):
    return 1e-5 if dtype == torch.float32 else 2e-3


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


SHAPES = [(1, 64, 100), (300, 64, 1000), (513, 256, 5000), (256, 40, 777), (1000, 128, 2048), (70, 2560, 3000)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{n}x{d}x{V}" for n, d, V in SHAPES])
def test_forward_matches_oracle(dtype, shape):
    n, d, V = shape
    h, W, y = _inputs(n, d, V, dtype)
    for T, post in ((1.0, Post()), (0.7, Post(0.5, 2.0, True)), (1.3, Post(0.25, 1.0, False))):
        out = fused_head(h.to(DEV), W.to(DEV), y.to(DEV), T, post).cpu()
        lp, ent, _ = ohead.head_forward(h, W, y, T, post.pre, post.post, post.tanh)
        tol = _tol(dtype)
        assert (out[:, 0].double() - lp).abs().max() <= tol, (T, post)
        assert (out[:, 1].double() - ent).abs().max() <= tol, (T, post)


# (1, 256, 64), (300, 256, 1024) and (513, 512, 4992): V a multiple of 64 and d of 256, so 16-bit grad_h reads W
# K-major as stored (4992 is not a multiple of the 256-wide tile); the others go through the staged W^T
BWD_SHAPES = [(1, 64, 100), (300, 64, 1000), (513, 256, 5000), (256, 40, 777), (70, 2560, 3000), (1, 256, 64),
              (300, 256, 1024), (513, 512, 4992)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", BWD_SHAPES, ids=str)
def test_backward_matches_oracle(dtype, shape):
    n, d, V = shape
    h, W, y = _inputs(n, d, V, dtype, seed=1)
    g = torch.randn(n, generator=torch.Generator().manual_seed(9))
    for T, post in ((1.0, Post()), (0.7, Post(0.5, 2.0, True))):
        hd = h.to(DEV).requires_grad_(True)
        Wd = W.to(DEV).requires_grad_(True)
        out = fused_head(hd, Wd, y.to(DEV), T, post)
        (out[:, 0] * g.to(DEV)).sum().backward()
        gh, gw = ohead.head_backward(h, W, y, T, g, post.pre, post.post, post.tanh)
        bar = 1e-4 if dtype == torch.float32 else 1e-2
        assert _rel(hd.grad.cpu(), gh) <= bar and _rel(Wd.grad.cpu(), gw) <= bar, (T, post)


def test_backward_over_two_passes_matches_fp32_reference():
    """More rows than one backward pass takes (32,768; here three passes of 23,296): each pass recomputes its dz,
    grad_h rows come from their own pass, and a 16-bit grad_W is the fp32 sum of the passes' partials, rounded
    once."""
    from tests.gpu_reference import head_fp32
    n, d, V = 65536 + 4096 + 3, 128, 1000
    gen = torch.Generator(device=DEV).manual_seed(21)
    h = torch.randn(n, d, device=DEV, generator=gen).to(torch.bfloat16)
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, V, (n,), device=DEV, generator=gen)
    g = torch.randn(n, device=DEV, generator=gen)
    hd, Wd = h.clone().requires_grad_(True), W.clone().requires_grad_(True)
    out = fused_head(hd, Wd, y, 0.7)
    (out[:, 0] * g).sum().backward()
    lp, ent, gr, gw = head_fp32(h, W.float(), y, 0.7, g=g)
    assert (out[:, 0] - lp).abs().max().item() <= 2e-3 and (out[:, 1] - ent).abs().max().item() <= 2e-3
    assert _rel(hd.grad, gr) <= 1e-2 and _rel(Wd.grad, gw) <= 1e-2
    # the rows of the last pass on their own
    assert _rel(hd.grad[2 * 23296:], gr[2 * 23296:]) <= 1e-2


FP8_SHAPES = [(1, 64, 100), (300, 64, 1000), (513, 256, 5000), (256, 48, 777), (70, 2560, 3000), (513, 512, 4992)]


@pytest.mark.parametrize("shape", FP8_SHAPES, ids=[f"{n}x{d}x{V}" for n, d, V in FP8_SHAPES])
def test_fp8_weights_match_oracle_on_dequantised_weights(shape):
    """e4m3 weights with per-row scales (bf16 hidden rows): logprob / entropy and grad_hidden against the oracle on
    the dequantised weights (e4m3 value x row scale), every row and through a compacted subset."""
    from octopus_amd.workloads import quantise_fp8_rows
    n, d, V = shape
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=3)
    Wq, scale = quantise_fp8_rows(W)
    W32 = Wq.float() * scale[:, None]
    g = torch.randn(n, generator=torch.Generator().manual_seed(5))
    for T, post in ((1.0, Post()), (0.7, Post(0.5, 2.0, True))):
        hd = h.to(DEV).requires_grad_(True)
        out = fused_head(hd, Wq.to(DEV), y.to(DEV), T, post, w_scale=scale.to(DEV))
        (out[:, 0] * g.to(DEV)).sum().backward()
        lp, ent, _ = ohead.head_forward(h, W32, y, T, post.pre, post.post, post.tanh)
        assert (out[:, 0].cpu().double() - lp).abs().max() <= 2e-3, (T, post)
        assert (out[:, 1].cpu().double() - ent).abs().max() <= 2e-3, (T, post)
        gh, _ = ohead.head_backward(h, W32, y, T, g, post.pre, post.post, post.tanh, want_w=False)
        assert _rel(hd.grad.cpu(), gh) <= 1e-2, (T, post)
    # scored subset: rows gathered through idx, outputs scattered back
    mask = torch.rand(n, generator=torch.Generator().manual_seed(6)) < 0.6
    mask[0] = True
    idx, count = head_op.compact_rows(mask.to(DEV))
    out = fused_head(h.to(DEV), Wq.to(DEV), y.to(DEV), 1.0, idx=idx, count=count, labels_via_idx=True,
                     scatter=True, w_scale=scale.to(DEV)).cpu()
    lp, ent, _ = ohead.head_forward(h[mask], W32, y[mask], 1.0)
    assert (out[~mask] == 0).all()
    assert (out[mask, 0].double() - lp).abs().max() <= 2e-3
    assert (out[mask, 1].double() - ent).abs().max() <= 2e-3


def test_compaction_is_bit_exact_nonzero():
    rng = np.random.default_rng(0)
    for n in (1, 63, 64, 65, 1023, 1024, 1025, 32768, 131072 + 7):
        m = torch.from_numpy(rng.random(n) < rng.random()).to(DEV)
        idx, count = head_op.compact_rows(m)
        ref = torch.nonzero(m)[:, 0]
        assert int(count.item()) == ref.numel()
        assert torch.equal(idx[:ref.numel()], ref)


def test_no_scored_rows_every_scored_row_and_zero_rows():
    """Edge cases of the compaction contract (the reference's `_scored_rows`, lm_head.py:124-130): a mask with no true
    entry gives a device count of 0, all-zero outputs and all-zero gradients (no tile of any GEMM runs); an all-true
    mask gives the unscored head bit for bit; zero rows give an empty [0, 2] output and empty gradients."""
    n, d, V = 300, 256, 1024
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=7)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    full = fused_head(hd, Wd, yd, 0.7)
    for fill, expect_full in ((False, False), (True, True)):
        mask = torch.full((n,), fill, dtype=torch.bool, device=DEV)
        idx, count = head_op.compact_rows(mask)
        assert int(count.item()) == (n if fill else 0)
        a = hd.clone().requires_grad_(True)
        b = Wd.clone().requires_grad_(True)
        out = fused_head(a, b, yd, 0.7, idx=idx, count=count, labels_via_idx=True, scatter=True)
        if expect_full:
            assert torch.equal(out, full)
        else:
            assert (out == 0).all()
        (out[:, 0] * torch.ones(n, device=DEV)).sum().backward()
        if not expect_full:
            assert (a.grad == 0).all() and (b.grad == 0).all()
        else:
            gh, gw = ohead.head_backward(h, W, y, 0.7, torch.ones(n))
            assert _rel(a.grad.cpu(), gh) <= 1e-2 and _rel(b.grad.cpu(), gw) <= 1e-2
    a = hd[:0].clone().requires_grad_(True)
    b = Wd.clone().requires_grad_(True)
    out = fused_head(a, b, yd[:0], 1.0)
    assert out.shape == (0, 2)
    out.sum().backward()
    assert a.grad.shape == (0, d) and (b.grad == 0).all()


def test_hidden_of_more_than_2_gib_through_idx():
    """A hidden matrix of 2 GiB or more read through idx (the GEMMs address mapped rows with 32-bit offsets): the
    library gathers the compact rows into its workspace first. Scored rows sit on both sides of the 2 GiB mark;
    outputs scattered to their positions and gradients against the oracle on the same rows."""
    rows_total, d, V = 270_000, 4096, 1024  # 2.21e9 bytes of bf16 hidden
    gen = torch.Generator(device=DEV).manual_seed(31)
    h = torch.randn(rows_total, d, device=DEV, generator=gen)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    assert h.numel() * 2 >= 2**31
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, V, (rows_total,), device=DEV, generator=gen)
    sel = torch.randperm(rows_total, generator=torch.Generator().manual_seed(32))[:1500]
    sel = torch.cat([sel, torch.tensor([0, rows_total - 1])]).unique()
    mask = torch.zeros(rows_total, dtype=torch.bool)
    mask[sel] = True
    idx, count = head_op.compact_rows(mask.to(DEV))
    g = torch.randn(sel.numel(), generator=torch.Generator().manual_seed(33))
    gfull = torch.zeros(rows_total)
    gfull[sel] = g
    a = h.requires_grad_(True)
    b = W.clone().requires_grad_(True)
    out = fused_head(a, b, y, 0.7, idx=idx, count=count, labels_via_idx=True, scatter=True)
    (out[:, 0] * gfull.to(DEV)).sum().backward()
    hs, ys = h.detach()[sel].cpu(), y[sel].cpu()
    lp, ent, _ = ohead.head_forward(hs, W.cpu(), ys, 0.7)
    o = out.detach()[sel].cpu().double()
    assert (o[:, 0] - lp).abs().max() <= 2e-3 and (o[:, 1] - ent).abs().max() <= 2e-3
    assert int((out.detach() != 0).any(dim=1).sum().item()) <= sel.numel()
    gh, gw = ohead.head_backward(hs, W.cpu(), ys, 0.7, g)
    assert _rel(a.grad[sel].cpu(), gh) <= 1e-2 and _rel(b.grad.cpu(), gw) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_extreme_logits_are_stable(dtype):
    """The online max / sum over vocabulary tiles at extreme logits. Every row's hidden vector is e_0, so logit j is
    W[j, 0] exactly: all-zero weights give logprob = -log V and entropy = log V (closed form); a 600-nat peak in the
    last vocabulary tile, with the other logits in [-50, 50], gives logprob 0 and entropy 0 at the peak's rows and
    about -600 elsewhere; logits near -1000 at T = 0.7 check the shift by the row max. Against the fp64 oracle, the
    absolute bar grows with the logits' magnitude (logprob = s_y - lse cancels two fp32 numbers of that size)."""
    n, d, V = 300, 64, 1000
    h = torch.zeros(n, d, dtype=dtype)
    h[:, 0] = 1.0
    gen = torch.Generator().manual_seed(41)
    base = torch.randint(-50, 51, (V,), generator=gen).to(torch.float32)
    y = torch.randint(0, V, (n,), generator=gen)
    y[::2] = 777
    tol0 = _tol(dtype)
    # all-zero weights: uniform over V
    W = torch.zeros(V, d, dtype=dtype)
    out = fused_head(h.to(DEV), W.to(DEV), y.to(DEV), 1.0).cpu().double()
    assert (out[:, 0] + np.log(V)).abs().max() <= tol0 and (out[:, 1] - np.log(V)).abs().max() <= tol0
    for T, col, big in ((1.0, base.clone().index_fill_(0, torch.tensor([777]), 600.0), 650.0),
                        (0.7, base / 10 - 1000.0, 1000.0 / 0.7)):
        W = torch.zeros(V, d)
        W[:, 0] = col
        W = W.to(dtype)
        hd = h.to(DEV).requires_grad_(True)
        Wd = W.to(DEV).requires_grad_(True)
        out = fused_head(hd, Wd, y.to(DEV), T)
        g = torch.randn(n, generator=torch.Generator().manual_seed(42))
        (out[:, 0] * g.to(DEV)).sum().backward()
        lp, ent, _ = ohead.head_forward(h, W, y, T)
        tol = tol0 + 4e-7 * big
        o = out.detach().cpu().double()
        assert torch.isfinite(o).all()
        assert (o[:, 0] - lp).abs().max() <= tol and (o[:, 1] - ent).abs().max() <= tol, T
        if T == 1.0:
            assert o[::2, 0].abs().max() <= tol and o[::2, 1].abs().max() <= tol  # the peak's rows
        gh, gw = ohead.head_backward(h, W, y, T, g)
        # the bar: the usual one plus the error of the reference's own composite in the same dtype (GEMM with its
        # logits in that dtype, fp32 log_softmax, autograd: dz cast to the dtype before the gradient GEMMs), which
        # is large where the weights' shared component makes grad_h a sum of large cancelling terms (at logits
        # near -1,400 nats: 1.2e-4 in fp32, 0.72 in bf16; this path: 1.6e-4 and 0.72)
        hr = h.detach().clone().requires_grad_(True)
        Wr = W.detach().clone().requires_grad_(True)
        (torch.log_softmax((hr @ Wr.T).float() / T, dim=1).gather(1, y[:, None])[:, 0] * g).sum().backward()
        bar = 1e-4 if dtype == torch.float32 else 1e-2
        bar_h = bar + 1.25 * _rel(hr.grad, gh)
        bar_w = bar + 1.25 * _rel(Wr.grad, gw)
        assert _rel(hd.grad.cpu(), gh) <= bar_h and _rel(Wd.grad.cpu(), gw) <= bar_w, (T, bar_h, bar_w)
    if dtype == torch.float32:  # _head_columns on the same logits, materialised: each dlogits row sums to 0
        from octopus_amd.rl import lm_head
        T = 0.7
        logits = (base / 10 - 1000.0).expand(n, V).contiguous()
        x = logits.to(DEV).requires_grad_(True)
        g = torch.randn(n, generator=torch.Generator().manual_seed(43))
        (lm_head._head_columns(x, T, y.to(DEV))[:, 0] * g.to(DEV)).sum().backward()
        s64 = logits.double() / T
        p64 = torch.softmax(s64, dim=1)
        dl64 = g.double()[:, None] * (torch.nn.functional.one_hot(y, V).double() - p64) / T
        assert (x.grad.cpu().double() - dl64).abs().max() <= 1e-5
        assert x.grad.cpu().double().sum(dim=1).abs().max() <= 1e-5


def test_hidden_of_more_than_2_gib_through_idx_over_two_backward_passes():
    """The gathered copy of the compact rows serves every backward pass: 70,000 scored rows (three passes of 23,552
    rows at most) of a 2.2 GB bf16 hidden matrix, against the chunked fp32 torch reference on the GPU."""
    from tests.gpu_reference import head_fp32
    rows_total, d, V = 270_000, 4096, 1000
    gen = torch.Generator(device=DEV).manual_seed(51)
    h = torch.randn(rows_total, d, device=DEV, generator=gen)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, V, (rows_total,), device=DEV, generator=gen)
    mask = torch.zeros(rows_total, dtype=torch.bool, device=DEV)
    mask[torch.randperm(rows_total, device=DEV, generator=gen)[:70_000]] = True
    idx, count = head_op.compact_rows(mask)
    n = int(count.item())
    assert n == 70_000
    g = torch.randn(rows_total, device=DEV, generator=gen) * mask
    a = h.requires_grad_(True)
    b = W.clone().requires_grad_(True)
    out = fused_head(a, b, y, 1.0, idx=idx, count=count, labels_via_idx=True, scatter=True)
    (out[:, 0] * g).sum().backward()
    sel = idx[:n]
    lp, ent, gr, gw = head_fp32(h.detach()[sel], W.float(), y[sel], 1.0, g=g[sel])
    assert (out.detach()[sel, 0] - lp).abs().max().item() <= 2e-3
    assert (out.detach()[sel, 1] - ent).abs().max().item() <= 2e-3
    assert _rel(a.grad[sel], gr) <= 1e-2 and _rel(b.grad, gw) <= 1e-2
    assert _rel(a.grad[sel][47104:], gr[47104:]) <= 1e-2  # the last pass's rows


def test_c_abi_plain_and_paired_row_state():
    """octo_head_fwd / octo_head_bwd through the C ABI with the plain natural-log lse (flags 0) and with the paired row
    state (OCTO_LSE_PAIR): the forward's outputs are the same bits either way, the plain lse is (m2 + l2S) ln 2 of the
    pair and matches the oracle, and both backward forms match the oracle's gradients."""
    import ctypes
    from octopus_amd import _lib
    n, d, V, T = 300, 256, 1024, 0.7
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=61)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    g = torch.randn(n, generator=torch.Generator().manual_seed(62))
    gd = g.to(DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lp_ref, ent_ref, lse_ref = ohead.head_forward(h, W, y, T)
    gh_ref, gw_ref = ohead.head_backward(h, W, y, T, g)
    res = {}
    for flags in (0, _lib.LSE_PAIR):
        out = torch.zeros(n, 2, device=DEV)
        lse = torch.zeros((n, 2) if flags else (n,), device=DEV)
        ws = torch.empty(_lib.workspace_bytes(n, d, V, _lib.BF16, 0), dtype=torch.uint8, device=DEV)
        _lib.call("octo_head_fwd", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None, P(yd),
                  None, None, n, d, V, flags, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse), P(out), 2, P(ws), ws.numel(),
                  st)
        wsb = torch.empty(_lib.workspace_bytes(n, d, V, _lib.BF16, _lib.WS_BACKWARD), dtype=torch.uint8, device=DEV)
        gh = torch.empty(n, d, dtype=torch.bfloat16, device=DEV)
        gw = torch.empty(V, d, dtype=torch.bfloat16, device=DEV)
        _lib.call("octo_head_bwd", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None, P(yd),
                  None, None, n, d, V, flags, 1.0 / T, 1.0, 1.0, 0, P(lse), P(gd), P(gh), d, _lib.BF16, P(gw),
                  _lib.BF16, P(wsb), wsb.numel(), st)
        torch.cuda.synchronize()
        res[flags] = (out.cpu(), lse.cpu(), gh.cpu(), gw.cpu())
        assert _rel(gh.cpu(), gh_ref) <= 1e-2 and _rel(gw.cpu(), gw_ref) <= 1e-2, flags
    (o0, l0, _, _), (o1, l1, _, _) = res[0], res[_lib.LSE_PAIR]
    assert torch.equal(o0, o1)
    assert ((l1[:, 0] + l1[:, 1]) * np.log(2.0) - l0).abs().max() <= 1e-6 * l0.abs().max() + 1e-6
    assert (l0.double() - lse_ref).abs().max() <= 2e-3
    assert (o0[:, 0].double() - lp_ref).abs().max() <= 2e-3 and (o0[:, 1].double() - ent_ref).abs().max() <= 2e-3


def test_scored_rows_equal_the_unscored_rows_bitwise():
    n, d, V = 777, 128, 3000
    h, W, y = _inputs(n, d, V, torch.bfloat16, seed=2)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    scored = torch.rand(n, generator=torch.Generator().manual_seed(3)) < 0.45
    idx, count = head_op.compact_rows(scored.to(DEV))
    full = fused_head(hd, Wd, yd, 0.7)
    part = fused_head(hd, Wd, yd, 0.7, idx=idx, count=count, labels_via_idx=True, scatter=True)
    s = scored.to(DEV)
    assert torch.equal(part[s], full[s]) and (part[~s] == 0).all()
    # gradients of a loss over the scored rows equal the unscored head's
    w = torch.randn(n, generator=torch.Generator().manual_seed(4)).to(DEV) * s
    grads = []
    for kw in (dict(), dict(idx=idx, count=count, labels_via_idx=True, scatter=True)):
        a = hd.clone().requires_grad_(True)
        b = Wd.clone().requires_grad_(True)
        (fused_head(a, b, yd, 0.7, **kw)[:, 0] * w).sum().backward()
        grads.append((a.grad, b.grad))
    assert torch.equal(grads[0][0], grads[1][0])
    # grad_W contracts over rows: the two runs sum the same terms in a different order before the bf16
    # rounding of the result, so they agree to bf16 resolution rather than bitwise
    assert _rel(grads[1][1].float(), grads[0][1].float()) < 2e-3


def test_pair_gather_and_expansion_match_the_reference_composition():
    """tree_head_output with the fused pair gather equals index_select + head + expansion (reference
    prefix_tree.py:419-421), values and gradients."""
    from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
    rng = np.random.default_rng(5)
    prefix = rng.integers(0, 500, 300)
    seqs = [np.concatenate([prefix, rng.integers(0, 500, k)]) for k in (40, 90, 7, 64)]
    flat = np.concatenate(seqs)
    cu = [0, *np.cumsum([len(s) for s in seqs]).tolist()]
    scored = rng.random(len(flat)) < 0.6
    meta = TreeMeta(build_tree(flat, cu, scored=scored), DEV)
    d, V = 64, 500
    h, W, _ = _inputs(meta.n_tokens, d, V, torch.float32, seed=6)
    hd = h.to(DEV)[None].requires_grad_(True)
    Wd = W.to(DEV).requires_grad_(True)

    def chunk(rows, labels):
        return fused_head(rows, Wd, labels, 0.9)

    chunk.octopus_fused_rows = lambda h2, pos, y: fused_head(h2, Wd, y, 0.9, idx=pos)
    out = tree_head_output(chunk, hd, meta)
    gw = torch.randn(out.shape, generator=torch.Generator().manual_seed(7)).to(DEV)
    (out * gw).sum().backward()
    g_fused = (hd.grad.clone(), Wd.grad.clone())
    hd.grad, Wd.grad = None, None
    pairs = fused_head(hd[0].index_select(0, meta.pair_pos), Wd, meta.pair_label, 0.9)
    ref = torch.cat([pairs, pairs.new_zeros(1, 2)]).index_select(0, meta.flat_pair)[None]
    (ref * gw).sum().backward()
    assert torch.equal(out, ref)
    assert _rel(g_fused[0], hd.grad) < 1e-6 and _rel(g_fused[1], Wd.grad) < 1e-6
    # the pairs themselves against the oracle
    lp, ent, _ = ohead.head_forward(h[meta.pair_pos.cpu()], W, meta.pair_label.cpu(), 0.9)
    assert (pairs[:, 0].detach().cpu().double() - lp).abs().max() < 1e-5


def test_bound_head_on_a_model_matches_its_own_logits():
    """The property of reference tests/test_lm_head.py:11-34 on the GPU, through the fused HIP head: once bound, a
    Llama, a softcapped Gemma2 and a Qwen3.5 (the reference's trained model: gated-delta-net linear attention and full
    attention layers) return each position's next-token log-probability and the entropy of their own fp32 logits
    (torch.distributions.Categorical), at T 1.0 and 0.7, to 1e-5."""
    from transformers import AutoModelForCausalLM
    from octopus_amd.rl.lm_head import bind_head
    from tests.tiny_models import families
    for name, config, _ in families():
        if name not in ("llama", "gemma2", "qwen3_5"):
            continue
        torch.manual_seed(3)
        model = AutoModelForCausalLM.from_config(config, attn_implementation="eager").to(DEV)
        model.eval()
        ids = torch.randint(0, config.vocab_size, (1, 19), generator=torch.Generator().manual_seed(4)).to(DEV)
        nxt = ids[0].roll(-1)
        with torch.no_grad():
            own = model(input_ids=ids).logits[0].double()
        for T in (1.0, 0.7):
            head = bind_head(model, T)
            head.octopus_labels, head.octopus_tree = nxt, None
            with torch.no_grad():
                cols = model(input_ids=ids).logits[0].double()
            want = torch.distributions.Categorical(logits=own / T)
            assert (cols[:, 0] - want.log_prob(nxt)).abs().max().item() <= 1e-5, (name, T)
            assert (cols[:, 1] - want.entropy()).abs().max().item() <= 1e-5, (name, T)


def test_head_columns_hip_matches_eager():
    """Reference tests/test_seq_tiles.py:145-165 for _head_columns: the HIP kernel against its eager twin."""
    from octopus_amd.rl import lm_head
    torch.manual_seed(0)
    logits = torch.randn(64, 1000, device=DEV, dtype=torch.bfloat16)
    labels = torch.randint(0, 1000, (64,), device=DEV)
    outs, grads = [], []
    for f in (lm_head._head_columns, lm_head._head_columns._torchdynamo_orig_callable):
        x = logits.detach().clone().float().requires_grad_() if f is not lm_head._head_columns else \
            logits.detach().clone().requires_grad_()
        out = f(x, 1.0, labels)
        out[:, 0].float().pow(2).sum().backward()
        outs.append(out.float())
        grads.append(x.grad.float())
    assert (outs[0] - outs[1]).abs().max() <= 2e-3
    assert (grads[0] - grads[1]).norm() <= 2e-2 * grads[1].norm() + 1e-6


def test_grpo_matches_oracle():
    rng = np.random.default_rng(8)
    n = 5000
    logp = np.log(rng.uniform(0.01, 1.0, n))
    prox = logp + rng.normal(0, 0.2, n)
    old = prox + rng.normal(0, 1.0, n)
    adv = rng.normal(0, 1, n)
    mask = (rng.random(n) < 0.7).astype(np.float32)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)  # noqa: E731
    for kw in (dict(prox=prox, old=old), dict(old=old), dict(prox=prox)):
        loss, g = head_op.grpo_loss(t(logp), None if "prox" not in kw else t(kw["prox"]),
                                    None if "old" not in kw else t(kw["old"]), t(adv), t(mask), 0.2, 0.28, 5.0)
        # the oracle on the same fp32-rounded inputs
        f = lambda a: np.asarray(a, dtype=np.float32).astype(np.float64)  # noqa: E731
        ref_loss, ref_g = ogrpo.grpo(f(logp), f(adv), mask, prox=None if "prox" not in kw else f(kw["prox"]),
                                     old=None if "old" not in kw else f(kw["old"]))
        assert abs(loss.item() - ref_loss) < 1e-4 * max(1.0, abs(ref_loss))
        assert np.abs(g.cpu().numpy() - ref_g).max() < 1e-6


def test_timing_hook_brackets_each_gemm_launch():
    """octo_timing_*: one gemm_stats launch per forward call, one each of the three backward GEMMs per backward
    call, with positive durations."""
    from octopus_amd import _lib
    h, W, y = _inputs(513, 256, 5000, torch.bfloat16, seed=3)
    hd, Wd = h.to(DEV).requires_grad_(True), W.to(DEV).requires_grad_(True)
    _lib.call("octo_timing_enable", 1)
    try:
        out = fused_head(hd, Wd, y.to(DEV), 1.0)
        out[:, 0].sum().backward()
        torch.cuda.synchronize()
        for name in ("gemm_stats", "gemm_dz", "gemm_store_grad_h", "gemm_store_grad_w"):
            n, ms = _lib.timing_read(name)
            assert n == 1 and ms > 0, name
    finally:
        _lib.call("octo_timing_enable", 0)


def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_small_heads_match_the_golden_fixtures(dtype):
    """The HIP path against the stored fp64 expectations (tests/golden/head_small.npz): forward columns and the
    gradients of sum(g * logprob), plain, temperature and soft-capped."""
    z = _golden("head_small.npz")
    for nm in ("plain", "temp", "softcap"):
        h, W, y, g = (torch.from_numpy(z[f"{nm}/{k}"]) for k in ("h", "W", "y", "g"))
        T, pre, post, tanh = z[f"{nm}/params"].tolist()
        hd = h.to(DEV, dtype).requires_grad_(True)
        Wd = W.to(DEV, dtype).requires_grad_(True)
        out = fused_head(hd, Wd, y.to(DEV), T, Post(pre, post, bool(tanh)))
        (out[:, 0] * g.to(DEV)).sum().backward()
        tol = _tol(dtype)
        o = out.detach().cpu().double()
        assert (o[:, 0] - torch.from_numpy(z[f"{nm}/logp"])).abs().max() <= tol, nm
        assert (o[:, 1] - torch.from_numpy(z[f"{nm}/ent"])).abs().max() <= tol, nm
        bar = 1e-4 if dtype == torch.float32 else 1e-2
        assert _rel(hd.grad.cpu(), torch.from_numpy(z[f"{nm}/grad_h"])) <= bar, nm
        assert _rel(Wd.grad.cpu(), torch.from_numpy(z[f"{nm}/grad_W"])) <= bar, nm


def test_cfg1_matches_the_golden_fixture():
    """The CPU-runnable configuration (N 512, d 1024, V 32,000, fp32), generated on the host as the fixture was,
    against its stored fp64 logprob / entropy at 1e-5."""
    from octopus_amd.workloads import CONFIGS, make_batch
    z = _golden("cfg1_expected.npz")
    b = make_batch(CONFIGS["cfg1"], "cpu")
    assert np.array_equal(b.labels.numpy(), z["labels"])
    out = fused_head(b.hidden.to(DEV), b.weight.to(DEV), b.labels.to(DEV), 1.0).cpu().double()
    assert (out[:, 0] - torch.from_numpy(z["logp"])).abs().max() <= 1e-5
    assert (out[:, 1] - torch.from_numpy(z["ent"])).abs().max() <= 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_fp8_row_quantiser_is_bit_exact(dtype):
    """octo_quantise_fp8_rows against the oracle (integer restatement of e4m3 rounding) and torch's float8
    conversion: the same codes and scales, bit for bit; rows of zeros, ties and half-subnormals included."""
    from octopus_amd.workloads import quantise_fp8_rows as torch_quantise
    from oracle import fp8 as ofp8
    g = torch.Generator().manual_seed(1)
    # d 2560: one wave per row, the row in registers; d 4100 (above 4096) and 36 (not a multiple of 8): the
    # workgroup-per-row form
    for V, d in ((777, 2560), (33, 4100), (50, 36)):
        W = torch.randn(V, d, generator=g) * 0.02
        W[3] = 0.0
        W[5, :6] = torch.tensor([448.0, 1.0625, -1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -(2.0 ** -11)])
        W = W.to(dtype)
        q, scale = head_op.quantise_fp8_rows(W.to(DEV))
        oq, oscale = ofp8.quantise_rows(W.float().numpy())
        assert np.array_equal(scale.cpu().numpy(), oscale), (V, d)
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), oq), (V, d)
        tq, ts = torch_quantise(W)  # torch on the CPU: IEEE fp32 division, e4m3 round to nearest even
        assert torch.equal(q.view(torch.uint8).cpu(), tq.view(torch.uint8)) and torch.equal(scale.cpu(), ts)


def test_fp8_row_quantiser_at_full_size_feeds_the_head():
    """The full [151,936, 2560] weight quantised on the device equals torch's CPU quantisation bit for bit, and
    the head on it equals the head on the CPU-quantised weight bitwise."""
    from octopus_amd.workloads import quantise_fp8_rows as torch_quantise
    V, d = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(1)
    W = (torch.randn(V, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    q, scale = head_op.quantise_fp8_rows(W)
    Wc = W.cpu()
    tq = torch.empty(V, d, dtype=torch.uint8)
    ts = torch.empty(V)
    for r0 in range(0, V, 16384):
        a, b = torch_quantise(Wc[r0:r0 + 16384])
        tq[r0:r0 + 16384], ts[r0:r0 + 16384] = a.view(torch.uint8), b
    assert torch.equal(q.view(torch.uint8).cpu(), tq) and torch.equal(scale.cpu(), ts)
    tq, ts = tq.to(DEV).view(torch.float8_e4m3fn), ts.to(DEV)
    h = torch.randn(300, d, device=DEV, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    y = torch.randint(0, V, (300,), device=DEV, generator=g)
    a = fused_head(h, q, y, 1.0, w_scale=scale)
    b = fused_head(h, tq, y, 1.0, w_scale=ts)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("variant", ["prox", "old", "prox+old"])
def test_forward_grpo_tail_matches_unfused(dtype, variant):
    """octo_head_fwd_grpo: the forward's outputs as octo_head_fwd's; g per compact row as octo_grpo_grad's on the
    forward's logprobs, gathered to compact order; the loss as its loss up to summation order; both against the
    oracle's GRPO restatement. The loss mask is a strict subset of the scored rows, so Z and the zero rows matter."""
    N, d, V = 1500, 64, 3000
    h, W, y = _inputs(N, d, V, dtype, seed=11)
    gen = torch.Generator().manual_seed(12)
    scored = torch.rand(N, generator=gen) < 0.6
    mask = (scored & (torch.rand(N, generator=gen) < 0.8)).float()
    adv = torch.randn(N, generator=gen)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    out, lse = head_op.head_fwd(hd, Wd, None, yd, idx, count, 1.0, 1.0, 1.0, False, True, True)
    lp = out[:, 0].cpu()
    prox = (lp + 0.3 * torch.randn(N, generator=gen)) if "prox" in variant else None
    old = (lp + 0.5 * torch.randn(N, generator=gen)) if "old" in variant else None
    dv = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    out2, lse2, g2, loss2 = head_op.head_fwd_grpo(hd, Wd, None, yd, idx, count, 1.0, 1.0, 1.0, False, True, True,
                                                  dv(prox), dv(old), adv.to(DEV), mask.to(DEV), 0.2, 0.28, 5.0)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    loss1, g1 = head_op.grpo_loss(out[:, 0], dv(prox), dv(old), adv.to(DEV), mask.to(DEV), 0.2, 0.28, 5.0)
    n = int(count.item())
    assert n == int(scored.sum())
    torch.testing.assert_close(g2[:n], g1[idx[:n]], rtol=1e-6, atol=0)
    assert abs(loss2.item() - loss1.item()) <= 1e-5 * max(1.0, abs(loss1.item()))
    lo, go = ogrpo.grpo(lp.numpy(), adv.numpy(), mask.numpy(), prox=None if prox is None else prox.numpy(),
                        old=None if old is None else old.numpy())
    assert np.abs(g2[:n].cpu().double().numpy() - go[idx[:n].cpu().numpy()]).max() <= 1e-6
    assert abs(loss2.item() - lo) <= 1e-5 * max(1.0, abs(lo))
