"""Every buffer the head's ops leave uninitialised is poisoned before the library sees it.

The torch ops allocate their workspaces, and the outputs the library writes whole, with torch.empty. Here torch.empty
fills every device tensor it returns with 0xFF bytes: NaN in fp32, bf16 and f16, -1 in the integer counters and row
lists. A kernel that reads a byte its call did not write first would then propagate a NaN, a -1 count or a wrong
offset, and a call whose result depends on what memory held before (a fresh process on a fresh GPU holds whatever an
earlier job left) would show it here every time. Each case runs twice, plainly and poisoned, and the results must be
equal bit for bit. Where float atomics sum in an order that varies (a prefix tree's pair rows sum their flat tokens'
GRPO weights; the loss), they must agree to 1e-6 relative, which a NaN or a stray value does not.

Cases: the recomputing backward in fp32 at a vocabulary of 300 (W^T staged, dz past V zero-filled; the chunk-major
caller's shape), in bf16 and f16 over several passes and chunks through the compaction map; the fused step in bf16
(one pass, three passes with fp32 grad_W partials, most rows rescaled at T 0.01), f16 (the dz-scale pass), fp8
weights (grad_h alone over a staged W^T) and fp32 (its forward-then-backward fallback); the step over a prefix tree's
pair rows; the bound route with a rest to back-propagate; and the chunk-major caller itself."""

import contextlib

import numpy as np
import pytest
import torch

from octopus_amd import _lib, head_op
from octopus_amd.head_op import fused_head
from tests.test_gpu_step import EPS, _batch, _rel, _step_ws, _tree_batch

pytestmark = pytest.mark.gpu
DEV = "cuda"
CODE = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


@contextlib.contextmanager
def poisoned():
    """torch.empty returns device tensors filled with 0xFF bytes while the block runs."""
    real = torch.empty

    def empty(*args, **kwargs):
        t = real(*args, **kwargs)
        if t.is_cuda and t.numel():
            t.reshape(-1).view(torch.uint8).fill_(0xFF)
        return t

    torch.empty = empty
    try:
        yield
    finally:
        torch.empty = real


def _twice(fn):
    """fn() plainly, then under poisoned(): both results, synchronised."""
    a = fn()
    torch.cuda.synchronize()
    with poisoned():
        b = fn()
        torch.cuda.synchronize()
    return a, b


def _same(a, b, what):
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), (what, i, (x.float() - y.float()).abs().max().item())


def _bwd_ws(n, d, V, code, flags, want):
    """The largest backward workspace (10% steps down from the queried size) whose plan satisfies want(plan)."""
    ws = _lib.workspace_bytes(n, d, V, code, _lib.WS_BACKWARD | flags)
    while ws > (1 << 16):
        try:
            plan = _lib.bwd_plan(n, d, V, code, flags, ws)
        except ValueError:
            plan = None
        if plan is not None and want(plan):
            return ws
        ws = ws * 9 // 10
    raise AssertionError("no workspace gives the wanted plan")


BWD_CASES = {  # N, d, V, dtype, T, frozen weight, wanted plan (rows per pass, passes, columns, chunks)
    "f32-v300": (230, 64, 300, torch.float32, 0.8, False, None),
    "bf16-chunks": (2600, 256, 5120, torch.bfloat16, 0.9, False, lambda p: p[3] >= 3),
    "f16-passes-chunks-grad_h": (2600, 256, 5120, torch.float16, 0.9, True, lambda p: p[1] >= 2 and p[3] >= 2),
    "bf16-two-passes": (40000, 64, 2048, torch.bfloat16, 0.9, False, None),
}


@pytest.mark.parametrize("case", list(BWD_CASES))
def test_recomputing_backward_reads_only_what_it_wrote(case):
    """fp32 at V 300 (no compaction), one pass of several vocabulary chunks (fp32 grad_h partials), grad_h alone over
    passes x chunks, and 40,000 rows in two passes (fp32 grad_W partials); the last three through the compaction."""
    N, d, V, dtype, T, frozen, want = BWD_CASES[case]
    h, W, y, scored, _, _, _ = _batch(N, d, V, dtype, seed=41, scored_frac=0.9)
    g = torch.randn(N, generator=torch.Generator().manual_seed(42)).to(DEV)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    ws = None
    if want is not None:
        ws = _bwd_ws(N, d, V, CODE[dtype], _lib.WS_NO_GRADW if frozen else 0, want)

    def run():
        head_op.BWD_WORKSPACE_BYTES = ws
        try:
            h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(not frozen)
            kw = {} if case == "f32-v300" else dict(idx=idx, count=count, labels_via_idx=True, scatter=True)
            out = fused_head(h1, W1, yd, T, **kw)
            (out[:, 0] * g).sum().backward()
        finally:
            head_op.BWD_WORKSPACE_BYTES = None
        return (out.detach(), h1.grad) + (() if frozen else (W1.grad,))

    a, b = _twice(run)
    assert all(torch.isfinite(t).all() for t in a)
    _same(a, b, case)


STEP_CASES = {
    "bf16-one-pass": (torch.bfloat16, 1, 0.9, False),
    "bf16-three-passes": (torch.bfloat16, 3, 0.9, False),
    "bf16-rescaled-T0.01": (torch.bfloat16, 3, 0.01, False),
    "f16-three-passes": (torch.float16, 3, 0.9, False),
    "fp8-grad_h-alone": (torch.bfloat16, 3, 0.9, True),
    "f32-fallback": (torch.float32, 1, 0.9, False),
}


@pytest.mark.parametrize("case", list(STEP_CASES))
def test_fused_step_reads_only_what_it_wrote(case):
    dtype, passes, T, fp8 = STEP_CASES[case]
    N, d, V = 2400, 256, 4096
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, dtype, seed=43)
    hd, yd = h.to(DEV), y.to(DEV)
    sc = None
    if fp8:
        q, sc = head_op.quantise_fp8_rows(W.to(DEV))
        Wd, code = q, _lib.FP8E4M3
    else:
        Wd, code = W.to(DEV), CODE[dtype]
    idx, count = head_op.compact_rows(scored.to(DEV))
    n = int(scored.sum())
    flags = _lib.WS_NO_GRADW if fp8 else 0
    ws = None
    if passes > 1:
        ws, plan = _step_ws(n, d, V, code, flags, lambda p: p[1] >= passes)
    with torch.no_grad():
        logp = fused_head(hd, Wd, yd, T, idx=idx, count=count, labels_via_idx=True, scatter=True, w_scale=sc)[:, 0]
    old = logp + noise.to(DEV)  # the behaviour logprobs near the current ones, so every row's GRPO weight is alive
    args = (hd, Wd, sc, yd, idx, count, 1.0 / T, 1.0, 1.0, False, True, True, None, old, adv.to(DEV),
            mask.to(DEV), *EPS)

    def run():
        head_op.STEP_WORKSPACE_BYTES = ws
        try:
            return head_op.head_step_grpo(*args, True, not fp8)
        finally:
            head_op.STEP_WORKSPACE_BYTES = None

    a, b = _twice(run)
    out, lse, g, loss = a[:4]
    assert torch.isfinite(out).all() and torch.isfinite(loss)
    _same((a[0], a[1], a[2]) + tuple(a[4:]), (b[0], b[1], b[2]) + tuple(b[4:]), case)
    assert abs(a[3].item() - b[3].item()) <= 1e-6 * max(1.0, abs(a[3].item()))
    assert all(torch.isfinite(t.float()).all() for t in a[4:])


@pytest.mark.parametrize("device_pairs", [False, True], ids=["host_pairs", "device_pairs"])
def test_tree_step_reads_only_what_it_wrote(device_pairs):
    from octopus_amd.head_op import fused_grpo_tree_head
    from octopus_amd.rl.prefix_tree import TreeMeta
    flat, cu, scored, tree, h, W, adv, mask = _tree_batch(107)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    meta = (TreeMeta.on_device(t(flat), t(np.asarray(cu)), t(tree.flat_to_tree), len(tree.tokens), t(scored))
            if device_pairs else TreeMeta(tree, DEV))
    hd, Wd = h.to(DEV)[None], W.to(DEV)
    old = torch.full((len(flat),), -8.0, device=DEV)

    def run():
        h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
        loss, cols = fused_grpo_tree_head(h1, W1, meta, 0.8, adv.to(DEV), mask.to(DEV), old=old)
        loss.backward()
        return cols, loss.detach().reshape(1), h1.grad, W1.grad

    a, b = _twice(run)
    assert torch.equal(a[0], b[0])
    for x, y in zip(a[1:], b[1:]):
        assert torch.isfinite(x).all() and _rel(y, x) <= 1e-6


def test_bound_route_with_a_rest_reads_only_what_it_wrote():
    """The objective plus another term on the logprob column: the held gradients scaled, the rest's recomputing
    backward accumulated into them."""
    N, d, V, T = 1800, 256, 4096, 0.9
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=47)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    grpo = head_op.GrpoInputs(adv=adv.to(DEV), old=(noise - 8.0).to(DEV), prox=None, mask=mask.to(DEV))

    def run():
        h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
        out = head_op.grpo_bound_head(h1, W1, yd, T, grpo, idx=idx, count=count)
        logp = out[:, 0]
        loss, _ = head_op.grpo_loss(logp, None, grpo.old, grpo.adv, grpo.mask, *EPS)
        (loss + 0.3 * (grpo.mask * logp.float().pow(2)).sum() / logp.numel()).backward()
        return out.detach(), h1.grad, W1.grad

    a, b = _twice(run)
    assert all(torch.isfinite(t).all() for t in a)
    assert torch.equal(a[0], b[0])
    for x, y in zip(a[1:], b[1:]):
        assert _rel(y, x) <= 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_chunk_major_caller_poisoned(dtype):
    """The chunk-major caller's own checks (chunked forward and reverse-chunk backward against the whole-tree run and
    the fp64 oracle) with every uninitialised buffer poisoned."""
    from tests.test_chunk_major_head import _run
    with poisoned():
        _run("cuda", dtype, 1e-6 if dtype == torch.float32 else 2e-3, 1e-5 if dtype == torch.float32 else 1e-2)
