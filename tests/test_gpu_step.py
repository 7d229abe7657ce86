"""octo_head_step_grpo: the head's GRPO step (forward, GRPO weight and loss, backward) in one call, the logits
computed once per row pass.

The forward half runs the forward's own statistics and merge per row, so its outputs (logprob, entropy, row state,
g) must equal octo_head_fwd_grpo's bit for bit and its loss up to summation order. The backward half builds dz from
the stored exponentials instead of a recompute (bf16: one scale per row times exponentials stored relative to a
per-row offset; f16: half-tile exponentials scaled into dz), so its gradients must match octo_head_bwd's for the same
g to the 16-bit roundings involved, and the fp64 oracle (oracle/head.py, with g from oracle/grpo.py on the same logprobs) within
the relative Frobenius bar 1e-2 (16-bit; 1e-4 for fp32, which runs the forward and the backward). The cases cover
the plan's branches: one pass and several (fp32 grad_W partials, passes past the device row count), W read K-major
as stored and W^T staged (V not a multiple of 64), the softcap, fp8 weights (grad_h only), the compacted rows read
through idx with labels per hidden row, and OCTO_GRADW_ACCUMULATE through the C ABI."""

import ctypes

import numpy as np
import pytest
import torch

from octopus_amd import _lib, head_op
from oracle import grpo as ogrpo
from oracle import head as ohead

pytestmark = pytest.mark.gpu
DEV = "cuda"
CODE = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}
EPS = (0.2, 0.28, 5.0)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _batch(N, d, V, dtype, seed, scored_frac=0.6, wscale=1.0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, d, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype)
    W = (torch.randn(V, d, generator=g) * 0.02 * wscale).to(dtype)
    y = torch.randint(0, V, (N,), generator=g)
    scored = torch.rand(N, generator=g) < scored_frac
    mask = (scored & (torch.rand(N, generator=g) < 0.85)).float()
    adv = torch.randn(N, generator=g)
    noise = 0.05 * torch.randn(N, generator=g)
    return h, W, y, scored, mask, adv, noise


def _step_ws(n, d, V, code, flags, want):
    """The largest workspace (shrinking by 10% steps from the queried size) whose step plan satisfies want(plan)."""
    ws = _lib.workspace_bytes(n, d, V, code, _lib.WS_STEP | flags)
    while ws > (1 << 16):
        try:
            plan = _lib.bwd_plan(n, d, V, code, _lib.WS_STEP | flags, ws)
        except ValueError:
            plan = None
        if plan is not None and want(plan):
            return ws, plan
        ws = ws * 9 // 10
    raise AssertionError("no workspace gives the wanted plan")


def _run(h, W, y, scored, mask, adv, old, T, post=(1.0, 1.0, False), w_scale=None, need_w=True, ws=None):
    """(step outputs, two-call outputs) on the GPU, both through compaction of the scored rows."""
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    sc = None if w_scale is None else w_scale.to(DEV)
    pre, pst, tanh = post
    args = (hd, Wd, sc, yd, idx, count, 1.0 / T, pre, pst, tanh, True, True, old.to(DEV), None, adv.to(DEV),
            mask.to(DEV), *EPS)
    head_op.STEP_WORKSPACE_BYTES = ws
    try:
        step = head_op.head_step_grpo(*args, True, need_w)
    finally:
        head_op.STEP_WORKSPACE_BYTES = None
    out, lse, g, loss = head_op.head_fwd_grpo(*args)
    grads = head_op.head_bwd(hd, Wd, sc, yd, idx, count, lse, g, 1.0 / T, pre, pst, tanh, True, True, need_w)
    torch.cuda.synchronize()
    return idx, count, step, (out, lse, g, loss) + tuple(grads)


def _check(h, W32, y, scored, mask, adv, old, T, post, step, two, need_w, bar, vs_two):
    out_s, lse_s, g_s, loss_s, gh_s, gw_s = step
    out_t, lse_t, g_t, loss_t, gh_t, gw_t = two
    # the forward half: the forward's own outputs
    assert torch.equal(out_s, out_t) and torch.equal(lse_s, lse_t) and torch.equal(g_s, g_t)
    assert abs(loss_s.item() - loss_t.item()) <= 1e-5 * max(1.0, abs(loss_t.item()))
    sel = scored.nonzero()[:, 0]
    n = sel.numel()
    # g and the loss against the oracle's GRPO on the same logprobs
    lp = out_s[:, 0].cpu().double().numpy()
    lo, go = ogrpo.grpo(lp, adv.numpy(), mask.numpy(), prox=old.double().numpy(), eps_lo=EPS[0], eps_hi=EPS[1],
                        reject_upper=EPS[2])
    assert np.abs(g_s[:n].cpu().double().numpy() - go[sel.numpy()]).max() <= 1e-6
    assert abs(loss_s.item() - lo) <= 1e-5 * max(1.0, abs(lo))
    # the backward half: against the two-call backward and the oracle on the scored rows
    gh_ref, gw_ref = ohead.head_backward(h[sel], W32, y[sel], T, g_s[:n].cpu(), *post, want_w=need_w)
    gh_s = gh_s.cpu()
    assert (gh_s[~scored] == 0).all()
    assert _rel(gh_s[sel], gh_ref) <= bar
    assert _rel(gh_s, gh_t.cpu()) <= vs_two
    if need_w:
        assert _rel(gw_s.cpu(), gw_ref) <= bar
        assert _rel(gw_s.cpu(), gw_t.cpu()) <= vs_two
    assert torch.isfinite(gh_s).all()


# (1500, 256, 5120): grad_h reads W K-major as stored; (1500, 136, 3001): V not a multiple of 64, W^T staged
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", [(1500, 256, 5120), (1500, 136, 3001)], ids=str)
def test_step_matches_forward_backward_and_oracle(dtype, shape):
    N, d, V = shape
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, dtype, seed=91)
    bar = 1e-4 if dtype == torch.float32 else 1e-2
    # 16-bit: dz differs from the backward's by the rounding of the stored exponential (bf16: 2^-9 relative in place
    # of the backward's rounding of dz, and the scaled h^T's; f16: 2^-11 relative besides it)
    vs_two = 1e-6 if dtype == torch.float32 else 4e-3
    for T, post in ((1.0, (1.0, 1.0, False)), (0.7, (0.5, 2.0, True))):
        lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None, y.to(DEV), None, None, 1.0 / T, *post, False, False)[0]
        old = lp0[:, 0].cpu() + noise
        idx, count, step, two = _run(h, W, y, scored, mask, adv, old, T, post)
        _check(h, W.float(), y, scored, mask, adv, old, T, post, step, two, True, bar, vs_two)


def test_step_over_passes_with_grad_w_partials_and_the_device_count():
    """Three passes over the 6,000 compact rows, 60% of them scored (the compaction puts the scored rows first): the
    first pass is all scored rows, the second reaches the device count, and the third starts past it, so its grad_W
    launch stores nothing and the second one's writes grad_W (adding the fp32 partials of the first)."""
    N, d, V = 6000, 256, 5120
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=92)
    ws, plan = _step_ws(N, d, V, _lib.BF16, 0, lambda p: p[1] == 3)
    n = int(scored.sum())
    assert plan[0] < n < 2 * plan[0], (plan, n)
    lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None, y.to(DEV), None, None, 1.0, 1.0, 1.0, False, False, False)[0]
    old = lp0[:, 0].cpu() + noise
    idx, count, step, two = _run(h, W, y, scored, mask, adv, old, 1.0, ws=ws)
    _check(h, W.float(), y, scored, mask, adv, old, 1.0, (1.0, 1.0, False), step, two, True, 1e-2, 4e-3)


def test_step_passes_against_the_fp32_reference():
    """Two passes (32,768 rows, then 7,232) without compaction, grad_W summed in fp32 across them: against the chunked
    fp32 torch reference on the GPU, and its second pass's rows on their own."""
    from tests.gpu_reference import head_fp32
    N, d, V = 40000, 128, 3000
    gen = torch.Generator(device=DEV).manual_seed(93)
    h = torch.randn(N, d, device=DEV, generator=gen).to(torch.bfloat16)
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, V, (N,), device=DEV, generator=gen)
    adv = torch.randn(N, device=DEV, generator=gen)
    mask = torch.ones(N, device=DEV)
    ws, plan = _step_ws(N, d, V, _lib.BF16, 0, lambda p: p[1] == 2)
    old = head_op.head_fwd(h, W, None, y, None, None, 1 / 0.7, 1.0, 1.0, False, False, False)[0][:, 0] + 0.01
    head_op.STEP_WORKSPACE_BYTES = ws
    try:
        out, lse, g, loss, gh, gw = head_op.head_step_grpo(h, W, None, y, None, None, 1 / 0.7, 1.0, 1.0, False,
                                                           False, False, old, None, adv, mask, *EPS, True, True)
    finally:
        head_op.STEP_WORKSPACE_BYTES = None
    lp, ent, gr, gwr = head_fp32(h, W.float(), y, 0.7, g=g)
    assert (out[:, 0] - lp).abs().max() <= 2e-3 and (out[:, 1] - ent).abs().max() <= 2e-3
    assert _rel(gh, gr) <= 1e-2 and _rel(gw, gwr) <= 1e-2, plan
    assert _rel(gh[plan[0]:], gr[plan[0]:]) <= 1e-2


def test_step_fp8_weights_to_hidden():
    """fp8 weights with per-row scales, backward to the hidden rows only (no grad_W for fp8): the row scales enter dz
    in the scaling kernel; against the two-call path and the oracle on the dequantised weights."""
    from octopus_amd.workloads import quantise_fp8_rows
    N, d, V = 1200, 512, 8192
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=94, wscale=3.0)
    Wq, scale = quantise_fp8_rows(W)
    W32 = Wq.float() * scale[:, None]
    lp0 = head_op.head_fwd(h.to(DEV), Wq.to(DEV), scale.to(DEV), y.to(DEV), None, None, 1.0, 1.0, 1.0, False, False,
                           False)[0]
    old = lp0[:, 0].cpu() + noise
    with pytest.raises(NotImplementedError):
        _run(h, Wq, y, scored, mask, adv, old, 1.0, w_scale=scale, need_w=True)
    idx, count, step, two = _run(h, Wq, y, scored, mask, adv, old, 1.0, w_scale=scale, need_w=False)
    _check(h, W32, y, scored, mask, adv, old, 1.0, (1.0, 1.0, False), step, two, False, 1e-2, 4e-3)


@pytest.mark.parametrize("passes", [1, 3])
def test_step_grad_h_alone_reads_a_staged_w_transpose(passes):
    """grad_h as the only gradient over 16,384 rows or more: the step stages W^T once per call and grad_h reads it
    K-contiguous (16-bit weights it could read as stored); in one pass and in three, against the two-call path and
    the oracle."""
    N, d, V = 20000, 256, 4096
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=97)
    ws = None
    if passes > 1:
        ws, _ = _step_ws(N, d, V, _lib.BF16, _lib.WS_NO_GRADW, lambda p: p[1] == passes)
    lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None, y.to(DEV), None, None, 1.0, 1.0, 1.0, False, False, False)[0]
    old = lp0[:, 0].cpu() + noise
    idx, count, step, two = _run(h, W, y, scored, mask, adv, old, 1.0, need_w=False, ws=ws)
    _check(h, W.float(), y, scored, mask, adv, old, 1.0, (1.0, 1.0, False), step, two, False, 1e-2, 4e-3)


def test_step_extreme_logits():
    """Every row's hidden vector is e_0, so logit j is W[j, 0]: a 600-nat peak in the last vocabulary tile against
    logits in [-50, 50] (the other tiles' exponentials scale to exact zeros; the rows not labelled with the peak lie
    far below their maximum and take the row-offset rescale), and logits near -1,000 at T 0.7 (each tile's maximum
    far from zero). The gradients against the two-call backward's, whose own agreement with the
    oracle at these logits is bounded in tests/test_gpu_head.py."""
    N, d, V = 300, 64, 1000
    h = torch.zeros(N, d, dtype=torch.bfloat16)
    h[:, 0] = 1.0
    gen = torch.Generator().manual_seed(95)
    base = torch.randint(-50, 51, (V,), generator=gen).to(torch.float32)
    y = torch.randint(0, V, (N,), generator=gen)
    y[::2] = 777
    scored = torch.ones(N, dtype=torch.bool)
    mask = torch.ones(N)
    adv = torch.randn(N, generator=gen)
    for T, col in ((1.0, base.clone().index_fill_(0, torch.tensor([777]), 600.0)), (0.7, base / 10 - 1000.0)):
        W = torch.zeros(V, d)
        W[:, 0] = col
        W = W.to(torch.bfloat16)
        lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None, y.to(DEV), None, None, 1.0 / T, 1.0, 1.0, False, False,
                               False)[0]
        old = lp0[:, 0].cpu() + 0.05 * torch.randn(N, generator=gen)
        idx, count, step, two = _run(h, W, y, scored, mask, adv, old, T)
        out_s, lse_s, g_s, loss_s, gh_s, gw_s = step
        out_t, lse_t, g_t, loss_t, gh_t, gw_t = two
        assert torch.equal(out_s, out_t) and torch.equal(g_s, g_t)
        assert torch.isfinite(gh_s).all() and torch.isfinite(gw_s).all()
        # grad_W has no cancellation: the step's dz against the backward's to their 16-bit rounding
        assert _rel(gw_s, gw_t) <= 4e-3, T
        # grad_h at logits near -1,000 is a sum of large cancelling terms (the weights share a -1,000 component): the
        # 16-bit rounding of dz dominates either way (2^-9 relative per element, about 0.7 of the result in the
        # two-call backward, tests/test_gpu_head.py); the step's rounding of its stored exponentials is of the same size
        gh_ref, _ = ohead.head_backward(h, W, y, T, g_s.cpu(), want_w=False)
        e_two = _rel(gh_t.cpu(), gh_ref)
        assert _rel(gh_s.cpu(), gh_ref) <= 1e-2 + 1.5 * e_two, (T, e_two)


@pytest.mark.parametrize("weights", ["bf16", "fp8"])
def test_step_rows_far_below_their_maximum_are_rescaled(weights):
    """bf16 operands store each row's exponentials relative to an offset 48 (base 2) above the row's label logit, so
    dz is one scale per row times the stored values; a row whose maximum lies more than 112 (base 2, 77.6 nats) above
    its label's logit is rescaled after the merge instead. At T 0.01 the logits spread over about +-100 nats: most
    rows, with random labels, take the rescale, and every third row, labelled with its own argmax, does not. Three
    passes with the device count inside the second; against the two-call route and the fp64 oracle."""
    from octopus_amd.workloads import quantise_fp8_rows
    N, d, V, T = 6000, 256, 5120, 0.01
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=98)
    sc, W32, code, flags, need_w = None, W.float(), _lib.BF16, 0, True
    if weights == "fp8":
        W, sc = quantise_fp8_rows(W)
        W32, code, flags, need_w = W.float() * sc[:, None], _lib.FP8E4M3, _lib.WS_NO_GRADW, False
    z = h.float() @ W32.T / T
    y[::3] = z.argmax(1)[::3]
    gap = (z.max(1).values - z.gather(1, y[:, None])[:, 0]) * 1.4426950408889634
    assert int((scored & (gap > 113)).sum()) > 500 and int((scored & (gap < 111)).sum()) > 500
    ws, plan = _step_ws(N, d, V, code, flags, lambda p: p[1] == 3)
    lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None if sc is None else sc.to(DEV), y.to(DEV), None, None, 1.0 / T,
                           1.0, 1.0, False, False, False)[0]
    old = lp0[:, 0].cpu() + noise
    idx, count, step, two = _run(h, W, y, scored, mask, adv, old, T, w_scale=sc, need_w=need_w, ws=ws)
    _check(h, W32, y, scored, mask, adv, old, T, (1.0, 1.0, False), step, two, need_w, 1e-2, 4e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_step_labels_outside_the_vocabulary_on_masked_rows(dtype):
    """A label outside [0, V) (here -1 and V) gives its row a logprob of NaN and no label entry; on a row the GRPO mask
    leaves out, g is 0. bf16 gives such a row the offset -inf, so it takes the rescale after the merge; either way its
    gradient rows must be exactly 0 and every other row's as the oracle's and the two-call route's."""
    N, d, V = 1500, 256, 5120
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, dtype, seed=99)
    bad = torch.zeros(N, dtype=torch.bool)
    bad[::7] = True
    y[bad] = torch.where(torch.arange(N)[bad] % 2 == 0, torch.tensor(-1), torch.tensor(V))
    mask[bad] = 0.0
    lp0 = head_op.head_fwd(h.to(DEV), W.to(DEV), None, y.to(DEV), None, None, 1.0, 1.0, 1.0, False, False, False)[0]
    old = lp0[:, 0].cpu() + noise
    idx, count, step, two = _run(h, W, y, scored, mask, adv, old, 1.0)
    out_s, lse_s, g_s, loss_s, gh_s, gw_s = step
    out_t, lse_t, g_t, loss_t, gh_t, gw_t = two
    sel = scored.nonzero()[:, 0]
    n = sel.numel()
    badc = bad[sel]
    assert int(badc.sum()) > 50 and torch.equal(g_s, g_t)
    assert torch.isnan(out_s[:, 0].cpu()[bad & scored]).all() and (g_s[:n].cpu()[badc] == 0).all()
    gh_s, gw_s = gh_s.cpu(), gw_s.cpu()
    assert torch.isfinite(gh_s).all() and torch.isfinite(gw_s).all()
    assert (gh_s[bad] == 0).all()
    good = sel[~badc]
    gh_ref, gw_ref = ohead.head_backward(h[good], W.float(), y[good], 1.0, g_s[:n].cpu()[~badc])
    assert _rel(gh_s[good], gh_ref) <= 1e-2 and _rel(gw_s, gw_ref) <= 1e-2
    assert _rel(gh_s, gh_t.cpu()) <= 4e-3 and _rel(gw_s, gw_t.cpu()) <= 4e-3


def test_step_grad_w_only():
    """grad_W without grad_h (the rows frozen): over two passes, against the two-call backward and the oracle."""
    N, d, V = 3000, 256, 5120
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=90)
    ws, plan = _step_ws(N, d, V, _lib.BF16, 0, lambda p: p[1] == 2)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    old = head_op.head_fwd(hd, Wd, None, yd, None, None, 1.0, 1.0, 1.0, False, False, False)[0][:, 0] + \
        noise.to(DEV)
    args = (hd, Wd, None, yd, idx, count, 1.0, 1.0, 1.0, False, True, True, old, None, adv.to(DEV), mask.to(DEV),
            *EPS)
    head_op.STEP_WORKSPACE_BYTES = ws
    try:
        out, lse, g, loss, gr, gw = head_op.head_step_grpo(*args, False, True)
    finally:
        head_op.STEP_WORKSPACE_BYTES = None
    assert gr.numel() == 0
    _, _, g2, _ = head_op.head_fwd_grpo(*args)
    _, gw2 = head_op.head_bwd(hd, Wd, None, yd, idx, count, lse, g2, 1.0, 1.0, 1.0, False, True, False, True)
    sel = scored.nonzero()[:, 0]
    _, gw_ref = ohead.head_backward(h[sel], W.float(), y[sel], 1.0, g[:sel.numel()].cpu())
    assert torch.equal(g, g2)
    assert _rel(gw.cpu(), gw_ref) <= 1e-2 and _rel(gw, gw2) <= 4e-3, plan


def test_step_with_no_scored_rows():
    N, d, V = 512, 64, 1024
    h, W, y, _, _, adv, noise = _batch(N, d, V, torch.bfloat16, seed=96)
    scored = torch.zeros(N, dtype=torch.bool)
    mask = torch.zeros(N)
    idx, count, step, two = _run(h, W, y, scored, mask, adv, noise, 1.0)
    out_s, lse_s, g_s, loss_s, gh_s, gw_s = step
    assert (out_s == 0).all() and loss_s.item() == 0.0
    assert (gh_s == 0).all() and (gw_s == 0).all()


def test_step_grad_w_accumulate_through_the_c_abi():
    """OCTO_GRADW_ACCUMULATE and fp32 gradient outputs through the C ABI, over two passes: grad_w += the step's
    grad_W; grad_h in fp32."""
    n, d, V, T = 3000, 256, 4096, 0.8
    h, W, y, _, _, adv, noise = _batch(n, d, V, torch.bfloat16, seed=97)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    old = (head_op.head_fwd(hd, Wd, None, yd, None, None, 1.0 / T, 1.0, 1.0, False, False, False)[0][:, 0].cpu()
           + noise).to(DEV)
    advd, maskd = adv.to(DEV), torch.ones(n, device=DEV)
    out = torch.zeros(n, 2, device=DEV)
    lse = torch.zeros(n, 2, device=DEV)
    g = torch.zeros(n, device=DEV)
    loss = torch.zeros((), device=DEV)
    tail = _lib.GrpoTail(P(old), None, P(advd), P(maskd), n, *EPS, P(g), P(loss))
    wsb, plan = _step_ws(n, d, V, _lib.BF16, 0, lambda p: p[1] == 2)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    gh = torch.empty(n, d, dtype=torch.float32, device=DEV)
    base = (torch.randn(V, d, generator=torch.Generator().manual_seed(98)) * 1e-3).to(torch.float32)
    gw = base.to(DEV).clone()
    _lib.call("octo_head_step_grpo", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None, P(yd),
              None, None, n, d, V, _lib.LSE_PAIR | _lib.GRADW_ACCUMULATE, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse),
              P(out), 2, ctypes.byref(tail), P(gh), d, _lib.F32, P(gw), _lib.F32, P(ws), ws.numel(), st)
    torch.cuda.synchronize()
    gh_ref, gw_ref = ohead.head_backward(h, W, y, T, g.cpu())
    assert _rel(gh.cpu(), gh_ref) <= 1e-2, plan
    assert _rel(gw.cpu() - base, gw_ref) <= 1e-2, plan
    # a workspace below the smallest plan is refused before anything is queued
    with pytest.raises(ValueError):
        _lib.call("octo_head_step_grpo", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None,
                  P(yd), None, None, n, d, V, _lib.LSE_PAIR, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse), P(out), 2,
                  ctypes.byref(tail), P(gh), d, _lib.F32, P(gw), _lib.F32, P(ws), 1 << 20, st)


def test_step_with_a_plain_lse_through_the_c_abi():
    """A C-ABI caller without OCTO_LSE_PAIR gets the natural-log lse per row; the row-offset dz scales and the rescale
    of rows far below their maximum then read the row state from it. At T 0.012 over two passes (about 2,200 of the
    3,000 rows rescaled),
    the outputs and g must equal the paired call's bit for bit, and the gradients match it to 1e-3 and the oracle
    to 1e-2."""
    n, d, V, T = 3000, 256, 4096, 0.012
    h, W, y, _, _, adv, noise = _batch(n, d, V, torch.bfloat16, seed=101)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    old = (head_op.head_fwd(hd, Wd, None, yd, None, None, 1.0 / T, 1.0, 1.0, False, False, False)[0][:, 0].cpu()
           + noise).to(DEV)
    advd, maskd = adv.to(DEV), torch.ones(n, device=DEV)
    wsb, plan = _step_ws(n, d, V, _lib.BF16, 0, lambda p: p[1] == 2)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    runs = []
    for flags, lse_cols in ((_lib.LSE_PAIR, 2), (0, 1)):
        out = torch.zeros(n, 2, device=DEV)
        lse = torch.zeros(n, lse_cols, device=DEV)
        g = torch.zeros(n, device=DEV)
        loss = torch.zeros((), device=DEV)
        tail = _lib.GrpoTail(P(old), None, P(advd), P(maskd), n, *EPS, P(g), P(loss))
        gh = torch.empty(n, d, dtype=torch.bfloat16, device=DEV)
        gw = torch.empty(V, d, dtype=torch.bfloat16, device=DEV)
        _lib.call("octo_head_step_grpo", P(hd), n, hd.stride(0), _lib.BF16, P(Wd), Wd.stride(0), _lib.BF16, None,
                  P(yd), None, None, n, d, V, flags, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse), P(out), 2,
                  ctypes.byref(tail), P(gh), d, _lib.BF16, P(gw), _lib.BF16, P(ws), ws.numel(), st)
        torch.cuda.synchronize()
        runs.append((out.cpu(), g.cpu(), gh.cpu(), gw.cpu()))
    (out_p, g_p, gh_p, gw_p), (out_l, g_l, gh_l, gw_l) = runs
    z = h.float() @ W.float().T / T
    gap = (z.max(1).values - z.gather(1, y[:, None])[:, 0]) * 1.4426950408889634
    assert int((gap > 113).sum()) > 1500 and int((gap < 111).sum()) > 500
    assert torch.equal(out_p, out_l) and torch.equal(g_p, g_l)
    assert _rel(gh_l, gh_p) <= 1e-3 and _rel(gw_l, gw_p) <= 1e-3
    gh_ref, gw_ref = ohead.head_backward(h, W.float(), y, T, g_l)
    assert _rel(gh_l, gh_ref) <= 1e-2 and _rel(gw_l, gw_ref) <= 1e-2, plan


def test_step_strided_rows_weight_and_grad_h_through_the_c_abi():
    """Hidden rows, weight and grad_h as strided views (row strides past d, bases offset into wider buffers) through
    the C ABI, over two passes: every output bitwise the contiguous call's (the same kernels and tile order, only the
    addressing differs), the loss to summation order."""
    n, d, V, T = 3000, 256, 4096, 0.8
    h, W, y, _, _, adv, noise = _batch(n, d, V, torch.bfloat16, seed=96)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    hw = torch.zeros(n, d + 64, dtype=torch.bfloat16, device=DEV)
    hw[:, 16:16 + d] = hd
    Ww = torch.zeros(V, d + 128, dtype=torch.bfloat16, device=DEV)
    Ww[:, 64:64 + d] = Wd
    hs, Ws = hw[:, 16:16 + d], Ww[:, 64:64 + d]
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    old = (head_op.head_fwd(hd, Wd, None, yd, None, None, 1.0 / T, 1.0, 1.0, False, False, False)[0][:, 0].cpu()
           + noise).to(DEV)
    advd, maskd = adv.to(DEV), torch.ones(n, device=DEV)
    wsb, plan = _step_ws(n, d, V, _lib.BF16, 0, lambda p: p[1] == 2)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)

    def call(hx, Wx, gh, ld_gh):
        out, lse, g = torch.zeros(n, 2, device=DEV), torch.zeros(n, 2, device=DEV), torch.zeros(n, device=DEV)
        loss = torch.zeros((), device=DEV)
        gw = torch.zeros(V, d, dtype=torch.bfloat16, device=DEV)
        tail = _lib.GrpoTail(P(old), None, P(advd), P(maskd), n, *EPS, P(g), P(loss))
        _lib.call("octo_head_step_grpo", P(hx), n, hx.stride(0), _lib.BF16, P(Wx), Wx.stride(0), _lib.BF16, None,
                  P(yd), None, None, n, d, V, _lib.LSE_PAIR, 1.0 / T, 1.0, 1.0, 0, None, None, P(lse), P(out), 2,
                  ctypes.byref(tail), P(gh), ld_gh, _lib.BF16, P(gw), _lib.BF16, P(ws), ws.numel(), st)
        torch.cuda.synchronize()
        return out, lse, g, loss, gw

    gh0 = torch.zeros(n, d, dtype=torch.bfloat16, device=DEV)
    r0 = call(hd, Wd, gh0, d)
    ghw = torch.zeros(n, d + 32, dtype=torch.bfloat16, device=DEV)
    r1 = call(hs, Ws, ghw, d + 32)
    for a, b in zip(r0[:3] + r0[4:], r1[:3] + r1[4:]):
        assert torch.equal(a, b), plan
    assert abs(r0[3].item() - r1[3].item()) <= 1e-6 * max(1.0, abs(r0[3].item()))
    assert torch.equal(ghw[:, :d], gh0) and (ghw[:, d:] == 0).all()
    gh_ref, _ = ohead.head_backward(h, W, y, T, r0[2].cpu(), want_w=False)
    assert _rel(gh0.float().cpu(), gh_ref) <= 1e-2


def test_fused_grpo_head_autograd_matches_the_two_call_route():
    """fused_grpo_head under autograd: loss.backward() (here of 2 x loss) gives the gradients the step computed,
    scaled, and they match the autograd route of fused_head then grpo_loss (the trainer's two-call composition) to
    the 16-bit rounding of dz; the columns and the loss match that route's; under no_grad nothing is kept."""
    from octopus_amd.head_op import fused_grpo_head, fused_head
    N, d, V, T = 1800, 256, 4096, 0.9
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=99)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True)
    old = (fused_head(hd, Wd, yd, T, **kw)[:, 0] + noise.to(DEV)).detach()
    advd, maskd = adv.to(DEV), mask.to(DEV)

    h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    loss1, out1 = fused_grpo_head(h1, W1, yd, T, advd, maskd, prox=old, **kw)
    assert not out1.requires_grad and loss1.requires_grad
    (2.0 * loss1).backward()

    h2, W2 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    out2 = fused_head(h2, W2, yd, T, **kw)
    loss2, _ = head_op.grpo_loss(out2[:, 0], old, None, advd, maskd, *EPS)
    (2.0 * loss2).backward()
    torch.cuda.synchronize()
    assert torch.equal(out1, out2.detach())
    assert abs(loss1.item() - loss2.item()) <= 1e-5 * max(1.0, abs(loss2.item()))
    assert (h1.grad[~scored.to(DEV)] == 0).all()
    assert _rel(h1.grad, h2.grad) <= 4e-3 and _rel(W1.grad, W2.grad) <= 4e-3
    with torch.no_grad():
        loss3, out3 = fused_grpo_head(h1, W1, yd, T, advd, maskd, prox=old, **kw)
    assert torch.equal(out3, out1) and not loss3.requires_grad


def test_fused_grpo_head_rounds_a_scaled_gradient_once():
    """A loss scale that bf16 cannot hold (1/3, a micro-batch normalisation) scales the held bf16 gradients with one
    rounding: (loss / 3).backward() gives exactly the unscaled call's gradients times fp32(1/3), rounded once to bf16.
    Rounding the scale to bf16 first would bias every element by bf16(1/3) / (1/3) - 1 = +0.2%."""
    from octopus_amd.head_op import fused_grpo_head
    N, d, V, T = 1500, 256, 4096, 1.0
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=17)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True)
    old = (noise.to(DEV) - 8.0).detach()
    advd, maskd = adv.to(DEV), mask.to(DEV)
    grads = []
    for scale in (1.0, 1 / 3):
        h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
        loss, _ = fused_grpo_head(h1, W1, yd, T, advd, maskd, prox=None, old=old, **kw)
        (loss * scale).backward()
        grads.append((h1.grad, W1.grad))
    torch.cuda.synchronize()
    third = torch.tensor(1 / 3, dtype=torch.float32, device=DEV)
    for g1, g3 in zip(*grads):
        assert g3.dtype == torch.bfloat16 and g1.abs().max() > 0
        assert torch.equal(g3, (g1.float() * third).to(torch.bfloat16))


def test_autograd_routes_take_transposed_views():
    """Hidden rows and weight handed in as transposed views (dense, column-major): the ops read them through
    contiguous copies and allocate their gradients row-major, as the library writes them, so the gradients that reach
    the views' bases are the contiguous run's, bit for bit. fused_head (the recomputing backward) and
    fused_grpo_head (the fused step)."""
    from octopus_amd.head_op import fused_grpo_head, fused_head
    N, d, V, T = 1200, 256, 4096, 0.8
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=23)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True)
    advd, maskd, old = adv.to(DEV), mask.to(DEV), (noise.to(DEV) - 8.0)
    wout = torch.randn(N, device=DEV)

    def run(route, transposed):
        hb = (hd.t().contiguous() if transposed else hd.clone()).requires_grad_(True)
        Wb = (Wd.t().contiguous() if transposed else Wd.clone()).requires_grad_(True)
        h1, W1 = (hb.t(), Wb.t()) if transposed else (hb, Wb)
        if transposed:
            assert not h1.is_contiguous() and not W1.is_contiguous()
        if route == "two-call":
            (fused_head(h1, W1, yd, T, **kw)[:, 0] * wout).sum().backward()
        else:
            fused_grpo_head(h1, W1, yd, T, advd, maskd, prox=None, old=old, **kw)[0].backward()
        gh, gw = hb.grad, Wb.grad
        return (gh.t(), gw.t()) if transposed else (gh, gw)

    for route in ("two-call", "step"):
        base, views = run(route, False), run(route, True)
        torch.cuda.synchronize()
        for a, b in zip(base, views):
            assert a.abs().max() > 0 and torch.equal(a, b), route


def _tree_batch(seed, n_seq=5, prefix=600, V=4096, d=256):
    """A packed prefix tree (sequences sharing a prefix, random continuations), its per-flat-token GRPO inputs."""
    from octopus_amd.rl.prefix_tree import build_tree
    rng = np.random.default_rng(seed)
    pre = rng.integers(0, V, prefix)
    seqs = [np.concatenate([pre, rng.integers(0, V, int(k))]) for k in rng.integers(100, 900, n_seq)]
    cu = np.concatenate([[0], np.cumsum([len(s) for s in seqs])])
    flat = np.concatenate(seqs)
    scored = rng.random(len(flat)) < 0.7
    tree = build_tree(flat, cu, scored=scored)
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(len(tree.tokens), d, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    W = (torch.randn(V, d, generator=g) * 0.02).to(torch.bfloat16)
    seq_of = np.repeat(np.arange(n_seq), np.diff(cu))
    adv = torch.from_numpy(rng.standard_normal(n_seq)[seq_of]).float()
    mask = torch.from_numpy((scored & (rng.random(len(flat)) < 0.9)).astype(np.float32))
    return flat, cu, scored, tree, h, W, adv, mask


@pytest.mark.parametrize("device_pairs,passes,T", [
    (False, 1, 0.8), (False, 3, 0.8), (True, 1, 0.8), (True, 3, 0.8), (True, 3, 0.012), (False, 1, 0.012),
], ids=["host_pairs-1", "host_pairs-3", "device_pairs-1", "device_pairs-3", "device_pairs-3-rescaled",
        "host_pairs-1-rescaled"])
def test_tree_step_matches_the_two_call_tree_route_and_oracle(device_pairs, passes, T):
    """fused_grpo_tree_head over a prefix tree's pair rows: each flat token's columns bitwise the two-call tree route's
    (tree_head_output over the bound head), the loss to summation order, the gradients of hidden (pair rows summed
    into tree positions) and W against that route's autograd (fused_head, pairs_expand, grpo_loss, backward) and
    against the fp64 oracle with each pair row's g the sum of its flat tokens' GRPO weights (oracle/grpo.py);
    pairs built on the host (no-pair as the appended row P) and on the device (P on the device, no-pair -1), in one
    pass and in three. At T 0.012 most pair rows lie far below their maximum and take the row-offset rescale, whose
    dz scales use the g the flat tokens sum into each pair row after the merge."""
    from octopus_amd.head_op import fused_grpo_tree_head, fused_head
    from octopus_amd.rl.prefix_tree import TreeMeta, tree_head_output
    flat, cu, scored, tree, h, W, adv, mask = _tree_batch(101)
    if T < 0.1:
        rows = h[torch.from_numpy(tree.pair_pos)].float()
        z = rows @ W.float().T / T
        lab = torch.from_numpy(tree.pair_label)
        gap = (z.max(1).values - z.gather(1, lab[:, None])[:, 0]) * 1.4426950408889634
        assert int((gap > 113).sum()) > 100 and int((gap < 111).sum()) > 20
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    meta = (TreeMeta.on_device(t(flat), t(np.asarray(cu)), t(tree.flat_to_tree), len(tree.tokens), t(scored))
            if device_pairs else TreeMeta(tree, DEV))
    P = len(tree.pair_pos)
    ws = None
    if passes > 1:
        n_max = meta.pair_pos.numel()
        ws, plan = _step_ws(n_max, h.shape[1], W.shape[0], _lib.BF16, 0, lambda p: p[1] == passes)
    Wd0 = W.to(DEV)

    def route(hd, Wd):
        def chunk(rows, labels):
            return fused_head(rows, Wd, labels, T)
        chunk.octopus_fused_rows = lambda h2, pos, y, count=None: fused_head(h2, Wd, y, T, idx=pos, count=count)
        return tree_head_output(chunk, hd, meta)

    out0 = route(h.to(DEV)[None], Wd0)
    prox = (out0[0, :, 0] + 0.05 * torch.randn(len(flat), generator=torch.Generator().manual_seed(3)).to(DEV))
    prox = prox.detach()
    advd, maskd = adv.to(DEV), mask.to(DEV)

    h1, W1 = h.to(DEV)[None].requires_grad_(True), Wd0.clone().requires_grad_(True)
    head_op.STEP_WORKSPACE_BYTES = ws
    try:
        loss1, out1 = fused_grpo_tree_head(h1, W1, meta, T, advd, maskd, prox=prox)
    finally:
        head_op.STEP_WORKSPACE_BYTES = None
    loss1.backward()
    h2, W2 = h.to(DEV)[None].requires_grad_(True), Wd0.clone().requires_grad_(True)
    out2 = route(h2, W2)
    loss2, _ = head_op.grpo_loss(out2[0, :, 0], prox, None, advd, maskd, *EPS)
    loss2.backward()
    torch.cuda.synchronize()
    assert torch.equal(out1, out2.detach())
    assert abs(loss1.item() - loss2.item()) <= 1e-5 * max(1.0, abs(loss2.item()))
    assert _rel(h1.grad, h2.grad) <= 4e-3 and _rel(W1.grad, W2.grad) <= 4e-3
    # the oracle: g per pair row = the sum of its flat tokens' weights, the gradients of the pair rows scattered
    lp_flat = out1[0, :, 0].cpu().double().numpy()
    _, g_flat = ogrpo.grpo(lp_flat, adv.numpy(), mask.numpy(), prox=prox.double().cpu().numpy())
    fp = tree.flat_pair
    g_pair = np.zeros(P)
    np.add.at(g_pair, fp[fp >= 0], g_flat[fp >= 0])
    rows = h[torch.from_numpy(tree.pair_pos)]
    gh_pairs, gw_ref = ohead.head_backward(rows, W.float(), torch.from_numpy(tree.pair_label), T,
                                           torch.from_numpy(g_pair))
    gh_ref = torch.zeros(len(tree.tokens), h.shape[1], dtype=torch.float64)
    gh_ref.index_add_(0, torch.from_numpy(tree.pair_pos), gh_pairs)
    assert _rel(h1.grad[0].cpu(), gh_ref) <= 1e-2 and _rel(W1.grad.cpu(), gw_ref) <= 1e-2


def test_step_hidden_of_more_than_2_gib_through_idx():
    """The fused step over a 2.2 GB bf16 hidden matrix read through the compaction (its compact rows gathered into the
    workspace first, OCTO_WS_GATHER): 70,000 scored rows of 270,000 in passes of the step's plan, against the chunked
    fp32 reference with the step's own GRPO weight."""
    from octopus_amd.head_op import fused_grpo_head
    from tests.gpu_reference import head_fp32
    rows_total, d, V = 270_000, 4096, 1000
    gen = torch.Generator(device=DEV).manual_seed(52)
    h = torch.randn(rows_total, d, device=DEV, generator=gen)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    W = (torch.randn(V, d, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, V, (rows_total,), device=DEV, generator=gen)
    scored = torch.zeros(rows_total, dtype=torch.bool, device=DEV)
    scored[torch.randperm(rows_total, device=DEV, generator=gen)[:70_000]] = True
    adv = torch.randn(rows_total, device=DEV, generator=gen)
    prox = -7.0 + 0.1 * torch.randn(rows_total, device=DEV, generator=gen)
    idx, count = head_op.compact_rows(scored)
    assert h.numel() * 2 >= 1 << 31 and head_op._gather_flag(h, idx) == _lib.WS_GATHER
    a, b = h.requires_grad_(True), W.clone().requires_grad_(True)
    loss, out = fused_grpo_head(a, b, y, 1.0, adv, scored.float(), prox=prox, idx=idx, count=count,
                                labels_via_idx=True, scatter=True)
    loss.backward()
    n = int(count.item())
    sel = idx[:n]
    _, g_flat = ogrpo.grpo(out[:, 0].double().cpu().numpy(), adv.double().cpu().numpy(), scored.cpu().numpy(),
                           prox=prox.double().cpu().numpy())
    g = torch.from_numpy(g_flat).float().to(DEV)[sel]
    lp, ent, gr, gw = head_fp32(h.detach()[sel], W.float(), y[sel], 1.0, g=g)
    assert (out[sel, 0] - lp).abs().max().item() <= 2e-3 and (out[sel, 1] - ent).abs().max().item() <= 2e-3
    assert _rel(a.grad[sel], gr) <= 1e-2 and _rel(b.grad, gw) <= 1e-2
    assert (a.grad[~scored] == 0).all()
