"""The bound GRPO route: the reference's unchanged call path (bind_head, then AReaL's loss on the head's columns and
loss.backward(); actor.py:166-171, 343-347) reaching the fused step.

bind_head's pre-hook binds the micro-batch's GRPO inputs; the head's forward then runs octo_head_step_grpo (or its
pair-row form), whose columns equal the plain forward's, and the backward fits the incoming dL/dlogprob as c times
the step's own GRPO weight: the held gradients scaled by c, plus the recompute backward of the rest, whose kernels
end at once when the rest is negligible. Checked here: the gradients against the two-call route (fused_head, the
loss, backward) to the 16-bit rounding of dz (4e-3 relative) and against the fp64 oracle (1e-2), for the objective
alone (times 1 and 1/3), for the objective plus another term on the logprob column (the rest then runs), over compact
rows and over a prefix tree's pair rows, and through a bound model; with the objective alone the recompute's dz
GEMM launches end at once (the library's timing hook)."""

import numpy as np
import pytest
import torch

from octopus_amd import _lib, head_op
from oracle import grpo as ogrpo
from oracle import head as ohead
from tests.test_gpu_step import EPS, _batch, _rel, _tree_batch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _flat_case(N=1800, d=256, V=4096, seed=7, T=0.9):
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, torch.bfloat16, seed=seed)
    hd, Wd, yd = h.to(DEV), W.to(DEV), y.to(DEV)
    idx, count = head_op.compact_rows(scored.to(DEV))
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True)
    old = (head_op.fused_head(hd, Wd, yd, T, **kw)[:, 0] + noise.to(DEV)).detach()
    grpo = head_op.GrpoInputs(adv=adv.to(DEV), old=old, prox=None, mask=mask.to(DEV))
    return h, W, y, scored, mask, adv, hd, Wd, yd, idx, count, old, grpo, T


def _objective(logp, grpo, scale, extra):
    """The trainer's loss on the logprob column: scale x the GRPO objective (reuse_train_logp: no proximal logprobs),
    plus extra x the mean of mask x logp^2 (a term of another form)."""
    loss, _ = head_op.grpo_loss(logp, None, grpo.old, grpo.adv, grpo.mask, *EPS)
    loss = scale * loss
    if extra:
        loss = loss + extra * (grpo.mask * logp.float().pow(2)).sum() / logp.numel()
    return loss


@pytest.mark.parametrize("scale,extra", [(1.0, 0.0), (1 / 3, 0.0), (1.0, 0.3)],
                         ids=["objective", "objective-third", "objective-plus-term"])
def test_bound_route_over_compact_rows(scale, extra):
    h, W, y, scored, mask, adv, hd, Wd, yd, idx, count, old, grpo, T = _flat_case()
    h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    out1 = head_op.grpo_bound_head(h1, W1, yd, T, grpo, idx=idx, count=count)
    _objective(out1[:, 0], grpo, scale, extra).backward()
    h2, W2 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    out2 = head_op.fused_head(h2, W2, yd, T, idx=idx, count=count, labels_via_idx=True, scatter=True)
    _objective(out2[:, 0], grpo, scale, extra).backward()
    torch.cuda.synchronize()
    assert torch.equal(out1.detach(), out2.detach())
    assert (h1.grad[~scored.to(DEV)] == 0).all()
    assert _rel(h1.grad, h2.grad) <= 4e-3 and _rel(W1.grad, W2.grad) <= 4e-3
    # the fp64 oracle: dL/dlogp of the same loss on the same logprobs, then the head's backward
    lp = out1[:, 0].detach().cpu().double().numpy()
    _, g = ogrpo.grpo(lp, adv.numpy(), mask.numpy(), old=old.cpu().double().numpy())
    g = scale * g + extra * 2.0 * mask.numpy() * lp / len(lp)
    at = np.flatnonzero(scored.numpy())
    gh, gw = ohead.head_backward(h[at], W.float(), y[at], T, torch.from_numpy(g[at]))
    gh_full = torch.zeros(h.shape, dtype=torch.float64)
    gh_full[at] = gh
    assert _rel(h1.grad.cpu(), gh_full) <= 1e-2 and _rel(W1.grad.cpu(), gw) <= 1e-2


def _dz_ms(fn):
    """Milliseconds of the gemm_dz launches queued by fn() (the library's timing hook)."""
    _lib.call("octo_timing_enable", 1)
    fn()
    torch.cuda.synchronize()
    launches, total = _lib.timing_read("gemm_dz")
    _lib.call("octo_timing_enable", 0)
    return launches, total


def test_bound_route_skips_the_recompute_for_the_objective():
    """With the objective as the loss (times 2), the residual backward's dz GEMMs end at once: their launches take a
    small fraction of the two-call route's, whose backward recomputes the logits. With another term in the loss they
    run in full."""
    h, W, y, scored, mask, adv, hd, Wd, yd, idx, count, old, grpo, T = _flat_case(N=6144, d=1024, V=32768, seed=11)
    times = {}
    for name, extra in (("objective", 0.0), ("plus-term", 0.3)):
        h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
        out1 = head_op.grpo_bound_head(h1, W1, yd, T, grpo, idx=idx, count=count)
        loss = _objective(out1[:, 0], grpo, 2.0, extra)
        times[name] = _dz_ms(loss.backward)
    h2, W2 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    out2 = head_op.fused_head(h2, W2, yd, T, idx=idx, count=count, labels_via_idx=True, scatter=True)
    loss2 = _objective(out2[:, 0], grpo, 2.0, 0.0)
    times["two-call"] = _dz_ms(loss2.backward)
    n_two, ms_two = times["two-call"]
    n_obj, ms_obj = times["objective"]
    n_term, ms_term = times["plus-term"]
    assert n_two > 0 and n_obj == n_two and n_term == n_two
    assert ms_obj < 0.2 * ms_two, times
    assert ms_term > 0.5 * ms_two, times


@pytest.mark.parametrize("extra", [0.0, 0.3], ids=["objective", "objective-plus-term"])
def test_bound_route_over_tree_pair_rows(extra):
    """grpo_bound_tree_head (device-built pairs): the columns bitwise the plain tree route's (tree_head_output over
    the bound head), the gradients of hidden and W against that route's autograd."""
    from octopus_amd.rl.prefix_tree import TreeMeta, tree_head_output
    flat, cu, scored, tree, h, W, adv, mask = _tree_batch(202)
    T = 0.85
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    meta = TreeMeta.on_device(t(flat), t(np.asarray(cu)), t(tree.flat_to_tree), len(tree.tokens), t(scored))
    Wd0 = W.to(DEV)

    def route(hd, Wd):
        def chunk(rows, labels):
            return head_op.fused_head(rows, Wd, labels, T)
        chunk.octopus_fused_rows = lambda h2, pos, y, count=None: head_op.fused_head(h2, Wd, y, T, idx=pos,
                                                                                      count=count)
        return tree_head_output(chunk, hd, meta)

    old = (route(h.to(DEV)[None], Wd0)[0, :, 0]
           + 0.05 * torch.randn(len(flat), generator=torch.Generator().manual_seed(5)).to(DEV)).detach()
    grpo = head_op.GrpoInputs(adv=adv.to(DEV), old=old, prox=None, mask=mask.to(DEV))
    h1, W1 = h.to(DEV)[None].requires_grad_(True), Wd0.clone().requires_grad_(True)
    out1 = head_op.grpo_bound_tree_head(h1, W1, meta, T, grpo)
    _objective(out1[0, :, 0], grpo, 1.0, extra).backward()
    h2, W2 = h.to(DEV)[None].requires_grad_(True), Wd0.clone().requires_grad_(True)
    out2 = route(h2, W2)
    _objective(out2[0, :, 0], grpo, 1.0, extra).backward()
    torch.cuda.synchronize()
    assert torch.equal(out1.detach(), out2.detach())
    assert _rel(h1.grad, h2.grad) <= 4e-3 and _rel(W1.grad, W2.grad) <= 4e-3


@pytest.mark.parametrize("tree", [False, True], ids=["flat", "tree"])
def test_bound_model_takes_the_step_through_the_trainers_call_path(tree):
    """A bf16 Llama and a Qwen3.5 bound by bind_head, called as the actor calls them (input_ids with the micro-batch's
    advantages, behaviour logprobs and loss mask as kwargs; the scored positions or the prefix tree set on the head),
    then the GRPO objective on the head's logprob column and backward: every parameter's gradient as with the step
    switched off (head.octopus_grpo_step = False: the plain route), the head's weight to the 16-bit rounding of dz
    (4e-3) and the decoder's parameters to 2e-2 (their bf16 backward carries the head's difference in grad_hidden
    through its own roundings), the columns bitwise; under no_grad the plain route runs."""
    from transformers import AutoModelForCausalLM
    from octopus_amd.rl.lm_head import bind_head
    from octopus_amd.rl.prefix_tree import TreeMeta, build_tree
    from tests.tiny_models import families
    for name, config, _ in families():
        if name not in ("llama", "qwen3_5"):
            continue
        torch.manual_seed(21)
        model = AutoModelForCausalLM.from_config(config, attn_implementation="eager").to(DEV, torch.bfloat16)
        rng = np.random.default_rng(9)
        T_len = 40
        ids = torch.from_numpy(rng.integers(0, config.vocab_size, (1, T_len))).to(DEV)
        mask = torch.from_numpy((rng.random((1, T_len)) < 0.7).astype(np.float32)).to(DEV)
        adv = torch.from_numpy(rng.standard_normal((1, T_len)).astype(np.float32)).to(DEV)
        head = bind_head(model, 0.8)
        head.octopus_labels = ids[0].roll(-1)
        head.octopus_scored = mask[0].bool()
        head.octopus_tree = None
        with torch.no_grad():
            old = model(input_ids=ids).logits[0, :, 0].float() + 0.05
        batch = dict(input_ids=ids, advantages=adv, logprobs=old[None], loss_mask=mask)
        if tree:  # two sequences sharing a 12-token prefix, run on the tree's positions by their head rows
            flat = ids[0].cpu().numpy().copy()
            flat[20:32] = flat[0:12]
            ids = torch.from_numpy(flat[None]).to(DEV)
            t = build_tree(flat, np.array([0, 20, T_len]), scored=mask[0].bool().cpu().numpy())
            meta = TreeMeta(t, DEV)
            batch["input_ids"] = ids
        grads = []
        for step_on in (True, False):
            model.zero_grad(set_to_none=True)
            head.octopus_grpo_step = step_on
            if tree:  # the head on the tree's hidden rows, as the actor's tree forward calls it
                head.octopus_tree = meta
                tree_ids = torch.from_numpy(np.asarray(t.tokens)[None]).to(DEV)
                hidden = model.get_decoder()(input_ids=tree_ids).last_hidden_state
                head.octopus_grpo = head_op.GrpoInputs(adv=adv[0], old=old, prox=None, mask=mask[0])
                cols = head(hidden)
            else:
                cols = model(**batch).logits
                assert head.octopus_grpo is not None
            loss, _ = head_op.grpo_loss(cols[0, :, 0], None, old, adv[0], mask[0], *EPS)
            loss.backward()
            grads.append({n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None})
            grads[-1]["cols"] = cols.detach().clone()
        torch.cuda.synchronize()
        on, off = grads
        assert torch.equal(on.pop("cols"), off.pop("cols")), name
        assert on.keys() == off.keys() and len(on) > 3
        head_w = next(n for n, p in model.named_parameters() if p is head.weight)
        assert _rel(on[head_w], off[head_w]) <= 4e-3, name
        for k in on:  # the decoder's bf16 backward carries the head's 4e-3 difference in grad_hidden through its own
            if off[k].norm() > 0:  # roundings
                assert _rel(on[k], off[k]) <= 2e-2, (name, k)
        with torch.no_grad():
            head.octopus_grpo_step = True
            head.octopus_tree = None
            plain = model(**batch).logits if not tree else None
        if plain is not None:
            head.octopus_grpo_step = False
            with torch.no_grad():
                assert torch.equal(plain, model(**batch).logits)


def test_bound_route_refuses_a_second_backward():
    """The held gradients are scaled in place and handed to autograd by the backward, so a second backward through
    the same graph (retain_graph) raises rather than scaling them again."""
    h, W, y, scored, mask, adv, hd, Wd, yd, idx, count, old, grpo, T = _flat_case(N=600)
    h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(True)
    out = head_op.grpo_bound_head(h1, W1, yd, T, grpo, idx=idx, count=count)
    loss = _objective(out[:, 0], grpo, 1.0, 0.0)
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="runs once"):
        loss.backward()


def _fit_call(src, idx, h, count):
    n = h.numel()
    c = torch.full((1,), -7.0, device=DEV)
    rest = torch.full((n,), -7.0, device=DEV)
    cr = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    skip = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    _lib.call("octo_grpo_fit", P(src), src.stride(0), P(idx), P(h), n, P(count), head_op.SPEC_TOL, P(c), P(rest),
              P(cr), P(skip), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return c.item(), rest, cr.item(), skip.item()


def test_grpo_fit_through_the_c_abi():
    """octo_grpo_fit against the same arithmetic in torch: a gathered through idx up to the device count (0 past it),
    c the least-squares multiple of h, rest = a - c h, and the rest's row count 0 (skip 1) exactly when it is
    negligible; with h = 0, c = 0 and the whole of a is the rest; with no rows, nothing to fit."""
    g = torch.Generator(device=DEV).manual_seed(5)
    N, n = 5000, 3000
    src = torch.randn(N, 2, device=DEV, generator=g)
    idx = torch.randperm(N, device=DEV, generator=g)[:n].sort().values
    h = torch.randn(n, device=DEV, generator=g)
    count = torch.tensor([2500], dtype=torch.int32, device=DEV)
    a = torch.where(torch.arange(n, device=DEV) < 2500, src[idx, 0], torch.zeros((), device=DEV))
    h[2500:] = 0.0
    c, rest, cr, skip = _fit_call(src, idx, h, count)  # unrelated a: the rest is everything but its h component
    c_ref = (a @ h / (h @ h)).item()
    assert abs(c - c_ref) <= 1e-5 * abs(c_ref) + 1e-7
    assert torch.allclose(rest, a - c * h, atol=1e-6) and (cr, skip) == (2500, 0)
    src2 = torch.zeros(N, 2, device=DEV)
    src2[idx[:2500], 0] = h[:2500] / 3  # a = h / 3 (rounded): c = 1/3 and a negligible rest
    c, rest, cr, skip = _fit_call(src2, idx, h, count)
    assert abs(c - 1 / 3) <= 1e-6 and (cr, skip) == (0, 1)
    assert rest.abs().max().item() <= 1e-6 * h.abs().max().item()
    c, rest, cr, skip = _fit_call(src, None, torch.zeros(n, device=DEV), None)  # h = 0, no idx, no count
    assert c == 0.0 and torch.equal(rest, src[:n, 0]) and (cr, skip) == (n, 0)
    c, rest, cr, skip = _fit_call(src, None, torch.zeros(0, device=DEV), None)  # no rows
    assert c == 0.0 and (cr, skip) == (0, 1)



@pytest.mark.parametrize("form", ["f16-softcap", "fp8-weights"])
def test_bound_route_with_other_operand_forms(form):
    """The bound route beyond bf16: f16 operands with the tanh soft-cap (post-head transform in the epilogue), and fp8
    weights with row scales (grad_h only, as a frozen quantised head). The objective plus another term on the logprob
    column, so both the held gradients and the rest's backward run; the gradients against the two-call route
    (fused_head, the same loss, backward) to the 16-bit rounding of dz."""
    N, d, V, T = 1800, 256, 4096, 0.9
    dtype = torch.float16 if form == "f16-softcap" else torch.bfloat16
    h, W, y, scored, mask, adv, noise = _batch(N, d, V, dtype, seed=13)
    hd, yd = h.to(DEV), y.to(DEV)
    post, sc = head_op.Post(), None
    if form == "f16-softcap":
        post, Wd = head_op.Post(0.5, 2.0, True), W.to(DEV)
    else:
        Wd, sc = head_op.quantise_fp8_rows(W.to(DEV))
    idx, count = head_op.compact_rows(scored.to(DEV))
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True, w_scale=sc)
    with torch.no_grad():
        old = head_op.fused_head(hd, Wd, yd, T, post, **kw)[:, 0] + noise.to(DEV)
    grpo = head_op.GrpoInputs(adv=adv.to(DEV), old=old, prox=None, mask=mask.to(DEV))
    need_w = form == "f16-softcap"
    h1, W1 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(need_w)
    out1 = head_op.grpo_bound_head(h1, W1, yd, T, grpo, post=post, idx=idx, count=count, w_scale=sc)
    _objective(out1[:, 0], grpo, 1.0, 0.3).backward()
    h2, W2 = hd.clone().requires_grad_(True), Wd.clone().requires_grad_(need_w)
    out2 = head_op.fused_head(h2, W2, yd, T, post, **kw)
    _objective(out2[:, 0], grpo, 1.0, 0.3).backward()
    torch.cuda.synchronize()
    assert torch.equal(out1.detach(), out2.detach())
    assert (h1.grad[~scored.to(DEV)] == 0).all() and _rel(h1.grad, h2.grad) <= 4e-3
    if need_w:
        assert _rel(W1.grad, W2.grad) <= 4e-3
    else:
        assert W1.grad is None
