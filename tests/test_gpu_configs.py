"""The five measured configurations at full size on the GPU.

Each runs the trainer's own route (compaction of the scored rows, fused forward written in place, GRPO
weight, fused backward through autograd) and is checked
  - against the fp64 oracle on a seeded subsample of scored rows (logprob / entropy),
  - against a chunked fp32 torch reference on the GPU over every row (outputs and gradients),
  - for size-independent properties: unscored rows exactly 0, grad rows of unscored positions exactly 0,
    compaction equal to torch.nonzero.
Bars: fp32 1e-5 abs; bf16 2e-3 abs (logprob, entropy); gradients relative Frobenius 1e-2."""

import pytest
import torch

from octopus_amd import head_op
from octopus_amd.head_op import fused_head
from octopus_amd.workloads import CONFIGS, dequantised, make_batch
from oracle import grpo as ogrpo
from oracle import head as ohead
from tests.gpu_reference import head_fp32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _check_subsample(b, out, W64, k=48, seed=11):
    """Oracle (fp64, CPU) on k scored rows."""
    at = torch.nonzero(b.scored.cpu())[:, 0]
    pick = at[torch.randperm(at.numel(), generator=torch.Generator().manual_seed(seed))[:k]]
    lp, ent, _ = ohead.head_forward(b.hidden[pick.to(DEV)].cpu(), W64, b.labels[pick.to(DEV)].cpu(),
                                    b.cfg.temperature)
    o = out[pick.to(DEV)].cpu().double()
    return (o[:, 0] - lp).abs().max().item(), (o[:, 1] - ent).abs().max().item()


@pytest.mark.parametrize("name", ["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"])
def test_configuration(name):
    cfg = CONFIGS[name]
    b = make_batch(cfg, DEV)
    torch.cuda.synchronize()
    tol = 1e-5 if cfg.dtype == torch.float32 else 2e-3
    idx, count = head_op.compact_rows(b.scored)
    ref_idx = torch.nonzero(b.scored)[:, 0]
    n = ref_idx.numel()
    assert int(count.item()) == n and torch.equal(idx[:n], ref_idx)

    need_rows = cfg.backward != "none"
    need_w = cfg.backward == "full"
    h = b.hidden.detach().requires_grad_(need_rows)
    W = b.weight.detach().requires_grad_(need_w)
    out = fused_head(h, W, b.labels, cfg.temperature, idx=idx, count=count, labels_via_idx=True, scatter=True,
                     w_scale=b.w_scale)
    assert (out[~b.scored] == 0).all()

    W32 = dequantised(b)  # fp32 weights the kernel stands for (bf16 values, or e4m3 * row scale)
    rows = b.hidden[ref_idx]
    g = None
    if need_rows:
        old = (out[:, 0].detach() + b.old_noise)
        loss, g_flat = head_op.grpo_loss(out[:, 0], old, None, b.adv, b.scored.float(), 0.2, 0.28, 5.0)
        loss.backward()
        g = g_flat[ref_idx]
        # the GRPO weight against its oracle on the same logprobs
        _, g_ref = ogrpo.grpo(out[:, 0].detach().double().cpu().numpy(), b.adv.double().cpu().numpy(),
                              b.scored.cpu().numpy(), prox=old.double().cpu().numpy())
        assert (g_flat.double().cpu() - torch.from_numpy(g_ref)).abs().max() < 1e-7
    lp_r, ent_r, gr_r, gw_r = head_fp32(rows, W32, b.labels[ref_idx], cfg.temperature, g=g, want_w=need_w)
    assert (out[ref_idx, 0] - lp_r).abs().max() <= tol
    assert (out[ref_idx, 1] - ent_r).abs().max() <= tol
    e_lp, e_ent = _check_subsample(b, out.detach(), W32.double().cpu())
    assert e_lp <= tol and e_ent <= tol, (e_lp, e_ent)
    if need_rows:
        assert (h.grad[~b.scored] == 0).all()
        assert _rel(h.grad[ref_idx].float(), gr_r) <= 1e-2
    if need_w:
        assert _rel(W.grad.float(), gw_r) <= 1e-2


@pytest.mark.parametrize("name", ["cfg3", "cfg4", "cfg5"])
def test_configuration_fused_step(name):
    """The fused GRPO step (`fused_grpo_head`, what bench.py times) at full size: its columns bitwise the two-call
    forward's, its GRPO weight against the oracle on those logprobs, and its gradients (loss.backward()) against the
    chunked fp32 reference for that weight over every scored row, plus the size-independent properties."""
    from octopus_amd.head_op import fused_grpo_head
    cfg = CONFIGS[name]
    b = make_batch(cfg, DEV)
    idx, count = head_op.compact_rows(b.scored)
    ref_idx = torch.nonzero(b.scored)[:, 0]
    kw = dict(idx=idx, count=count, labels_via_idx=True, scatter=True, w_scale=b.w_scale)
    out0 = fused_head(b.hidden, b.weight, b.labels, cfg.temperature, **kw)
    old = (out0[:, 0] + b.old_noise).detach()
    need_w = cfg.backward == "full"
    h = b.hidden.detach().requires_grad_(True)
    W = b.weight.detach().requires_grad_(need_w)
    loss, out = fused_grpo_head(h, W, b.labels, cfg.temperature, b.adv, b.scored.float(), prox=old, **kw)
    loss.backward()
    torch.cuda.synchronize()
    assert torch.equal(out, out0.detach())
    lo, g_ref = ogrpo.grpo(out[:, 0].double().cpu().numpy(), b.adv.double().cpu().numpy(), b.scored.cpu().numpy(),
                           prox=old.double().cpu().numpy())
    assert abs(loss.item() - lo) <= 1e-5 * max(1.0, abs(lo))
    g = torch.from_numpy(g_ref).float().to(DEV)[ref_idx]
    _, _, gr_r, gw_r = head_fp32(b.hidden[ref_idx], dequantised(b), b.labels[ref_idx], cfg.temperature, g=g,
                                 want_w=need_w)
    assert (h.grad[~b.scored] == 0).all()
    assert _rel(h.grad[ref_idx].float(), gr_r) <= 1e-2
    if need_w:
        assert _rel(W.grad.float(), gw_r) <= 1e-2


@pytest.mark.parametrize("name,device_pairs", [("cfg3", True), ("cfg5", False)])
def test_configuration_fused_tree_step(name, device_pairs):
    """The fused GRPO step over the prefix tree's (position, label) pair rows (`fused_grpo_tree_head`) at full size:
    the root-plus-branches workload flattened into its sequences (root unscored, branches scored, a tenth of the
    scored tokens masked out of the loss), the tree's hidden rows as the configuration's. Each flat token's columns
    bitwise the two-call tree route's (tree_head_output over the bound head), the loss against grpo_loss on them,
    the gradients against that route's autograd and against the chunked fp32 reference on the pair rows with each
    pair row's g the sum of its flat tokens' oracle GRPO weights (oracle/grpo.py), scattered into tree positions;
    a subsample of pair rows' logprobs against the fp64 oracle. Pairs built on the device (cfg3) and the host
    (cfg5)."""
    import numpy as np
    from octopus_amd.head_op import fused_grpo_tree_head
    from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
    cfg = CONFIGS[name]
    b = make_batch(cfg, DEV)
    root, branches = cfg.segments[0], cfg.segments[1:]
    rng = np.random.default_rng(7)
    r_tok = rng.integers(0, cfg.V, root[0])
    seqs = [np.concatenate([r_tok, rng.integers(0, cfg.V, n)]) for n, _, _ in branches]
    flat = np.concatenate(seqs).astype(np.int64)
    cu = np.array([0, *np.cumsum([len(x) for x in seqs])], dtype=np.int64)
    scored = np.ones(len(flat), dtype=bool)
    for a in cu[:-1]:
        scored[a:a + root[0]] = False
    tree = build_tree(flat, cu, scored=scored)
    assert len(tree.tokens) == cfg.N
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    meta = (TreeMeta.on_device(t(flat), t(cu), t(tree.flat_to_tree), len(tree.tokens), t(scored))
            if device_pairs else TreeMeta(tree, DEV))
    seq_of = np.repeat(np.arange(len(seqs)), np.diff(cu))
    adv = t(rng.standard_normal(len(seqs))[seq_of].astype(np.float32))
    mask = t((scored & (rng.random(len(flat)) < 0.9)).astype(np.float32))
    T, ws = cfg.temperature, b.w_scale
    need_w = cfg.backward == "full"

    def route(hd, Wd):
        def chunk(rows, labels):
            return fused_head(rows, Wd, labels, T, w_scale=ws)
        chunk.octopus_fused_rows = lambda h2, pos, y, count=None: fused_head(h2, Wd, y, T, idx=pos, count=count,
                                                                            w_scale=ws)
        return tree_head_output(chunk, hd, meta)

    out0 = route(b.hidden[None], b.weight)
    prox = (out0[0, :, 0] + b.old_noise[:1].new_tensor(rng.standard_normal(len(flat)) * 0.01)).detach()
    h1 = b.hidden.detach()[None].requires_grad_(True)
    W1 = b.weight.detach().clone().requires_grad_(need_w)
    loss1, out1 = fused_grpo_tree_head(h1, W1, meta, T, adv, mask, prox=prox, w_scale=ws)
    loss1.backward()
    h2 = b.hidden.detach()[None].requires_grad_(True)
    W2 = b.weight.detach().clone().requires_grad_(need_w)
    out2 = route(h2, W2)
    loss2, _ = head_op.grpo_loss(out2[0, :, 0], prox, None, adv, mask, 0.2, 0.28, 5.0)
    loss2.backward()
    torch.cuda.synchronize()
    assert torch.equal(out1, out2.detach())
    assert abs(loss1.item() - loss2.item()) <= 1e-5 * max(1.0, abs(loss2.item()))
    assert _rel(h1.grad, h2.grad) <= 4e-3
    if need_w:
        assert _rel(W1.grad.float(), W2.grad.float()) <= 4e-3

    # the fp32 reference on the pair rows, g per pair row from the oracle's per-flat-token weights
    lp = out1[0, :, 0].double().cpu().numpy()
    lo, g_flat = ogrpo.grpo(lp, adv.double().cpu().numpy(), mask.cpu().numpy(), prox=prox.double().cpu().numpy())
    assert abs(loss1.item() - lo) <= 1e-5 * max(1.0, abs(lo))
    fp = tree.flat_pair
    P = len(tree.pair_pos)
    g_pair = np.zeros(P)
    np.add.at(g_pair, fp[fp >= 0], g_flat[fp >= 0])
    pos = torch.from_numpy(tree.pair_pos).to(DEV)
    labels = torch.from_numpy(tree.pair_label).to(DEV)
    W32 = dequantised(b)
    _, _, gr_p, gw_r = head_fp32(b.hidden[pos], W32, labels, T, g=torch.from_numpy(g_pair).float().to(DEV),
                                 want_w=need_w)
    gr_r = torch.zeros(cfg.N, cfg.d, device=DEV).index_add_(0, pos, gr_p)
    assert _rel(h1.grad[0].float(), gr_r) <= 1e-2
    if need_w:
        assert _rel(W1.grad.float(), gw_r) <= 1e-2
    # fp64 oracle on a seeded subsample of pair rows, read at a flat token of each
    pick = np.random.default_rng(11).choice(P, 32, replace=False)
    at = np.full(P, -1)
    where = np.nonzero(fp >= 0)[0]
    at[fp[where]] = where  # a flat token of each pair row (all of a pair's tokens carry its columns)
    lp_o, ent_o, _ = ohead.head_forward(b.hidden[pos[pick]].cpu(), W32.double().cpu(), labels[pick].cpu(), T)
    o = out1[0, torch.from_numpy(at[pick]).to(DEV)].cpu().double()
    assert (o[:, 0] - lp_o).abs().max().item() <= 2e-3 and (o[:, 1] - ent_o).abs().max().item() <= 2e-3
