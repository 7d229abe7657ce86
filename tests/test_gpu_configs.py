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
