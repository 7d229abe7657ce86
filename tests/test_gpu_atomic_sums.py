"""The two sums the library forms with fp32 atomics, whose order varies run to run: the GRPO loss scalar of
octo_head_fwd_grpo (one atomic add per 16-row workgroup of the merge, the rows of a workgroup summed in LDS in a fixed
order) and octo_pairs_grad (one atomic add per flat position into its pair row). Everything else of those calls is
deterministic and must repeat bit for bit; the sums must stay within the fp32 summation bound of an fp64 sum of the
same terms, (additions) x 2^-24 x sum |term|, on every run."""

import numpy as np
import pytest
import torch

from octopus_amd import head_op
from oracle import grpo as ogrpo

pytestmark = pytest.mark.gpu
DEV = "cuda"
U32 = 2.0 ** -24


def test_grpo_loss_scalar_varies_only_within_its_rounding_bound():
    N, d, V = 24576, 256, 4096
    gen = torch.Generator().manual_seed(101)
    h = torch.randn(N, d, generator=gen)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).to(DEV)
    W = (torch.randn(V, d, generator=gen) * 0.05).to(torch.bfloat16).to(DEV)
    y = torch.randint(0, V, (N,), generator=gen).to(DEV)
    scored = torch.rand(N, generator=gen) < 0.75
    mask = scored.float()
    adv = torch.randn(N, generator=gen)
    idx, count = head_op.compact_rows(scored.to(DEV))
    base, _ = head_op.head_fwd(h, W, None, y, idx, count, 1.0, 1.0, 1.0, False, True, True)
    old = (base[:, 0].cpu() + 0.05 * torch.randn(N, generator=gen)).to(DEV)
    runs = []
    for _ in range(6):
        out, lse, g, loss = head_op.head_fwd_grpo(h, W, None, y, idx, count, 1.0, 1.0, 1.0, False, True, True,
                                                  old, None, adv.to(DEV), mask.to(DEV), 0.2, 0.28, 5.0)
        torch.cuda.synchronize()
        runs.append((out.cpu(), lse.cpu(), g.cpu(), float(loss.item())))
    for out, lse, g, _ in runs[1:]:  # the GEMM, the merge and the per-row weights are deterministic
        assert torch.equal(out, runs[0][0]) and torch.equal(lse, runs[0][1]) and torch.equal(g, runs[0][2])
    lp = runs[0][0][:, 0].double().numpy()
    prox, A, m = old.double().cpu().numpy(), adv.double().numpy(), mask.numpy() != 0
    loss_ref, _ = ogrpo.grpo(lp, A, mask.numpy(), prox=prox)  # (old logp passed as the proximal logp)
    # the per-token terms in fp64 (no behaviour weight: old not given), |term| summed / Z: the bound's scale
    r = np.exp(lp - prox)
    terms = np.where(m, np.maximum(-A * r, -A * np.clip(r, 0.8, 1.28)), 0.0)
    scale = float(np.abs(terms).sum()) / max(1, int(m.sum()))
    additions = int(np.ceil(int(scored.sum()) / 16)) + 16  # one atomic add per 16-row workgroup, then 16 in LDS
    bound = additions * U32 * scale
    losses = [x[3] for x in runs]
    for loss in losses:
        assert abs(loss - loss_ref) <= bound, (loss, loss_ref, bound)
    assert max(losses) - min(losses) <= 2 * bound


def test_pairs_grad_atomic_sums_stay_within_their_rounding_bound():
    T, P, C = 200_000, 3_000, 2
    gen = torch.Generator().manual_seed(102)
    flat_pair = torch.randint(-1, P, (T,), generator=gen)  # many flat positions per pair; -1: none
    grad = torch.randn(T, C, generator=gen)
    ref = torch.zeros(P + 1, C, dtype=torch.float64).index_add_(0, flat_pair.clamp(min=-1) % (P + 1),
                                                                grad.double())[:P]
    mult = torch.bincount(flat_pair[flat_pair >= 0], minlength=P).double()
    absum = torch.zeros(P, C, dtype=torch.float64).index_add_(0, flat_pair[flat_pair >= 0],
                                                             grad[flat_pair >= 0].abs().double())
    bound = (mult[:, None] * U32 * absum).clamp(min=1e-30)
    for _ in range(3):
        gp = head_op.pairs_grad(grad.to(DEV), flat_pair.to(DEV), P).cpu().double()
        assert ((gp - ref).abs() <= bound).all()
