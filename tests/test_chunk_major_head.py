"""The head as chunk_major calls it (reference octopus/rl/chunk_major.py:321, 339-346, 350-363).

run_forward calls `head(hidden_rows[chunk pair rows], labels)` chunk by chunk under no_grad and writes each output into
`pairs[P + 1, C]`; run_backward folds the flat gradient into pair rows with index_add_, then recomputes the chunks in
reverse order with gradients on and back-propagates each chunk's rows. The head is
`functools.partial(_chunked_rows, head)` (actor.py:177) and reads `head.weight` at every call, so a weight swapped in
between forward and backward (FSDP's unsharded tensor) is the one used and the one that receives the gradient
(lm_head.py:116-117).

Checked: the chunked forward equals tree_head_output over the whole tree, and the reverse-chunk backward gives the
same hidden and weight gradients as one backward through it; and both against the fp64 oracle on the same inputs
(the pair rows' columns expanded by oracle.head.tree_output; the gradients of the loss whose dL/dlogprob per pair is
the folded flat gradient), at the path's bars. The HIP path on the GPU, the composite path on the CPU."""

import functools

import numpy as np
import pytest
import torch

from octopus_amd.rl.lm_head import _chunked_rows, bind_head
from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
from oracle import head as ohead

SMALL = dict(vocab_size=300, hidden_size=64, intermediate_size=64, num_hidden_layers=1, num_attention_heads=2,
             num_key_value_heads=1, head_dim=32)


def _tree(rng):
    prefix = rng.integers(0, 300, 120)
    seqs = [np.concatenate([prefix[:int(rng.integers(40, 121))], rng.integers(0, 300, int(k))])
            for k in rng.integers(5, 60, 7)]
    flat = np.concatenate(seqs)
    cu = [0, *np.cumsum([len(s) for s in seqs]).tolist()]
    return build_tree(flat, cu, scored=rng.random(len(flat)) < 0.7)


def _run(dev, dtype, tol_out, tol_grad):
    from transformers import AutoModelForCausalLM, LlamaConfig
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(LlamaConfig(**SMALL)).to(dev, dtype)
    head = bind_head(model, 0.8)
    head_fn = functools.partial(_chunked_rows, head)
    rng = np.random.default_rng(3)
    tree = _tree(rng)
    meta = TreeMeta(tree, dev)
    P = len(tree.pair_pos)
    hidden = torch.randn(1, len(tree.tokens), SMALL["hidden_size"], device=dev).to(dtype)
    gflat = torch.randn(1, len(tree.flat_pair), 2, device=dev)

    # whole tree, one autograd graph
    h_all = hidden.clone().requires_grad_(True)
    out_all = tree_head_output(head_fn, h_all, meta)
    (out_all.float() * gflat).sum().backward()
    gw_all, gh_all = head.weight.grad.clone(), h_all.grad.clone()
    head.weight.grad = None

    # chunk-major: pair rows split into uneven chunks
    cuts = sorted(set([0, P, *rng.integers(1, P, 3).tolist()]))
    chunks = [torch.arange(a, b, device=dev) for a, b in zip(cuts[:-1], cuts[1:])]
    h_cm = hidden.clone().requires_grad_(True)
    with torch.no_grad():
        pairs = None
        for rows in chunks:
            out = head_fn(h_cm[0].index_select(0, meta.pair_pos[rows]), meta.pair_label[rows])
            if pairs is None:
                pairs = out.new_zeros(P + 1, out.shape[1])
            pairs[rows] = out
        out_cm = pairs.index_select(0, meta.flat_pair)[None]
    assert (out_cm.float() - out_all.detach().float()).abs().max().item() <= tol_out

    # the unsharded weight is swapped in again before the backward pass
    old = head.weight
    head.weight = torch.nn.Parameter(old.detach().clone())
    grad_pairs = gflat.new_zeros(P + 1, 2).index_add_(0, meta.flat_pair, gflat[0])
    for rows in reversed(chunks):
        with torch.enable_grad():
            out = head_fn(h_cm[0].index_select(0, meta.pair_pos[rows]), meta.pair_label[rows])
            torch.autograd.backward([out], [grad_pairs.index_select(0, rows).to(out.dtype)])
    assert old.grad is None and head.weight.grad is not None

    def rel(a, b):
        return ((a.double() - b.double()).norm() / b.double().norm()).item()

    # each route against the fp64 oracle on the same inputs first, so that a failure names the route: the pair rows'
    # columns expanded to the flat positions, and the gradients of the loss whose dL/dlogprob per pair is
    # grad_pairs[:, 0] (the entropy column is detached), the hidden gradient folded back onto the tree rows the pairs
    # read (chunk_major.py:339-363)
    rows = hidden[0].index_select(0, meta.pair_pos).cpu()
    W = old.detach().cpu()
    labels = meta.pair_label.cpu()
    lp, ent, _ = ohead.head_forward(rows, W, labels, 0.8)
    want_out = ohead.tree_output(torch.stack([lp, ent], 1), meta.flat_pair.cpu())
    tol_oracle = 1e-5 if dtype == torch.float32 else 2e-3
    assert (out_all[0].detach().cpu().double() - want_out).abs().max().item() <= tol_oracle, "whole-tree columns"
    assert (out_cm[0].cpu().double() - want_out).abs().max().item() <= tol_oracle, "chunked columns"
    gh_pairs, gw_want = ohead.head_backward(rows, W, labels, 0.8, grad_pairs[:P, 0].cpu())
    gh_want = torch.zeros(hidden.shape[1], hidden.shape[2], dtype=torch.float64).index_add_(
        0, meta.pair_pos.cpu(), gh_pairs)
    bar = 1e-4 if dtype == torch.float32 else 1e-2
    assert rel(gh_all[0].cpu(), gh_want) <= bar and rel(gw_all.cpu(), gw_want) <= bar, "whole-tree gradients"
    assert rel(h_cm.grad[0].cpu(), gh_want) <= bar and rel(head.weight.grad.cpu(), gw_want) <= bar, \
        "chunked gradients"
    # then the two routes against each other, at the tighter bar of their shared arithmetic
    assert rel(head.weight.grad, gw_all) <= tol_grad
    assert rel(h_cm.grad, gh_all) <= tol_grad


def test_chunk_major_head_cpu():
    _run("cpu", torch.float32, 1e-5, 1e-5)  # chunking changes the CPU GEMM blocking: fp32 rounding only


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_chunk_major_head_hip(dtype):
    # bf16: each chunk's grad_W is rounded to bf16 before autograd sums the chunks (the reference's own
    # accumulation), against one fp32-summed grad_W over the whole tree
    _run("cuda", dtype, 1e-6 if dtype == torch.float32 else 2e-3, 1e-5 if dtype == torch.float32 else 1e-2)
