"""Pins the oracle (CPU) against things other than its own formulas: transformers' model logits with
torch.log_softmax, brute-force Python, closed-form cases, finite differences, torch autograd, torch.nonzero
and the reference's own hand-built prefix-tree cases (tests/test_prefix_tree.py:28-50, 165-188, 430-434)."""

import math

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import grpo as ogrpo
from oracle import head as ohead
from oracle import pairs as opairs
from tests.tiny_models import NAMES

F64 = torch.float64


def test_columns_match_brute_force_python():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(5, 7, generator=g, dtype=F64) * 3
    labels = torch.tensor([0, 6, 3, 3, 1])
    for T in (1.0, 0.7):
        lp, ent, lse = ohead.columns(logits, T, labels)
        for r in range(5):
            s = [x / T for x in logits[r].tolist()]
            L = math.log(math.fsum(math.exp(v) for v in s))
            p = [math.exp(v - L) for v in s]
            assert abs(lse[r].item() - L) < 1e-12
            assert abs(lp[r].item() - (s[labels[r]] - L)) < 1e-12
            assert abs(ent[r].item() + math.fsum(pi * math.log(pi) for pi in p)) < 1e-12


def test_columns_closed_forms():
    V = 1000
    lp, ent, lse = ohead.columns(torch.zeros(3, V, dtype=F64), 0.7, torch.tensor([0, 5, 999]))
    assert torch.allclose(lp, torch.full((3,), -math.log(V), dtype=F64), atol=1e-12)
    assert torch.allclose(ent, torch.full((3,), math.log(V), dtype=F64), atol=1e-12)
    peaked = torch.zeros(2, V, dtype=F64)
    peaked[0, 7] = peaked[1, 3] = 200.0
    lp, ent, _ = ohead.columns(peaked, 1.0, torch.tensor([7, 4]))
    assert abs(lp[0].item()) < 1e-60 and ent[0].item() < 1e-60
    assert abs(lp[1].item() + 200.0) < 1e-9  # a label that is not the peak


@pytest.mark.parametrize("k", range(len(NAMES)), ids=NAMES)
def test_head_forward_matches_the_models_own_logits(k):
    """The oracle on the lm_head input, with the family's post-head transform, gives the log-probability of each
    position's next token and the entropy of the model's own logits (the property of reference
    tests/test_lm_head.py:11-34), here against torch.distributions.Categorical in fp64 at T 1.0 and 0.7, to 1e-5."""
    from transformers import AutoModelForCausalLM
    from tests.tiny_models import families
    _, config, (pre, post, tanh) = families()[k]
    torch.manual_seed(20 + k)
    model = AutoModelForCausalLM.from_config(config, attn_implementation="eager")
    model.eval()
    ids = torch.randint(0, config.vocab_size, (1, 17), generator=torch.Generator().manual_seed(30 + k))
    nxt = ids[0].roll(-1)
    head_in = []
    handle = model.get_output_embeddings().register_forward_hook(lambda mod, inp, out: head_in.append(inp[0]))
    with torch.no_grad():
        own = model(input_ids=ids).logits[0].double()
    handle.remove()
    W = model.get_output_embeddings().weight.detach()
    for T in (1.0, 0.7):
        lp, ent, _ = ohead.head_forward(head_in[0][0], W, nxt, T, pre=pre, post=post, tanh=tanh)
        want = torch.distributions.Categorical(logits=own / T)
        assert (lp.double() - want.log_prob(nxt)).abs().max().item() <= 1e-5, T
        assert (ent.double() - want.entropy()).abs().max().item() <= 1e-5, T


@pytest.mark.parametrize("post", [dict(), dict(pre=0.5, post=2.0, tanh=True), dict(pre=0.25)])
def test_backward_matches_autograd(post):
    g = torch.Generator().manual_seed(1)
    n, d, V = 9, 6, 11
    h = torch.randn(n, d, generator=g, dtype=F64, requires_grad=True)
    W = torch.randn(V, d, generator=g, dtype=F64, requires_grad=True)
    y = torch.randint(0, V, (n,), generator=g)
    gl = torch.randn(n, generator=g, dtype=F64)
    T = 0.7
    z = h @ W.T
    zp = post["post"] * torch.tanh(post["pre"] * z) if post.get("tanh") else post.get("pre", 1.0) * z
    logp = torch.log_softmax(zp / T, -1).gather(1, y[:, None])[:, 0]
    (logp * gl).sum().backward()
    gh, gw = ohead.head_backward(h.detach(), W.detach(), y, T, gl, **post)
    assert torch.allclose(gh, h.grad, atol=1e-12) and torch.allclose(gw, W.grad, atol=1e-12)


def test_backward_matches_finite_differences():
    g = torch.Generator().manual_seed(2)
    n, d, V = 3, 4, 5
    h = torch.randn(n, d, generator=g, dtype=F64)
    W = torch.randn(V, d, generator=g, dtype=F64)
    y = torch.tensor([4, 0, 2])
    gl = torch.tensor([0.3, -1.2, 0.8], dtype=F64)
    T, eps = 0.9, 1e-6

    def loss(hh, WW):
        return (ohead.head_forward(hh, WW, y, T, pre=0.5, post=2.0, tanh=True)[0] * gl).sum().item()

    gh, gw = ohead.head_backward(h, W, y, T, gl, pre=0.5, post=2.0, tanh=True)
    for X, G in ((h, gh), (W, gw)):
        for idx in np.ndindex(*X.shape):
            Xp, Xm = X.clone(), X.clone()
            Xp[idx] += eps
            Xm[idx] -= eps
            num = (loss(Xp, W) - loss(Xm, W)) / (2 * eps) if X is h else (loss(h, Xp) - loss(h, Xm)) / (2 * eps)
            assert abs(num - G[idx].item()) < 1e-7


def test_scored_rows_are_the_unscored_rows_and_zero_elsewhere():
    g = torch.Generator().manual_seed(3)
    h = torch.randn(12, 8, generator=g, dtype=F64)
    W = torch.randn(20, 8, generator=g, dtype=F64)
    y = torch.randint(0, 20, (12,), generator=g)
    scored = torch.rand(12, generator=g) < 0.4
    full = ohead.scored_rows(h, W, y, None, 0.7)
    part = ohead.scored_rows(h, W, y, scored, 0.7)
    assert torch.equal(part[scored], full[scored]) and (part[~scored] == 0).all()


def test_compaction_is_nonzero():
    rng = np.random.default_rng(0)
    for n in (0, 1, 63, 64, 65, 1000, 4097):
        m = rng.random(n) < rng.random()
        assert np.array_equal(opairs.compact(m), torch.nonzero(torch.from_numpy(m))[:, 0].numpy())


def _flat(seqs):
    from tests.tiny_models import packed
    return packed(seqs)


def test_trie_pairs_expand_to_flat_positions():
    """Reference tests/test_prefix_tree.py:165-176: tree tokens 1 2 3 4 9; flat position 1 ('2') asks for a
    different next token per sequence (3 vs 9); last positions ask for none."""
    flat, cu = _flat([[1, 2, 3, 4], [1, 2, 9]])
    tokens, f2t, posid = opairs.tree_positions(flat, cu)
    assert tokens.tolist() == [1, 2, 3, 4, 9] and posid.tolist() == [0, 1, 2, 3, 2]
    pos, lab, fp = opairs.pairs(flat, cu)
    assert fp[3] == -1 and fp[6] == -1
    assert (pos[fp[1]], lab[fp[1]]) == (1, 3) and (pos[fp[5]], lab[fp[5]]) == (1, 9)
    assert fp[0] == fp[4]  # "1" -> "2" in both sequences: one pair


@pytest.mark.parametrize("case", [0, 1, 2, 3])
def test_tree_output_gives_each_flat_position_its_pairs_row(case):
    """oracle.head.tree_output (prefix_tree.py:419-421: a zero row appended, then index_select by flat_pair) pinned by
    definition on the reference's hand-built forests and a random deduplicated one (tests/golden/prefix_pairs.json,
    the case of tests/test_prefix_tree.py:165-176 first): with each pair row made to name its pair, the position p
    that asks receives the row of (tree position of p, flat[p + 1]), every other position zeros. A wrong index, a
    missing zero row or a pair mixed up with its neighbour fails it."""
    import json
    import os
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "prefix_pairs.json")))[case]
    flat, cu = np.array(fx["flat"], dtype=np.int64), np.array(fx["cu"], dtype=np.int64)
    scored = None if fx["scored"] is None else np.array(fx["scored"], dtype=bool)
    tokens, f2t, _ = opairs.tree_positions(flat, cu)
    pos, lab, fp = opairs.pairs(flat, cu, scored)
    pair_rows = torch.stack([torch.as_tensor(pos, dtype=F64), torch.as_tensor(lab, dtype=F64)], 1)
    for none_marker in (-1, len(pos)):  # -1, or the appended zero row's index P (TreeMeta's form)
        fpx = np.where(fp < 0, none_marker, fp)
        out = ohead.tree_output(pair_rows, fpx)
        ends = set(int(e) - 1 for e in cu[1:])
        for p in range(len(flat)):
            asks = p not in ends and (scored is None or bool(scored[p]))
            want = [float(f2t[p]), float(flat[p + 1])] if asks else [0.0, 0.0]
            assert out[p].tolist() == want, (case, p)


def test_trie_pairs_of_scored_positions():
    """Reference tests/test_prefix_tree.py:179-188."""
    flat, cu = _flat([[1, 2, 3, 4], [1, 2, 3, 5], [1, 2, 9]])
    scored = np.isin(np.arange(flat.size), [1, 9])
    pos, lab, fp = opairs.pairs(flat, cu, scored)
    fpos, flab, ffp = opairs.pairs(flat, cu)
    assert len(pos) == 2 and (fp[~scored] == -1).all()
    for p in (1, 9):
        assert (pos[fp[p]], lab[fp[p]]) == (fpos[ffp[p]], flab[ffp[p]])
    assert ffp[1] == ffp[5]


def test_trie_dedups_shared_prefixes_and_keeps_every_sequence_exact():
    """Reference tests/test_prefix_tree.py:28-50."""
    rng = np.random.default_rng(0)
    prefix = rng.integers(0, 1000, 50)
    seqs = []
    for tail in (7, 3, 12):  # three continuations of the shared 50-token prefix
        seqs.append(np.concatenate([prefix, rng.integers(0, 1000, tail)]))
    seqs.append(np.concatenate([prefix[:20], rng.integers(0, 1000, 5)]))
    seqs.append(seqs[1].copy())
    seqs.append(rng.integers(1000, 2000, 9))
    flat, cu = _flat(seqs)
    tokens, f2t, posid = opairs.tree_positions(flat, cu)
    assert len(tokens) == 50 + 7 + 3 + 12 + 5 + 9
    pos, lab, fp = opairs.pairs(flat, cu)
    for a, b in zip(cu[:-1], cu[1:]):
        for p in range(a, b):
            if p == b - 1:
                assert fp[p] == -1
                continue
            assert tokens[pos[fp[p]]] == flat[p] and lab[fp[p]] == flat[p + 1]
            assert posid[pos[fp[p]]] == p - a


def test_trie_pairs_with_vocab_above_2_20():
    """Reference tests/test_prefix_tree.py:430-434."""
    big = (1 << 21) + 3
    flat, cu = _flat([[5, big, 7], [5, big, (1 << 20) + 9]])
    tokens, _, _ = opairs.tree_positions(flat, cu)
    pos, lab, fp = opairs.pairs(flat, cu)
    got = [(int(tokens[pos[fp[p]]]), int(lab[fp[p]])) for p in (0, 1, 3, 4)]
    assert got == [(5, big), (big, 7), (5, big), (big, (1 << 20) + 9)]


def test_grpo_closed_forms():
    n = 6
    logp = np.log(np.array([0.5, 0.2, 0.9, 0.1, 0.3, 0.4]))
    mask = np.array([1, 1, 1, 1, 1, 0])
    # reuse_train_logp: r == 1 inside the clip range, w = exp(logp - old); g = -A w / Z
    old = logp - np.array([0.01, -0.02, 0.0, 0.05, 2.0, 0.0])  # token 4: w = e^2 > 5: rejected
    adv = np.array([1.0, -2.0, 0.0, 0.5, 1.0, 3.0])
    loss, g = ogrpo.grpo(logp, adv, mask, old=old)
    w = np.exp(logp - old)
    Z = 5
    expect = np.array([-adv[i] * w[i] / Z for i in range(n)])
    expect[4] = 0.0  # rejected
    expect[5] = 0.0  # masked
    assert np.allclose(g, expect, atol=1e-15)
    assert abs(loss - sum(-adv[i] * w[i] for i in range(4)) / Z) < 1e-15
    # PPO ratio against a proximal policy: r above 1 + eps_hi with A > 0 is clipped (no gradient), with A < 0 not
    prox = logp - np.log(np.array([1.5, 1.5, 0.5, 0.5, 1.0, 1.0]))
    _, g2 = ogrpo.grpo(logp, np.array([1.0, -1.0, 1.0, -1.0, 2.0, 1.0]), mask, prox=prox)
    r = np.exp(logp - prox)
    assert g2[0] == 0.0 and abs(g2[1] - (1.0 * r[1] / Z)) < 1e-15
    assert abs(g2[2] - (-1.0 * r[2] / Z)) < 1e-15 and g2[3] == 0.0
    assert abs(g2[4] - (-2.0 / Z)) < 1e-15


def test_grpo_matches_torch_autograd_and_finite_differences():
    rng = np.random.default_rng(4)
    n = 40
    logp = np.log(rng.uniform(0.05, 1.0, n))
    prox = logp + rng.normal(0, 0.3, n)
    old = prox + rng.normal(0, 0.8, n)
    adv = rng.normal(0, 1, n)
    mask = rng.random(n) < 0.7
    loss, g = ogrpo.grpo(logp, adv, mask, prox=prox, old=old)
    # torch's maximum / clamp define the tie and boundary rules the restatement follows
    lp = torch.tensor(logp, requires_grad=True)
    A, m = torch.tensor(adv), torch.tensor(mask)
    w = torch.exp(torch.tensor(prox) - torch.tensor(old))
    w = torch.where(w > 5.0, torch.zeros_like(w), w)
    r = torch.exp(lp - torch.tensor(prox))
    pg = torch.maximum(-A * r, -A * torch.clamp(r, 0.8, 1.28)) * w
    L = torch.where(m, pg, torch.zeros_like(pg)).sum() / m.sum()
    L.backward()
    assert abs(L.item() - loss) < 1e-12 and np.allclose(lp.grad.numpy(), g, atol=1e-12)
    eps = 1e-7
    for t in range(n):
        a, b = logp.copy(), logp.copy()
        a[t] += eps
        b[t] -= eps
        num = (ogrpo.grpo(a, adv, mask, prox=prox, old=old)[0] - ogrpo.grpo(b, adv, mask, prox=prox, old=old)[0])
        assert abs(num / (2 * eps) - g[t]) < 1e-6


def test_baseline_matches_the_oracle():
    """oracle.baseline (the reference algorithm as run for the CPU baseline: CHUNK-row checkpointed chunks, autograd
    backward) agrees with the fp64 closed forms in fp32 over more than one chunk."""
    from oracle import baseline
    g = torch.Generator().manual_seed(6)
    n, d, V, T = 2048 + 300, 32, 257, 0.7
    h = torch.randn(n, d, generator=g)
    W = torch.randn(V, d, generator=g) * 0.3
    y = torch.randint(0, V, (n,), generator=g)
    gl = torch.randn(n, generator=g)
    out, gh, gw = baseline.fwd_bwd(h, W, y, T, gl)
    lp, ent, _ = ohead.head_forward(h, W, y, T)
    oh, ow = ohead.head_backward(h, W, y, T, gl)
    assert torch.allclose(out[:, 0].double(), lp, atol=1e-5) and torch.allclose(out[:, 1].double(), ent, atol=1e-5)
    assert ((gh.double() - oh).norm() / oh.norm()).item() < 1e-5
    assert ((gw.double() - ow).norm() / ow.norm()).item() < 1e-5


def test_e4m3_rounding_matches_torch_float8():
    """oracle.fp8 against torch's float8_e4m3fn conversion: every finite code, the midpoints between neighbouring
    codes (ties to even) and their fp32 neighbours, and a strided sweep of all fp32 bit patterns up to 448."""
    codes = np.arange(256, dtype=np.uint8)
    vals = ofp8.e4m3_value(codes)
    assert np.array_equal(np.nan_to_num(vals[:127], nan=1e9),
                          np.nan_to_num(torch.from_numpy(codes[:127]).view(torch.float8_e4m3fn).double().numpy(),
                                        nan=1e9))
    mag = np.unique(np.abs(vals[np.isfinite(vals)]))
    mids = (mag[:-1] + mag[1:]) / 2
    x = np.concatenate([vals[np.isfinite(vals)], mids, -mids]).astype(np.float32)
    x = np.concatenate([x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))])
    sweep = np.arange(0, np.float32(448).view(np.uint32) + 1, 997, dtype=np.uint32).view(np.float32)
    x = np.concatenate([x, sweep, -sweep])
    x = x[np.abs(x) <= 448]
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ofp8.e4m3_bits(x), want)


def test_fp8_row_quantiser_matches_torch():
    from octopus_amd.workloads import quantise_fp8_rows
    g = torch.Generator().manual_seed(0)
    W = torch.randn(64, 96, generator=g) * 0.02
    W[3] = 0.0
    W[5, :4] = torch.tensor([448.0, 1.0625, -1.1875, 2.0 ** -10])  # scale 1: ties and a half-subnormal
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        q, scale = ofp8.quantise_rows(W.to(dt).float().numpy())
        tq, ts = quantise_fp8_rows(W.to(dt))
        assert np.array_equal(scale, ts.numpy()) and np.array_equal(q, tq.view(torch.uint8).numpy())
        # the dequantised weight is within half an e4m3 step of the row-scaled weight
        deq = ofp8.e4m3_value(q) * scale[:, None]
        assert np.all(np.abs(deq - W.to(dt).double().numpy()) <= scale[:, None] * 16 * (1 + 1e-6) + 1e-30)
