"""The label-pair section of build_tree (reference prefix_tree.py:156-166) on the device (octo_label_pairs),
bit-exact against the oracle's per-token trie and against the host restatement, and the head run on pairs whose
count stays on the device.

Cases: random forests with shared prefixes, duplicates, empty sequences and scored masks; the reference's
hand-built cases (tests/golden/prefix_pairs.json, labels above 2^20 included); trees at the measured sizes (a
16,384-token root under 16 branches of 7,168; 300 sequences through one 64-token prefix, so 300 asks share each
prefix position); tree positions out of range, which are counted and given no pair."""

import json
import os

import numpy as np
import pytest
import torch

from octopus_amd import head_op
from octopus_amd.head_op import fused_head
from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
from oracle import head as ohead
from oracle import pairs as opairs

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "prefix_pairs.json")


def _flat(seqs):
    from tests.tiny_models import packed
    return packed(seqs)


def _forest(rng, n_seq, vocab=6):
    base = [rng.integers(0, vocab, rng.integers(1, 30)) for _ in range(3)]
    seqs = []
    for _ in range(n_seq):
        b = base[rng.integers(0, 3)]
        cut = int(rng.integers(0, len(b) + 1))
        seqs.append(np.concatenate([b[:cut], rng.integers(0, vocab, rng.integers(0, 8))]))
    return seqs


def _device(flat, cu, f2t, T_tree, scored, none_as_count=False):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    pos, lab, fp, count = head_op.label_pairs(t(flat), t(np.asarray(cu, dtype=np.int64)), t(f2t), T_tree,
                                              None if scored is None else t(scored), none_as_count)
    c = count.cpu().tolist()
    P = c[0]
    return pos[:P].cpu().numpy(), lab[:P].cpu().numpy(), fp.cpu().numpy(), c


def _check(flat, cu, scored, f2t=None, T_tree=None, ref=None):
    if f2t is None:
        tokens, f2t, _ = opairs.tree_positions(flat, cu)
        T_tree = len(tokens)
    pos, lab, fp = ref if ref is not None else opairs.pairs(flat, cu, scored)
    dpos, dlab, dfp, c = _device(flat, cu, f2t, T_tree, scored)
    assert c == [len(pos), 0]
    assert np.array_equal(dpos, pos) and np.array_equal(dlab, lab) and np.array_equal(dfp, fp)
    _, _, dfp2, _ = _device(flat, cu, f2t, T_tree, scored, none_as_count=True)
    assert np.array_equal(dfp2, np.where(fp < 0, len(pos), fp))


def test_device_pairs_match_the_trie_oracle_on_random_forests():
    for seed in range(40):
        rng = np.random.default_rng(seed)
        flat, cu = _flat(_forest(rng, int(rng.integers(1, 12))))
        if len(flat) == 0:
            continue
        scored = None if seed % 3 == 0 else (rng.random(len(flat)) < 0.5)
        _check(flat, cu, scored)


def test_device_pairs_on_the_reference_cases():
    cases = json.load(open(GOLDEN))
    assert len(cases) >= 4
    for c in cases:
        flat = np.asarray(c["flat"], dtype=np.int64)
        scored = None if c["scored"] is None else np.asarray(c["scored"], dtype=bool)
        ref = tuple(np.asarray(c[k], dtype=np.int64) for k in ("pair_pos", "pair_label", "flat_pair"))
        _check(flat, c["cu"], scored, np.asarray(c["flat_to_tree"], dtype=np.int64), len(c["tree_tokens"]), ref)


def test_device_pairs_at_measured_sizes_match_the_host_restatement():
    rng = np.random.default_rng(11)
    # 16 branches of 7,168 under a 16,384-token root; labels past 2^20; prompt rows unscored
    root = rng.integers(0, 151936, 16384)
    seqs = [np.concatenate([root, rng.integers(0, (1 << 21), 7168)]) for _ in range(16)]
    flat, cu = _flat(seqs)
    scored = np.ones(len(flat), dtype=bool)
    for a in cu[:-1]:
        scored[a:a + 16384] = False
    # 300 sequences through one 64-token prefix, branching on few distinct next tokens
    pre = rng.integers(0, 50, 64)
    seqs2 = [np.concatenate([pre, rng.integers(0, 4, int(rng.integers(0, 40)))]) for _ in range(300)]
    for flat_, cu_, sc in ((flat, cu, scored), (*_flat(seqs2), None), (*_flat(seqs2), rng.random(
            sum(len(s) for s in seqs2)) < 0.7)):
        tree = build_tree(flat_, cu_, scored=sc)
        _check(flat_, cu_, sc, tree.flat_to_tree, len(tree.tokens), (tree.pair_pos, tree.pair_label, tree.flat_pair))


def test_tree_positions_out_of_range_are_counted_and_get_no_pair():
    flat, cu = _flat([[1, 2, 3, 4], [1, 2, 9]])
    f2t = np.array([0, 1, 2, 3, 0, 7, 4], dtype=np.int64)  # position 5 -> tree position 7 of 5
    dpos, dlab, dfp, c = _device(flat, cu, f2t, 5, None)
    assert c == [3, 1]
    assert dfp.tolist() == [0, 1, 2, -1, 0, -1, -1]
    assert dpos.tolist() == [0, 1, 2] and dlab.tolist() == [2, 3, 4]


def test_head_on_device_pairs_equals_the_host_pairs():
    """tree_head_output over TreeMeta.on_device (P on the device) equals it over the host TreeMeta, values
    bitwise and gradients, and the pair rows agree with the oracle."""
    rng = np.random.default_rng(5)
    prefix = rng.integers(0, 500, 300)
    seqs = [np.concatenate([prefix, rng.integers(0, 500, k)]) for k in (40, 90, 7, 64)]
    flat, cu = _flat(seqs)
    scored = rng.random(len(flat)) < 0.6
    tree = build_tree(flat, cu, scored=scored)
    host = TreeMeta(tree, DEV)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    dev = TreeMeta.on_device(t(flat), t(np.asarray(cu)), t(tree.flat_to_tree), len(tree.tokens), t(scored))
    d, V = 64, 500
    g = torch.Generator().manual_seed(6)
    h = torch.randn(len(tree.tokens), d, generator=g)
    W = torch.randn(V, d, generator=g) * 0.02
    gw = torch.randn(len(flat), 2, generator=torch.Generator().manual_seed(7)).to(DEV)[None]
    outs, grads = [], []
    for meta in (host, dev):
        hd = h.to(DEV)[None].requires_grad_(True)
        Wd = W.to(DEV).requires_grad_(True)

        def chunk(rows, labels):
            return fused_head(rows, Wd, labels, 0.9)

        chunk.octopus_fused_rows = lambda h2, pos, y, count=None: fused_head(h2, Wd, y, 0.9, idx=pos, count=count)
        out = tree_head_output(chunk, hd, meta)
        (out * gw).sum().backward()
        outs.append(out.detach())
        grads.append((hd.grad, Wd.grad))
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(grads[0], grads[1]):
        assert ((a - b).norm() / b.norm()).item() < 1e-6
    P = int(dev.pair_count.item())
    assert P == len(tree.pair_pos)
    lp, ent, _ = ohead.head_forward(h[tree.pair_pos], W, torch.from_numpy(tree.pair_label), 0.9)
    rows = outs[1][0][torch.from_numpy(np.flatnonzero(tree.flat_pair >= 0)).to(DEV)].cpu().double()
    want = lp[torch.from_numpy(tree.flat_pair[tree.flat_pair >= 0])]
    assert (rows[:, 0] - want).abs().max() < 1e-5
