"""The oracle against the committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py), and
the seeded workload generator against its recorded checksums. CPU only."""

import json
import os

import numpy as np
import torch

from oracle import head as ohead
from oracle import pairs as opairs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _small():
    z = np.load(os.path.join(GOLDEN, "head_small.npz"))
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def test_oracle_reproduces_the_small_head_fixtures():
    z, names = _small()
    assert names == ["plain", "softcap", "temp"]
    for nm in names:
        h, W, y, g = (torch.from_numpy(z[f"{nm}/{k}"]) for k in ("h", "W", "y", "g"))
        T, pre, post, tanh = z[f"{nm}/params"].tolist()
        lp, ent, lse = ohead.head_forward(h, W, y, T, pre, post, bool(tanh))
        assert np.allclose(lp.numpy(), z[f"{nm}/logp"], atol=1e-12, rtol=0)
        assert np.allclose(ent.numpy(), z[f"{nm}/ent"], atol=1e-12, rtol=0)
        assert np.allclose(lse.numpy(), z[f"{nm}/lse"], atol=1e-12, rtol=0)
        gh, gw = ohead.head_backward(h, W, y, T, g, pre, post, bool(tanh))
        assert np.allclose(gh.float().numpy(), z[f"{nm}/grad_h"], atol=1e-9, rtol=1e-6)
        assert np.allclose(gw.float().numpy(), z[f"{nm}/grad_W"], atol=1e-9, rtol=1e-6)
        # the stored inputs are bf16 values (the GPU tests feed them as bf16 without rounding)
        assert torch.equal(h.to(torch.bfloat16).float(), h) and torch.equal(W.to(torch.bfloat16).float(), W)


def test_cfg1_generator_and_oracle_match_the_fixture():
    from octopus_amd.workloads import CONFIGS, make_batch
    z = np.load(os.path.join(GOLDEN, "cfg1_expected.npz"))
    b = make_batch(CONFIGS["cfg1"], "cpu")
    assert abs(b.hidden.double().sum().item() - float(z["h_sum"])) < 1e-6
    assert abs(b.weight.double().sum().item() - float(z["W_sum"])) < 1e-9
    assert abs(b.hidden.double().pow(2).sum().item() - float(z["h_sq"])) < 1e-6
    assert abs(b.weight.double().pow(2).sum().item() - float(z["W_sq"])) < 1e-9
    assert np.array_equal(b.labels.numpy(), z["labels"])
    lp, ent, lse = ohead.head_forward(b.hidden[:64], b.weight, b.labels[:64], 1.0)
    assert np.allclose(lp.numpy(), z["logp"][:64], atol=1e-12, rtol=0)
    assert np.allclose(ent.numpy(), z["ent"][:64], atol=1e-12, rtol=0)
    assert np.allclose(lse.numpy(), z["lse"][:64], atol=1e-12, rtol=0)


def test_oracle_reproduces_the_prefix_pair_fixtures():
    cases = json.load(open(os.path.join(GOLDEN, "prefix_pairs.json")))
    assert [c["name"] for c in cases] == ["expand", "scored", "dedup", "vocab_above_2_20"]
    for c in cases:
        scored = None if c["scored"] is None else np.array(c["scored"], dtype=bool)
        tokens, f2t, posid = opairs.tree_positions(np.array(c["flat"]), c["cu"])
        pos, lab, fp = opairs.pairs(np.array(c["flat"]), c["cu"], scored)
        assert tokens.tolist() == c["tree_tokens"] and posid.tolist() == c["position_ids"]
        assert f2t.tolist() == c["flat_to_tree"]
        assert pos.tolist() == c["pair_pos"] and lab.tolist() == c["pair_label"] and fp.tolist() == c["flat_pair"]


def test_product_tree_matches_the_prefix_pair_fixtures():
    """The product's run-grouping tree builder (octopus_amd.rl.prefix_tree) on the same cases, bit-exact."""
    from octopus_amd.rl.prefix_tree import build_tree
    for c in json.load(open(os.path.join(GOLDEN, "prefix_pairs.json"))):
        scored = None if c["scored"] is None else np.array(c["scored"], dtype=bool)
        t = build_tree(np.array(c["flat"]), c["cu"], scored=scored)
        assert t.tokens.tolist() == c["tree_tokens"] and t.position_ids.tolist() == c["position_ids"]
        assert t.pair_pos.tolist() == c["pair_pos"] and t.pair_label.tolist() == c["pair_label"]
        assert t.flat_pair.tolist() == c["flat_pair"]
