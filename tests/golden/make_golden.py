"""Writes the committed golden fixtures of the LM-head path (run from the repo root:
`python tests/golden/make_golden.py`). Test infrastructure: the expected values come from the oracle (fp64),
whose own pins are in tests/test_oracle.py; the fixtures freeze them so that a change to the oracle, the seeded
generators or the product is caught against stored numbers.

  head_small.npz       tiny heads with their inputs (bf16-representable values stored as fp32) and expected
                       logprob / entropy / lse (fp64) and gradients (fp32) for g = dL/dlogprob, plain and soft-capped
  cfg1_expected.npz    the CPU-runnable configuration (N 512, d 1024, V 32,000, fp32, T 1.0): expected logprob,
                       entropy and lse per row, plus input checksums of the seeded generator
  prefix_pairs.json    the reference's hand-built prefix-tree cases (tests/test_prefix_tree.py:28-50, 165-188,
                       430-434 of the reference): token sequences, scored masks, and the expected tree tokens,
                       position ids, label pairs and flat->pair map
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import head as ohead  # noqa: E402
from oracle import pairs as opairs  # noqa: E402

SMALL = [  # (name, n, d, V, T, pre, post, tanh, seed)
    ("plain", 40, 64, 600, 1.0, 1.0, 1.0, False, 1),
    ("temp", 33, 48, 401, 0.7, 1.0, 1.0, False, 2),
    ("softcap", 24, 32, 300, 1.3, 0.5, 2.0, True, 3),
]


def head_small() -> dict:
    out = {}
    for name, n, d, V, T, pre, post, tanh, seed in SMALL:
        g = torch.Generator().manual_seed(seed)
        h = torch.randn(n, d, generator=g)
        h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).float()
        W = (torch.randn(V, d, generator=g) * 0.02).to(torch.bfloat16).float()
        y = torch.randint(0, V, (n,), generator=g)
        gl = torch.randn(n, generator=g)
        lp, ent, lse = ohead.head_forward(h, W, y, T, pre, post, tanh)
        gh, gw = ohead.head_backward(h, W, y, T, gl, pre, post, tanh)
        out.update({f"{name}/h": h.numpy(), f"{name}/W": W.numpy(), f"{name}/y": y.numpy(),
                    f"{name}/g": gl.numpy(), f"{name}/params": np.array([T, pre, post, float(tanh)]),
                    f"{name}/logp": lp.numpy(), f"{name}/ent": ent.numpy(), f"{name}/lse": lse.numpy(),
                    f"{name}/grad_h": gh.float().numpy(), f"{name}/grad_W": gw.float().numpy()})
    return out


def cfg1() -> dict:
    from octopus_amd.workloads import CONFIGS, make_batch
    b = make_batch(CONFIGS["cfg1"], "cpu")
    lp, ent, lse = ohead.head_forward(b.hidden, b.weight, b.labels, CONFIGS["cfg1"].temperature)
    return {"logp": lp.numpy(), "ent": ent.numpy(), "lse": lse.numpy(), "labels": b.labels.numpy(),
            "h_sum": np.float64(b.hidden.double().sum()), "W_sum": np.float64(b.weight.double().sum()),
            "h_sq": np.float64(b.hidden.double().pow(2).sum()), "W_sq": np.float64(b.weight.double().pow(2).sum())}


def _flat(seqs):
    return np.concatenate(seqs), [0, *np.cumsum([len(s) for s in seqs]).tolist()]


def prefix_cases() -> list:
    rng = np.random.default_rng(0)
    prefix = rng.integers(0, 1000, 50)
    dedup = [np.concatenate([prefix, rng.integers(0, 1000, n)]) for n in (7, 3, 12)]
    dedup.append(np.concatenate([prefix[:20], rng.integers(0, 1000, 5)]))
    dedup.append(dedup[1].copy())
    dedup.append(rng.integers(1000, 2000, 9))
    cases = [
        ("expand", [np.array([1, 2, 3, 4]), np.array([1, 2, 9])], None),
        ("scored", [np.array([1, 2, 3, 4]), np.array([1, 2, 3, 5]), np.array([1, 2, 9])], [1, 9]),
        ("dedup", dedup, None),
        ("vocab_above_2_20", [np.array([5, (1 << 21) + 3, 7]), np.array([5, (1 << 21) + 3, (1 << 20) + 9])], None),
    ]
    out = []
    for name, seqs, scored_at in cases:
        flat, cu = _flat(seqs)
        scored = None
        if scored_at is not None:
            scored = np.zeros(len(flat), dtype=bool)
            scored[scored_at] = True
        tokens, f2t, posid = opairs.tree_positions(flat, cu)
        pos, lab, fp = opairs.pairs(flat, cu, scored)
        out.append({"name": name, "flat": flat.tolist(), "cu": cu,
                    "scored": None if scored is None else scored.astype(int).tolist(),
                    "tree_tokens": tokens.tolist(), "position_ids": posid.tolist(), "flat_to_tree": f2t.tolist(),
                    "pair_pos": pos.tolist(), "pair_label": lab.tolist(), "flat_pair": fp.tolist()})
    return out


def main() -> None:
    np.savez_compressed(os.path.join(HERE, "head_small.npz"), **head_small())
    np.savez_compressed(os.path.join(HERE, "cfg1_expected.npz"), **cfg1())
    with open(os.path.join(HERE, "prefix_pairs.json"), "w") as f:
        json.dump(prefix_cases(), f, indent=1)
    for fn in sorted(os.listdir(HERE)):
        print(fn, os.path.getsize(os.path.join(HERE, fn)))


if __name__ == "__main__":
    main()
