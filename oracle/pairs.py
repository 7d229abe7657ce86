"""Oracle for the index work of the head path (test infrastructure only).

  compaction  octopus/rl/lm_head.py:128  `scored.nonzero()[:, 0]`: ascending positions of true entries
  tree        octopus/rl/prefix_tree.py:67-166  (no mounts): tree position of every flat token and the
              (tree position, next token) pairs, restated with a per-token trie in plain Python — a
              different construction from the product's run-grouping, so that the two pin each other.
              Pre-order over a per-token trie whose children are kept in first-insertion order gives the
              same numbering as the reference's run nodes (a run is a chain of single-child tokens).
"""

from __future__ import annotations

import numpy as np


def compact(mask) -> np.ndarray:
    m = np.asarray(mask).reshape(-1) != 0
    return np.array([i for i, f in enumerate(m.tolist()) if f], dtype=np.int64)


def tree_positions(flat, cu):
    """(tree_tokens, flat_to_tree, position_ids) by inserting the sequences into a per-token trie."""
    flat = [int(x) for x in np.asarray(flat).tolist()]
    cu = [int(c) for c in cu]
    children: list[dict] = [{}]  # node 0 is a virtual root; node k > 0 is one token
    token = [None]
    flat_nodes = []
    for a, b in zip(cu[:-1], cu[1:]):
        node = 0
        for t in flat[a:b]:
            nxt = children[node].get(t)
            if nxt is None:
                nxt = len(token)
                children[node][t] = nxt  # dicts keep insertion order: first appearance first
                children.append({})
                token.append(t)
            node = nxt
            flat_nodes.append(node)
    order = {}
    depth = {}
    stack = [(c, 0) for c in reversed(list(children[0].values()))]
    while stack:
        node, dep = stack.pop()
        order[node] = len(order)
        depth[node] = dep
        stack.extend((c, dep + 1) for c in reversed(list(children[node].values())))
    tree_tokens = np.empty(len(order), dtype=np.int64)
    position_ids = np.empty(len(order), dtype=np.int64)
    for node, pos in order.items():
        tree_tokens[pos] = token[node]
        position_ids[pos] = depth[node]
    flat_to_tree = np.array([order[n] for n in flat_nodes], dtype=np.int64)
    return tree_tokens, flat_to_tree, position_ids


def pairs(flat, cu, scored=None):
    """(pair_pos, pair_label, flat_pair): every scored flat position with a next token in its sequence asks
    for (its tree position, that token); distinct asks sorted by (position, label); -1 where no ask."""
    flat = [int(x) for x in np.asarray(flat).tolist()]
    cu = [int(c) for c in cu]
    _, f2t, _ = tree_positions(flat, cu)
    n = len(flat)
    sc = [True] * n if scored is None else [bool(x) for x in np.asarray(scored).tolist()]
    asks = {}
    for a, b in zip(cu[:-1], cu[1:]):
        for p in range(a, b - 1):
            if sc[p]:
                asks[p] = (int(f2t[p]), flat[p + 1])
    keys = sorted(set(asks.values()))
    row = {k: i for i, k in enumerate(keys)}
    flat_pair = np.full(n, -1, dtype=np.int64)
    for p, k in asks.items():
        flat_pair[p] = row[k]
    pos = np.array([k[0] for k in keys], dtype=np.int64)
    lab = np.array([k[1] for k in keys], dtype=np.int64)
    return pos, lab, flat_pair
