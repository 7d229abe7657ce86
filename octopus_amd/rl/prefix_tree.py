"""Prefix-tree pieces of the LM-head path (octopus/rl/prefix_tree.py): the tree of a packed micro-batch as
far as the head needs it, its (tree position, next token) label pairs, and `tree_head_output`, which runs
the head once per pair and expands the pairs back to the flat per-sequence layout.

Layout rules follow the reference (prefix_tree.py:67-166) so that tree positions, and with them every pair
index, are identical:
  - a node is the longest run of tokens its sequences share from its start (until they differ or the
    shortest one ends); its children are grouped by their next token, in the order the sequences appear;
  - nodes are laid out in pre-order, so node ranges tile [0, T_tree) and a child follows its parent's subtree
    position in depth-first order;
  - a token's position id is its position on its own path.
Mounts (cross-branch reads) belong to the attention layers, not to the head, and are rejected.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Node:
    start: int  # [start, end) in tree order
    end: int
    parent: int  # index into nodes, -1 for a root
    depth: int
    path: np.ndarray  # tree indices of the ancestors' tokens and this node's, in order


@dataclass
class Tree:
    tokens: np.ndarray  # (T_tree,)
    nodes: list
    position_ids: np.ndarray  # (T_tree,)
    pair_pos: np.ndarray  # (P,) tree position whose hidden state scores a label
    pair_label: np.ndarray  # (P,) that label (the next token)
    flat_pair: np.ndarray  # (T_flat,) pair of each flat position, -1 when none
    flat_to_tree: np.ndarray | None = None  # (T_flat,) tree position of each flat token (input of on_device)


def _shared_run(seqs: list, ids: list, offset: int) -> int:
    """Length of the run the sequences `ids` share from `offset` (they all have a token there)."""
    ref = seqs[ids[0]]
    n = len(ref) - offset
    for i in ids[1:]:
        s = seqs[i]
        m = min(len(ref), len(s))
        differ = np.flatnonzero(ref[offset:m] != s[offset:m])
        n = min(n, int(differ[0]) if differ.size else m - offset)
    return n


def build_tree(flat: np.ndarray, cu, mounts=None, scored: np.ndarray | None = None) -> Tree:
    """Prefix tree of the sequences flat[cu[i]:cu[i+1]] and its label pairs.

    scored: (T_flat,) bool, the flat positions whose head output is used (None: all). A pair exists for
    each distinct (tree position, next token) of a scored position that has a next token; pairs are sorted
    by (position, label). flat_pair maps each flat position to its pair, or -1."""
    if mounts:
        raise NotImplementedError("mounted (cross-branch) reads are not part of the LM-head path")
    flat = np.asarray(flat)
    cu = [int(c) for c in cu]
    seqs = [flat[a:b] for a, b in zip(cu[:-1], cu[1:])]
    nodes: list[Node] = []
    tokens: list[np.ndarray] = []
    terminal = [-1] * len(seqs)
    n_tree = 0

    def groups(ids: list, end: int, here: int) -> list:
        """Sequences continuing after `end`, grouped by their next token (first-appearance order);
        the ones ending at `end` terminate at node `here`."""
        out: dict[int, list] = {}
        for i in ids:
            if len(seqs[i]) == end:
                terminal[i] = here
            else:
                out.setdefault(int(seqs[i][end]), []).append(i)
        return [(g, end, here) for g in out.values()]

    todo = groups(list(range(len(seqs))), 0, -1)[::-1]  # a stack: pre-order = first group first
    while todo:
        ids, offset, parent = todo.pop()
        length = _shared_run(seqs, ids, offset)
        parent_path = nodes[parent].path if parent >= 0 else np.empty(0, dtype=np.int64)
        nodes.append(Node(n_tree, n_tree + length, parent, nodes[parent].depth + 1 if parent >= 0 else 0,
                          np.concatenate([parent_path, np.arange(n_tree, n_tree + length, dtype=np.int64)])))
        tokens.append(seqs[ids[0]][offset:offset + length])
        n_tree += length
        todo.extend(groups(ids, offset + length, len(nodes) - 1)[::-1])

    tree_tokens = np.concatenate(tokens) if tokens else np.empty(0, dtype=flat.dtype)
    position_ids = np.empty(n_tree, dtype=np.int64)
    for node in nodes:
        first = len(node.path) - (node.end - node.start)
        position_ids[node.start:node.end] = np.arange(first, first + node.end - node.start)
    flat_to_tree = np.concatenate([nodes[t].path if t >= 0 else np.empty(0, dtype=np.int64) for t in terminal]
                                  + [np.empty(0, dtype=np.int64)])
    pair_pos, pair_label, flat_pair = label_pairs(flat, cu, flat_to_tree, scored)
    return Tree(tree_tokens, nodes, position_ids, pair_pos, pair_label, flat_pair, flat_to_tree)


def label_pairs(flat: np.ndarray, cu, flat_to_tree: np.ndarray, scored: np.ndarray | None = None):
    """(pair_pos, pair_label, flat_pair) of prefix_tree.py:156-166: flat position p (scored, not the last
    of its sequence) asks for the logprob of flat[p + 1] at tree position flat_to_tree[p]; equal asks share
    one pair; pairs sorted by (tree position, label)."""
    flat = np.asarray(flat)
    n = len(flat)
    asks = np.ones(n, dtype=bool) if scored is None else np.asarray(scored, dtype=bool).copy()
    ends = np.asarray(cu[1:], dtype=np.int64) - 1
    asks[ends] = False
    pos = flat_to_tree[asks].astype(np.int64)
    label = flat[1:][asks[:-1]].astype(np.int64) if n else np.empty(0, dtype=np.int64)
    if pos.size == 0:
        return np.empty(0, dtype=np.int64), np.empty(0, dtype=np.int64), np.full(n, -1, dtype=np.int64)
    uniq, inverse = np.unique(np.stack([pos, label], axis=1), axis=0, return_inverse=True)
    flat_pair = np.full(n, -1, dtype=np.int64)
    flat_pair[asks] = inverse.reshape(-1)
    return uniq[:, 0].copy(), uniq[:, 1].copy(), flat_pair


class TreeMeta:
    """The tree's pair tensors on a device (prefix_tree.py:200-205): pair_pos, pair_label and flat_pair,
    with -1 (no pair) mapped to P, the index of an appended zero row.

    `TreeMeta.on_device` builds the same pairs on a HIP device instead of on the host: then pair_pos and
    pair_label have T_flat entries of which the first P are the pairs, P stays on the device (`pair_count`),
    and flat_pair holds -1 where a position has no pair."""

    pair_count = None  # [1] int32 on the device when the pairs were built there

    def __init__(self, tree: Tree, device):
        self.n_tokens = len(tree.tokens)
        self.pair_pos = torch.from_numpy(np.ascontiguousarray(tree.pair_pos)).to(device)
        self.pair_label = torch.from_numpy(np.ascontiguousarray(tree.pair_label)).to(device)
        flat_pair = tree.flat_pair.copy()
        flat_pair[flat_pair < 0] = len(tree.pair_pos)
        self.flat_pair = torch.from_numpy(flat_pair).to(device)

    @classmethod
    def on_device(cls, flat: torch.Tensor, cu: torch.Tensor, flat_to_tree: torch.Tensor, n_tokens: int,
                  scored: torch.Tensor | None = None) -> "TreeMeta":
        """The pair section of build_tree (prefix_tree.py:156-166) run by the octo_label_pairs kernels on the
        device of `flat`: flat [T_flat] tokens, cu [n_seq + 1] sequence offsets, flat_to_tree [T_flat] tree
        position of each flat token (the tree built on the host), n_tokens = T_tree."""
        from octopus_amd.head_op import label_pairs
        self = cls.__new__(cls)
        self.n_tokens = int(n_tokens)
        self.pair_pos, self.pair_label, self.flat_pair, count = label_pairs(flat, cu, flat_to_tree, n_tokens, scored)
        self.pair_count = count[:1]
        return self


def tree_head_output(chunk_fn, hidden: torch.Tensor, meta: TreeMeta) -> torch.Tensor:
    """[1, T_tree, H] hidden -> [1, T_flat, C]: chunk_fn(rows, labels) -> [n, C] run on the pair rows, then
    each flat position takes its pair's row (0 where it has none).

    On HIP tensors a chunk_fn carrying `octopus_fused_rows(hidden2d, pair_pos, labels)` (the bound head)
    gathers the pair rows inside its GEMM instead of materialising them, and the expansion is the
    octohead::pairs_expand kernel."""
    fused = getattr(chunk_fn, "octopus_fused_rows", None)
    if meta.pair_count is not None and not (hidden.is_cuda and fused is not None):
        raise ValueError("pairs built on the device (TreeMeta.on_device) need a HIP hidden and the bound head")
    if hidden.is_cuda and fused is not None:
        if meta.pair_count is not None:  # P on the device: rows at and past it are left out by the head
            pairs = fused(hidden[0], meta.pair_pos, meta.pair_label, count=meta.pair_count)
        else:
            pairs = fused(hidden[0], meta.pair_pos, meta.pair_label)
    else:
        pairs = chunk_fn(hidden[0].index_select(0, meta.pair_pos), meta.pair_label)
    if hidden.is_cuda and pairs.dtype == torch.float32:
        from octopus_amd.head_op import pairs_expand
        return pairs_expand(pairs, meta.flat_pair).unsqueeze(0)
    pairs = torch.cat([pairs, pairs.new_zeros(1, pairs.shape[1])])
    return pairs.index_select(0, meta.flat_pair).unsqueeze(0)
