"""Oracle for the head arithmetic (test infrastructure only), restating in fp64:

  octopus/rl/lm_head.py:102-105  _head_chunk    z = post(h . W^T)
  octopus/rl/lm_head.py:108-112  _head_columns  s = z / T; logprob = s_y - logsumexp(s); entropy = -sum p log p
  octopus/rl/lm_head.py:115-130  _chunked_rows / _scored_rows (rows, scoring, zeros elsewhere)
  octopus/rl/prefix_tree.py:416-421 tree_head_output (pairs, then expansion with a zero row)
and the backward that autograd derives for them: with g_r = dL/dlogprob_r (entropy detached),
  dL/dz_rj = g_r (1[j = y_r] - p_rj) / T * post'(z_rj),  grad_h = dz . W,  grad_W = dz^T . h.

post(z) = post * tanh(pre * z) (softcap) or post * pre * z, the fused form of the recorded post-head ops.
Everything is computed in float64 on the CPU, in row blocks so large vocabularies fit in memory.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def post_z(z: torch.Tensor, pre: float = 1.0, post: float = 1.0, tanh: bool = False) -> torch.Tensor:
    return post * torch.tanh(pre * z) if tanh else post * pre * z


def post_dz(z: torch.Tensor, pre: float = 1.0, post: float = 1.0, tanh: bool = False) -> torch.Tensor:
    """d post(z) / dz."""
    if tanh:
        t = torch.tanh(pre * z)
        return post * pre * (1 - t * t)
    return torch.full_like(z, post * pre)


def columns(logits: torch.Tensor, temperature: float, labels: torch.Tensor):
    """(logprob, entropy, lse) per row of materialised logits, fp64."""
    s = logits.to(F64) / temperature
    m = s.max(dim=1, keepdim=True).values
    e = torch.exp(s - m)
    S = e.sum(1, keepdim=True)
    lse = (m + torch.log(S))[:, 0]
    p = e / S
    logp_y = s.gather(1, labels.view(-1, 1).long())[:, 0] - lse
    entropy = lse - (p * s).sum(1)
    return logp_y, entropy, lse


def head_forward(h: torch.Tensor, W: torch.Tensor, labels: torch.Tensor, temperature: float,
                 pre: float = 1.0, post: float = 1.0, tanh: bool = False, block: int = 256):
    """(logprob, entropy, lse) [n] fp64 of rows h [n, d] against W [V, d]."""
    W64 = W.to(F64)
    outs = []
    for r0 in range(0, h.shape[0], block):
        z = h[r0:r0 + block].to(F64) @ W64.T
        outs.append(columns(post_z(z, pre, post, tanh), temperature, labels[r0:r0 + block]))
    if not outs:
        e = torch.empty(0, dtype=F64)
        return e, e, e
    return tuple(torch.cat(c) for c in zip(*outs))


def head_backward(h: torch.Tensor, W: torch.Tensor, labels: torch.Tensor, temperature: float, g: torch.Tensor,
                  pre: float = 1.0, post: float = 1.0, tanh: bool = False, block: int = 256,
                  want_h: bool = True, want_w: bool = True):
    """(grad_h [n, d], grad_W [V, d]) fp64 of L with dL/dlogprob = g."""
    W64 = W.to(F64)
    n = h.shape[0]
    gh = torch.zeros(n, W.shape[1], dtype=F64) if want_h else None
    gw = torch.zeros(W.shape, dtype=F64) if want_w else None
    for r0 in range(0, n, block):
        hb = h[r0:r0 + block].to(F64)
        z = hb @ W64.T
        s = post_z(z, pre, post, tanh) / temperature
        p = torch.softmax(s, dim=1)
        onehot = torch.zeros_like(p)
        onehot.scatter_(1, labels[r0:r0 + block].view(-1, 1).long(), 1.0)
        dz = g[r0:r0 + block].to(F64).view(-1, 1) * (onehot - p) / temperature * post_dz(z, pre, post, tanh)
        if want_h:
            gh[r0:r0 + block] = dz @ W64
        if want_w:
            gw += dz.T @ hb
    return gh, gw


def scored_rows(h: torch.Tensor, W: torch.Tensor, labels: torch.Tensor, scored, temperature: float, **post):
    """[T, 2] fp64: (logprob, entropy) at scored rows, exactly 0 elsewhere (lm_head.py:124-130)."""
    out = torch.zeros(h.shape[0], 2, dtype=F64)
    at = torch.arange(h.shape[0]) if scored is None else torch.as_tensor(scored).bool().nonzero()[:, 0]
    lp, ent, _ = head_forward(h[at], W, labels[at], temperature, **post)
    out[at, 0], out[at, 1] = lp, ent
    return out


def tree_output(pairs_out: torch.Tensor, flat_pair) -> torch.Tensor:
    """[T_flat, C]: pair row flat_pair[t] for each flat position, a zero row where it is -1 or P."""
    fp = torch.as_tensor(flat_pair).long()
    P = pairs_out.shape[0]
    out = torch.zeros(fp.numel(), pairs_out.shape[1], dtype=pairs_out.dtype)
    ok = (fp >= 0) & (fp < P)
    out[ok] = pairs_out[fp[ok]]
    return out
