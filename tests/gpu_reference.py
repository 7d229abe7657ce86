"""Chunked fp32 torch reference of the head on the GPU (tests only): the "plain PyTorch fp32 reference" for
full-size configurations, where the fp64 CPU oracle can only afford a subsample of rows.

logits = rows.float() @ W.float().T per chunk (W given as fp32, e.g. dequantised fp8), post-head
transform, fp32 log-softmax / T, entropy; backward in closed form dz = g (onehot - p) / T * post'(z),
grad_rows = dz @ W, grad_W = dz^T @ rows, all fp32."""

from __future__ import annotations

import torch


def _post(z, pre, post, tanh):
    return post * torch.tanh(pre * z) if tanh else (post * pre) * z


def _dpost(z, pre, post, tanh):
    if tanh:
        t = torch.tanh(pre * z)
        return post * pre * (1 - t * t)
    return post * pre


def head_fp32(rows, W32, labels, temperature, g=None, pre=1.0, post=1.0, tanh=False, chunk=2048, want_w=True):
    """(logp [n], entropy [n], grad_rows [n, d] or None, grad_W [V, d] or None), fp32."""
    n = rows.shape[0]
    logp = torch.empty(n, device=rows.device)
    ent = torch.empty(n, device=rows.device)
    gr = torch.empty(n, W32.shape[1], device=rows.device) if g is not None else None
    gw = torch.zeros_like(W32) if (g is not None and want_w) else None
    for r0 in range(0, n, chunk):
        h = rows[r0:r0 + chunk].float()
        y = labels[r0:r0 + chunk]
        z = h @ W32.T
        s = _post(z, pre, post, tanh) / temperature
        lp = torch.log_softmax(s, dim=1)
        p = lp.exp()
        logp[r0:r0 + chunk] = lp.gather(1, y[:, None])[:, 0]
        ent[r0:r0 + chunk] = -(p * lp).sum(1)
        if g is not None:
            p.neg_()
            p.scatter_add_(1, y[:, None], torch.ones_like(y[:, None], dtype=p.dtype))
            dz = p * (g[r0:r0 + chunk, None].float() / temperature)
            if tanh:
                dz *= _dpost(z, pre, post, tanh)
            else:
                dz *= pre * post
            gr[r0:r0 + chunk] = dz @ W32
            if want_w:
                gw.addmm_(dz.T, h)
        del z, s, lp, p
    return logp, ent, gr, gw
