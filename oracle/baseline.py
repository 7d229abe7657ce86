"""The reference algorithm as the reference runs it, for the timed CPU baseline (test infrastructure only).

Clean-room torch restatement of octopus/rl/lm_head.py:102-121 on the host CPU:
  - rows in CHUNK = 2048-row chunks (lm_head.py:20, 118-121), each under non-reentrant checkpoint;
  - logits = rows @ W.T in the input dtype (bf16 GEMM, lm_head.py:105);
  - fp32 log-softmax of logits / T, detached entropy, label gather (lm_head.py:108-112);
  - backward by autograd: the chunk is recomputed, dlogits arrives in the input dtype (the backward of
    `.float()`), then dlogits @ W and dlogits^T @ rows; W.grad accumulates across chunks in W's dtype.
"""

from __future__ import annotations

import time

import torch
from torch.utils.checkpoint import checkpoint

CHUNK = 2048


def _columns(logits, temperature, labels):
    logp = torch.log_softmax(logits.float() / temperature, dim=-1)
    ent = (-(logp.exp() * logp).sum(-1)).detach()
    return torch.stack([logp.gather(-1, labels[:, None])[:, 0], ent], dim=-1)


def chunked_rows(rows, weight, labels, temperature):
    return torch.cat([checkpoint(lambda h, y: _columns(h @ weight.T, temperature, y), h, y, use_reentrant=False)
                      for h, y in zip(rows.split(CHUNK), labels.split(CHUNK))])


def fwd_bwd(rows, weight, labels, temperature, g):
    """One training pass: forward columns, then backward of sum(g * logprob). Returns (out, grad_rows, grad_W)."""
    rows = rows.detach().requires_grad_(True)
    weight = weight.detach().requires_grad_(True)
    out = chunked_rows(rows, weight, labels, temperature)
    (out[:, 0] * g).sum().backward()
    return out.detach(), rows.grad, weight.grad


def time_chunks(d: int, V: int, n_chunks: int, temperature: float = 1.0, dtype=torch.bfloat16, seed: int = 0,
                repeats: int = 3) -> dict:
    """Median seconds of one fwd+bwd pass over n_chunks * CHUNK rows (1 warm-up, then `repeats` timed)."""
    gen = torch.Generator().manual_seed(seed)
    n = n_chunks * CHUNK
    rows = torch.randn(n, d, generator=gen).to(dtype)
    weight = (torch.randn(V, d, generator=gen) * 0.02).to(dtype)
    labels = torch.randint(0, V, (n,), generator=gen)
    g = torch.randn(n, generator=gen) / n
    fwd_bwd(rows[:CHUNK], weight, labels[:CHUNK], temperature, g[:CHUNK])  # warm-up
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fwd_bwd(rows, weight, labels, temperature, g)
        times.append(time.perf_counter() - t0)
    times.sort()
    return {"seconds": times[len(times) // 2], "rows": n, "threads": torch.get_num_threads()}
