"""Oracle for the GRPO objective at the head's output (test infrastructure only).

Restates AReaL's decoupled PPO/GRPO actor loss as the reference configures it (grpo_loss_fn, cited by the
reference at docs/rl-plan-episodes.md:496-497; eps_clip 0.2, eps_clip_higher 0.28, rejection of behaviour
ratio > 5.0 in grpo.yaml:103-118; objective in paper/main.tex:421-424). AReaL itself is not in the
reference tree (un-vendored), so no reference test pins it; the checks in tests/test_oracle.py pin this
restatement by closed-form cases, finite differences and torch autograd.

Per token t with mask m_t != 0 (Z = number of such tokens, at least 1):
    r_t = exp(logp_t - prox_t)            prox = logp (value only) when not given (reuse_train_logp)
    w_t = exp(prox_t - old_t)             1 when old is not given; 0 when w_t > reject_upper > 0
    L   = sum_t w_t * max(-A_t r_t, -A_t clip(r_t, 1 - eps_lo, 1 + eps_hi)) / Z
    g_t = dL/dlogp_t = w_t * r_t * (-A_t) * [branch weight] / Z
where the max's gradient goes to the larger branch, half to each on a tie (torch.maximum), and the clipped
branch passes gradient only for r_t inside [1 - eps_lo, 1 + eps_hi] (torch.clamp).
"""

from __future__ import annotations

import numpy as np


def grpo(logp, adv, mask, prox=None, old=None, eps_lo=0.2, eps_hi=0.28, reject_upper=5.0):
    """(loss, g) in float64."""
    logp = np.asarray(logp, dtype=np.float64)
    adv = np.asarray(adv, dtype=np.float64)
    m = np.asarray(mask) != 0
    px = logp if prox is None else np.asarray(prox, dtype=np.float64)
    Z = max(1, int(m.sum()))
    r = np.exp(logp - px)
    if old is None:
        w = np.ones_like(logp)
    else:
        w = np.exp(px - np.asarray(old, dtype=np.float64))
        if reject_upper > 0:
            w = np.where(w > reject_upper, 0.0, w)
    lo, hi = 1.0 - eps_lo, 1.0 + eps_hi
    a = -adv * r
    b = -adv * np.clip(r, lo, hi)
    ga = np.where(a > b, 1.0, np.where(a < b, 0.0, 0.5))
    gb = 1.0 - ga
    inside = (r >= lo) & (r <= hi)
    dmax = ga * (-adv) + gb * (-adv) * inside
    g = np.where(m, w * dmax * r / Z, 0.0)
    loss = float(np.where(m, w * np.maximum(a, b), 0.0).sum() / Z)
    return loss, g
