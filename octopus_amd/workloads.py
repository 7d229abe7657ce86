"""Seeded synthetic workloads of the LM-head path (the five configurations it is measured and checked on).

Seeds, one generator per tensor: hidden 0, W 1, targets 2, advantages 3, old-logp noise 4, tree shape 5.
  hidden  ~ N(0, 1), then RMS-normalised: x / sqrt(mean(x^2) + 1e-6)
  W       ~ N(0, 0.02)
  targets ~ Zipf(1.1) over ranks 1..V mapped through a seeded permutation of the vocabulary (uniform for cfg1)

  cfg1  N 512,     d 1024, V 32,000,  fp32, T 1.0, every row scored, forward only
  cfg2  N 32,768,  d 2560, V 151,936, bf16, T 1.0, every row scored, forward only
  cfg3  N 32,768,  d 2560, V 151,936, bf16, T 1.0, tree: 8,192-token root (masked) + 12 branches x 2,048
        (scored); per-branch advantage ~ N(0, 1); old logp = logp + N(0, 0.01); fused fwd + bwd
  cfg4  N 65,536,  d 4096, V 128,256, bf16, T 0.7, tree of depth 3, fan-out 4: a 4,096-token root, shared nodes
        of 8,192 tokens, leaves of U[1024, 4096] tokens, laid out in pre-order until N tokens (the last trimmed);
        every node above the leaves is shared prefix (masked): 56.2% masked, 28,672 scored; fwd + bwd
  cfg5  N 131,072, d 2560, V 151,936, W fp8 e4m3 with per-row scale absmax / 448, hidden bf16, T 1.0; a
        16,384-token root (masked) + 16 branches x 7,168 (scored); fwd + bwd to hidden
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

SEED_HIDDEN, SEED_W, SEED_TARGETS, SEED_ADV, SEED_OLD, SEED_TREE = 0, 1, 2, 3, 4, 5


@dataclass
class Config:
    name: str
    N: int
    d: int
    V: int
    dtype: torch.dtype
    temperature: float
    backward: str  # "none", "full" (grad_h and grad_W), "hidden"
    zipf: bool = True
    fp8_weight: bool = False
    segments: list = field(default_factory=list)  # [(length, scored, advantage_group)]


CFG4_INNER = 8192  # tokens of each shared node between the root and the leaves


def _tree_cfg4(N: int = 65536, seed: int = SEED_TREE) -> list:
    """The recursive DAG of the d 4096 / V 128,256 workload, as [(tokens, scored, advantage group)] in pre-order: a
    4,096-token root, depth 3, fan-out 4; the leaves (the branches' own tokens, scored) draw U[1024, 4096] tokens from
    the seed; the shared nodes between root and leaves hold CFG4_INNER tokens each; nodes are laid out until N tokens,
    the last one trimmed. Every node above the leaves is deduplicated prefix (masked): 56.2% of the 65,536 tokens at
    seed 5 (28,672 scored rows in 12 leaves), against about 55% in the workload's description."""
    rng = np.random.default_rng(seed)
    segs = []
    total = 0

    def visit(depth: int, group: int):
        nonlocal total
        if total >= N:
            return
        leaf = depth == 3
        n = 4096 if depth == 0 else (int(rng.integers(1024, 4097)) if leaf else CFG4_INNER)
        n = min(n, N - total)
        segs.append((n, leaf, group))
        total += n
        if not leaf:
            for c in range(4):
                visit(depth + 1, group * 4 + c)

    while total < N:
        visit(0, len(segs))
    return segs


CONFIGS = {
    "cfg1": Config("cfg1", 512, 1024, 32000, torch.float32, 1.0, "none", zipf=False, segments=[(512, True, 0)]),
    "cfg2": Config("cfg2", 32768, 2560, 151936, torch.bfloat16, 1.0, "none", segments=[(32768, True, 0)]),
    "cfg3": Config("cfg3", 32768, 2560, 151936, torch.bfloat16, 1.0, "full",
                   segments=[(8192, False, 0)] + [(2048, True, b + 1) for b in range(12)]),
    "cfg4": Config("cfg4", 65536, 4096, 128256, torch.bfloat16, 0.7, "full", segments=_tree_cfg4()),
    "cfg5": Config("cfg5", 131072, 2560, 151936, torch.bfloat16, 1.0, "hidden", fp8_weight=True,
                   segments=[(16384, False, 0)] + [(7168, True, b + 1) for b in range(16)]),
}


def scaled(cfg: Config, N: int | None = None, d: int | None = None, V: int | None = None) -> Config:
    """The same configuration at smaller sizes (segments shrunk proportionally) for CPU-checkable parity."""
    N2, d2, V2 = N or cfg.N, d or cfg.d, V or cfg.V
    segs, acc = [], 0
    for i, (n, s, g) in enumerate(cfg.segments):
        m = max(1, round(n * N2 / cfg.N)) if i < len(cfg.segments) - 1 else max(1, N2 - acc)
        m = min(m, N2 - acc)
        if m <= 0:
            break
        segs.append((m, s, g))
        acc += m
    return Config(cfg.name + f"@{N2}x{d2}x{V2}", N2, d2, V2, cfg.dtype, cfg.temperature, cfg.backward, cfg.zipf,
                  cfg.fp8_weight, segs)


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def zipf_targets(n: int, V: int, s: float = 1.1, seed: int = SEED_TARGETS, device="cpu") -> torch.Tensor:
    """n targets with P(rank k) proportional to k^-s over ranks 1..V, ranks mapped through a seeded permutation."""
    g = _gen(seed, "cpu")
    w = torch.arange(1, V + 1, dtype=torch.float64).pow(-s)
    cdf = torch.cumsum(w / w.sum(), 0)
    u = torch.rand(n, generator=g, dtype=torch.float64)
    ranks = torch.searchsorted(cdf, u).clamp_(max=V - 1)
    perm = torch.randperm(V, generator=g)
    return perm[ranks].to(device)


def quantise_fp8_rows(W: torch.Tensor):
    """(Wq e4m3, scale [V] fp32) with scale = row absmax / 448 (the e4m3 maximum)."""
    W32 = W.float()
    scale = (W32.abs().amax(dim=1) / 448.0).clamp_(min=1e-12)
    Wq = (W32 / scale[:, None]).clamp_(-448, 448).to(torch.float8_e4m3fn)
    return Wq, scale.contiguous()


@dataclass
class Batch:
    cfg: Config
    hidden: torch.Tensor       # [N, d]
    weight: torch.Tensor       # [V, d] (bf16/fp32; fp8 when cfg.fp8_weight)
    w_scale: torch.Tensor | None
    labels: torch.Tensor       # [N] int64
    scored: torch.Tensor       # [N] bool
    adv: torch.Tensor          # [N] fp32 (per segment group)
    old_noise: torch.Tensor    # [N] fp32 ~ N(0, 0.01)


def make_batch(cfg: Config, device="cpu") -> Batch:
    gh = _gen(SEED_HIDDEN, device)
    x = torch.randn(cfg.N, cfg.d, generator=gh, device=device, dtype=torch.float32)
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    hidden = x.to(cfg.dtype)
    del x
    gw = _gen(SEED_W, device)
    W = torch.empty(cfg.V, cfg.d, device=device, dtype=torch.float32).normal_(0.0, 0.02, generator=gw)
    w_scale = None
    if cfg.fp8_weight:
        weight, w_scale = quantise_fp8_rows(W)
    else:
        weight = W.to(cfg.dtype)
    del W
    if cfg.zipf:
        labels = zipf_targets(cfg.N, cfg.V, device=device)
    else:
        labels = torch.randint(0, cfg.V, (cfg.N,), generator=_gen(SEED_TARGETS, "cpu")).to(device)
    scored = torch.zeros(cfg.N, dtype=torch.bool)
    groups = torch.zeros(cfg.N, dtype=torch.int64)
    at = 0
    for n, s, grp in cfg.segments:
        scored[at:at + n] = s
        groups[at:at + n] = grp
        at += n
    adv_per_group = torch.randn(int(groups.max()) + 1, generator=_gen(SEED_ADV, "cpu"))
    adv = adv_per_group[groups]
    old_noise = torch.randn(cfg.N, generator=_gen(SEED_OLD, "cpu")) * 0.01
    return Batch(cfg, hidden, weight, w_scale, labels, scored.to(device), adv.to(device), old_noise.to(device))


def dequantised(batch: Batch) -> torch.Tensor:
    """fp32 weights the fp8 path stands for: e4m3 value * row scale."""
    if batch.w_scale is None:
        return batch.weight.float()
    return batch.weight.float() * batch.w_scale[:, None]
