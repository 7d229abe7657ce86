"""Token tiling entry points of the trainer (octopus/rl/seq_tiles.py:34-56, 91-115), as the LM-head path
uses them: the `_fused` wrapper, TILE, `tiled` and `no_inner`.

`_fused` never compiles. In the reference it wraps element-wise blocks in torch.compile (Inductor, i.e.
Triton kernels on a GPU, seq_tiles.py:44-47); here every GPU block of the head path is a hand-written HIP
kernel, so `_fused(fn)` returns a dispatcher that runs the HIP implementation registered for fn on HIP
tensors and fn itself (eager torch) on CPU tensors. The eager function stays reachable as
`._torchdynamo_orig_callable`, the attribute the reference's compiled-vs-eager test reads
(tests/test_seq_tiles.py:157). COMPILE is kept for the flag's readers (OCTOPUS_COMPILE); it selects nothing.
"""

from __future__ import annotations

import contextlib
import functools
import os

import torch
from torch.utils.checkpoint import checkpoint

TILE = 16384
_INNER = True  # tiles checkpointed; no_inner() turns this off
COMPILE = os.environ.get("OCTOPUS_COMPILE", "1") != "0"


def _fused(fn=None, *, hip=None):
    """fn on CPU tensors, `hip` (same signature) on HIP tensors. Usable as @_fused or @_fused(hip=...)."""
    if fn is None:
        return functools.partial(_fused, hip=hip)

    @functools.wraps(fn)
    def run(*args, **kwargs):
        if hip is not None and any(isinstance(a, torch.Tensor) and a.is_cuda for a in args):
            return hip(*args, **kwargs)
        return fn(*args, **kwargs)

    run._torchdynamo_orig_callable = fn
    return run


def _checkpoint(fn, *args):
    return checkpoint(fn, *args, use_reentrant=False) if _INNER else fn(*args)


_REFERENCE_TILES = "octopus.rl.seq_tiles"  # the trainer's own module, whose flag its patched decoder layers read


@contextlib.contextmanager
def no_inner():
    """Tiles run without their own checkpoints (a caller's checkpoint recomputes them instead). The decoder layers the
    trainer patches read the flag of the trainer's own seq_tiles module (octopus/rl/seq_tiles.py:35, 92), so when that
    module is loaded its flag is switched as well (and restored after): chunk_major's reverse-chunk recompute
    (chunk_major.py:356) then plans the same activations whichever of the two modules it imports no_inner from."""
    import sys
    global _INNER
    ref = sys.modules.get(_REFERENCE_TILES)
    ref_before = getattr(ref, "_INNER", None)
    _INNER = False
    if ref is not None:
        ref._INNER = False
    try:
        yield
    finally:
        _INNER = True
        if ref is not None:
            ref._INNER = ref_before


def tiled(fn, *xs):
    """fn over [B, T, ...] inputs (None passes through), TILE tokens at a time along dim 1, each tile
    recomputed in backward; outputs (a tensor or a tuple of tensors) concatenated along dim 1."""
    parts = [None if x is None else x.split(TILE, dim=1) for x in xs]
    n = len(next(p for p in parts if p is not None))
    outs = [_checkpoint(fn, *(None if p is None else p[i] for p in parts)) for i in range(n)]
    if isinstance(outs[0], tuple):
        return tuple(torch.cat(cols, dim=1) for cols in zip(*outs))
    return torch.cat(outs, dim=1)
