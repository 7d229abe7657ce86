"""The chunked LM head (octopus/rl/lm_head.py), MI355X edition: each position's (logprob of its next token,
entropy) without materialising the [tokens x vocab] logits.

Call surface kept from the reference: CHUNK, bind_head, _chunked_head_forward, _scored_rows, _chunked_rows,
_head_chunk, _head_columns (a module global looked up at call time), _post_head_ops / _post_head / _Tail /
_skipping. The trainer sets head.octopus_labels, head.octopus_scored and head.octopus_tree per call; the
output is [1, T_flat, 2] with column 0 the logprob and column 1 the (detached) entropy, 0 where a position
is not scored or has no next token.

Routing: rows on a HIP device run the fused path (octopus_amd.head_op: one MFMA GEMM with the softmax
epilogue per tile, a recompute backward, compaction and pair gathers inside the kernels; no CHUNK loop,
since no [CHUNK, V] logits ever exist). Rows on the CPU run the reference's own composite semantics in
torch (CHUNK-row checkpointed chunks of `hidden @ W.T` then `_head_columns`), so a CPU model behaves as it
does under the reference. A HIP path never falls back to torch: an unsupported dtype or post-head op raises.
"""

from __future__ import annotations

import contextlib
import functools
import types

import torch
from torch.overrides import TorchFunctionMode
from torch.utils import _pytree as pytree
from torch.utils.checkpoint import checkpoint

from octopus_amd.rl.prefix_tree import tree_head_output
from octopus_amd.rl.seq_tiles import _fused

CHUNK = 2048  # rows per checkpointed chunk of the CPU composite path (lm_head.py:20)

_LOGITS = object()  # stands for the head's logits in a recorded post-head op (func, args, kwargs)

# Tensor methods that write into their first operand (besides the name_ methods and out= calls)
_WRITES = {"__setitem__", "__iadd__", "__isub__", "__imul__", "__itruediv__", "__ifloordiv__", "__imod__",
           "__ipow__", "__imatmul__", "__iand__", "__ior__", "__ixor__", "__ilshift__", "__irshift__"}


def _replace(tree, match, value):
    """tree with each leaf for which match(leaf) holds replaced by value."""
    return pytree.tree_map(lambda leaf: value if match(leaf) else leaf, tree)


class _ChainProbe(TorchFunctionMode):
    """While active, follows one tensor's lineage through a forward: after start(t), every torch function that reads
    the newest tensor of the lineage is recorded as (func, args, kwargs) with that tensor replaced by _LOGITS, and its
    result becomes the newest. A write into the lineage, or a read of any tensor of it but the newest (the flow
    forks), cannot be replayed by one chain of ops: NotImplementedError."""

    def __init__(self):
        super().__init__()
        self.lineage: list = []
        self.ops: list = []

    def start(self, t: torch.Tensor) -> None:
        self.lineage = [t]

    def __torch_function__(self, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        value = func(*args, **kwargs)
        if not self.lineage:
            return value
        read = [x for x in pytree.tree_leaves((args, kwargs)) if any(x is t for t in self.lineage)]
        if not read:
            return value
        name = getattr(func, "__name__", repr(func))
        newest = self.lineage[-1]
        if any(x is not newest for x in read):
            raise NotImplementedError(f"post-head logits: {name} reads an earlier result of the head's output; "
                                      "one chain of ops cannot reproduce that")
        if value is None or name in _WRITES or "out" in kwargs or (name.endswith("_") and not name.endswith("__")):
            raise NotImplementedError(f"post-head logits: {name} writes them in place; it cannot be replayed")
        if isinstance(value, torch.Tensor):  # (metadata queries such as .shape return other types)
            self.ops.append(_replace((func, args, kwargs), lambda leaf: leaf is newest, _LOGITS))
            if value is not newest:
                self.lineage.append(value)
        return value


@contextlib.contextmanager
def _forwards(replacements: dict):
    """Each module's forward replaced by the given callable for the duration (instance attributes, restored after)."""
    before = {m: m.__dict__.get("forward") for m in replacements}
    try:
        for m, f in replacements.items():
            m.forward = f
        yield
    finally:
        for m, f in before.items():
            if f is None:
                m.__dict__.pop("forward", None)
            else:
                m.forward = f


class _Countdown:
    """The bound head's output and how many post-head ops of the model are still to pass over it."""
    __slots__ = ("out", "left")

    def __init__(self, out: torch.Tensor, left: int):
        self.out, self.left = out, left


class _Tail(torch.Tensor):
    """The bound head's output as the model's own forward sees it after its lm_head. The model's post-head ops ran
    inside the head already (on each chunk's logits), so each op the model applies to it returns the head's output
    again, until the ops recorded at bind time have passed; queries that return no tensor (shape, dtype, ...) are
    answered from the output itself."""
    _octo_countdown: _Countdown = None

    @classmethod
    def __torch_function__(cls, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        countdown = next(x._octo_countdown for x in pytree.tree_leaves((args, kwargs)) if isinstance(x, _Tail))
        with torch._C.DisableTorchFunctionSubclass():
            value = func(*args, **kwargs)
        if not isinstance(value, torch.Tensor):
            return value
        countdown.left -= 1
        return countdown.out if countdown.left <= 0 else _as_tail(countdown)


def _as_tail(countdown: _Countdown) -> _Tail:
    t = countdown.out.as_subclass(_Tail)
    t._octo_countdown = countdown
    return t


def _skipping(out: torch.Tensor, n: int) -> torch.Tensor:
    """out, seen through the model's next n post-head ops (out itself when n == 0)."""
    return out if n <= 0 else _as_tail(_Countdown(out, n))


def _post_head(ops: list, logits: torch.Tensor) -> torch.Tensor:
    """The recorded post-head ops applied in order to logits, each to the previous op's result."""
    def apply(x, op):
        func, args, kwargs = _replace(op, lambda leaf: leaf is _LOGITS, x)
        return func(*args, **kwargs)
    return functools.reduce(apply, ops, logits)


def _post_head_ops(model, head) -> list:
    """The ops the model's own forward applies to its lm_head output (Granite's / logits_scaling, Falcon-H1's
    * lm_head_multiplier, Gemma2's tanh soft-cap, ...). The module that owns the head runs its forward once with every
    other child answering zero hidden states and the head answering zero logits, under a _ChainProbe that follows
    those logits to the forward's result. NotImplementedError unless that result is the end of one chain of ops on
    them (a further submodule, an in-place write or a fork is not)."""
    owner = next((m for m in model.modules() if any(c is head for c in m.children())), None)
    if owner is None:
        raise NotImplementedError("the head is not a submodule of the model")
    V, H = head.weight.shape
    dtype = head.weight.dtype
    from transformers.modeling_outputs import MoeModelOutputWithPast
    zero_states = MoeModelOutputWithPast(last_hidden_state=torch.zeros(1, 1, H, dtype=dtype))
    probe = _ChainProbe()

    def zero_logits(*_, **__):
        z = torch.zeros(1, 1, V, dtype=dtype)
        probe.start(z)
        return z

    stand_ins = {c: (zero_logits if c is head else (lambda *_, **__: zero_states)) for c in owner.children()}
    with _forwards(stand_ins), probe:
        result = type(owner).forward(owner, input_ids=torch.zeros(1, 1, dtype=torch.long), use_cache=False)
    if not probe.lineage or getattr(result, "logits", None) is not probe.lineage[-1]:
        raise NotImplementedError(f"{type(owner).__name__}: its logits are not its lm_head output after one chain of "
                                  "ops; the chunked head cannot reproduce them")
    return probe.ops


_DIV = {torch.Tensor.__truediv__, torch.Tensor.div, torch.div, torch.true_divide, torch.Tensor.true_divide}
_MUL = {torch.Tensor.__mul__, torch.Tensor.__rmul__, torch.Tensor.mul, torch.mul}
_TANH = {torch.tanh, torch.Tensor.tanh}


def _fused_post(ops: list):
    """The recorded post-head chain as the fused epilogue's transform z' = post * tanh(pre * z) (one tanh)
    or post * pre * z (scalar scales only). Other chains raise NotImplementedError: the fused path has no
    torch fallback."""
    from octopus_amd.head_op import Post
    pre, post, tanh = 1.0, 1.0, False
    for func, args, kwargs in ops:
        others = [a for a in pytree.tree_leaves((args, kwargs)) if a is not _LOGITS]
        scalar = None
        if len(others) == 1 and isinstance(others[0], (int, float)) and not isinstance(others[0], bool):
            scalar = float(others[0])
        if func in _TANH and not others and not tanh:
            tanh = True
        elif func in _DIV and scalar is not None and args and args[0] is _LOGITS and scalar != 0:
            if tanh:
                post /= scalar
            else:
                pre /= scalar
        elif func in _MUL and scalar is not None:
            if tanh:
                post *= scalar
            else:
                pre *= scalar
        else:
            raise NotImplementedError(f"post-head op {getattr(func, '__name__', func)} has no fused HIP epilogue")
    if tanh and post <= 0 or not tanh and pre * post <= 0:
        raise NotImplementedError("post-head logit scale must be positive for the fused HIP epilogue")
    return Post(pre, post, tanh)


def _head_chunk(weight: torch.Tensor, temperature: float, post: list, hidden: torch.Tensor,
                labels: torch.Tensor) -> torch.Tensor:
    """One chunk of the composite path: logits in the input dtype, the model's post-head ops, columns."""
    return _head_columns(_post_head(post, hidden @ weight.T), temperature, labels)


def _head_columns_hip(logits: torch.Tensor, temperature: float, labels: torch.Tensor) -> torch.Tensor:
    from octopus_amd.head_op import head_columns
    return head_columns(logits, temperature, labels)


@_fused(hip=_head_columns_hip)
def _head_columns(logits: torch.Tensor, temperature: float, labels: torch.Tensor) -> torch.Tensor:
    """[n, V] logits -> [n, 2]: fp32 log-softmax of logits / T at the label, and the entropy (detached)."""
    s = logits.float() / temperature
    logp = s - torch.logsumexp(s, dim=-1, keepdim=True)
    entropy = (-(logp.exp() * logp).sum(-1)).detach()
    return torch.stack([logp.gather(1, labels.unsqueeze(1)).squeeze(1), entropy], dim=-1)


def _hip_head(self, rows, labels, **kw) -> torch.Tensor:
    from octopus_amd.head_op import fused_head
    return fused_head(rows, self.weight, labels, self.octopus_temperature, _fused_post(self.octopus_post),
                      w_scale=getattr(self, "octopus_w_scale", None), **kw)


def _chunked_rows(self, rows: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """[n, H] rows, [n] labels -> [n, 2] (logprob, entropy). self.weight is read at each call (FSDP swaps
    in the unsharded weight). HIP: one fused call. CPU: CHUNK rows at a time, each recomputed in backward."""
    if rows.is_cuda:
        return _hip_head(self, rows, labels)

    def chunk(h, y):
        return _head_chunk(self.weight, self.octopus_temperature, self.octopus_post, h, y)

    return torch.cat([checkpoint(chunk, h, y, use_reentrant=False)
                      for h, y in zip(rows.split(CHUNK), labels.split(CHUNK))])


def _scored_rows(self, rows: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """_chunked_rows at the positions self.octopus_scored marks ([n] bool; None: all), exactly 0 elsewhere.
    HIP: the compaction kernel builds the row list on the device (no host sync) and the head gathers its
    rows and labels and writes each output row in place."""
    if self.octopus_scored is None:
        return _chunked_rows(self, rows, labels)
    if rows.is_cuda:
        from octopus_amd.head_op import compact_rows
        idx, count = compact_rows(self.octopus_scored)
        return _hip_head(self, rows, labels, idx=idx, count=count, labels_via_idx=True, scatter=True)
    at = self.octopus_scored.nonzero()[:, 0]
    out = _chunked_rows(self, rows.index_select(0, at), labels.index_select(0, at))
    return out.new_zeros(len(rows), out.shape[1]).index_copy(0, at, out)


def _pair_rows(self):
    """The head as tree_head_output's chunk_fn; on HIP tensors the pair gather runs inside the GEMM."""
    def rows_fn(rows, y):
        return _chunked_rows(self, rows, y)

    rows_fn.octopus_fused_rows = lambda hidden2d, pair_pos, y, count=None: _hip_head(self, hidden2d, y, idx=pair_pos,
                                                                                      count=count)
    return rows_fn


# AReaL's micro-batch keys of the GRPO objective's per-token inputs, which the model's forward receives beside
# input_ids and loss_mask (actor.py:80-91 reads loss_mask there): the advantages (actor.py:293-303), the behaviour
# logprobs (spool.py:29-30) and the proximal logprobs, absent under prox_logp_method reuse_train_logp
# (grpo.yaml:103-118, whose constants GrpoInputs carries). Under ppo_update all of them are rolled onto the position
# that scores each token, as the loss mask is (actor.py:80-91).
GRPO_KEYS = ("advantages", "logprobs", "loss_mask")


def grpo_inputs(kwargs: dict):
    """The GRPO inputs of a micro-batch's model kwargs (head_op.GrpoInputs, flat per position), or None when any of
    GRPO_KEYS is missing (compute_logp's batch, or a forward outside training)."""
    if any(kwargs.get(k) is None for k in GRPO_KEYS):
        return None
    from octopus_amd.head_op import GrpoInputs
    prox = kwargs.get("prox_logp")
    return GrpoInputs(adv=kwargs["advantages"].reshape(-1), old=kwargs["logprobs"].reshape(-1),
                      prox=None if prox is None else prox.reshape(-1), mask=kwargs["loss_mask"].reshape(-1))


def _bound_grpo(self, hidden: torch.Tensor, n_flat: int):
    """The micro-batch's GRPO inputs when this call takes the fused GRPO step: HIP tensors, a gradient asked for,
    inputs bound for n_flat positions and the step switched on (head.octopus_grpo_step)."""
    grpo = getattr(self, "octopus_grpo", None)
    if grpo is None or not getattr(self, "octopus_grpo_step", True) or not hidden.is_cuda:
        return None
    if not torch.is_grad_enabled() or not (hidden.requires_grad or self.weight.requires_grad):
        return None
    return grpo if grpo.adv.numel() == n_flat else None


def _chunked_head_forward(self, hidden: torch.Tensor) -> torch.Tensor:
    """[1, T, H] hidden -> [1, T_flat, 2]. The model's own post-head ops then leave the output as it is
    (they ran inside the head). A tree micro-batch (self.octopus_tree) scores its label pairs.

    With the micro-batch's GRPO inputs bound (bind_head's pre-hook) and a gradient asked for, HIP tensors take the
    fused GRPO step (head_op.grpo_bound_head / grpo_bound_tree_head): the same columns, whose backward only scales the
    gradients the step computed when the trainer's loss is the GRPO objective, and adds the recompute backward of any
    other part of dL/dlogprob."""
    tree = self.octopus_tree
    if tree is not None:
        grpo = _bound_grpo(self, hidden, tree.flat_pair.numel())
        if grpo is not None:
            from octopus_amd.head_op import grpo_bound_tree_head
            out = grpo_bound_tree_head(hidden, self.weight, tree, self.octopus_temperature, grpo,
                                       post=_fused_post(self.octopus_post), w_scale=getattr(self, "octopus_w_scale",
                                                                                           None))
        else:
            out = tree_head_output(_pair_rows(self), hidden, tree)
    else:
        rows = hidden.reshape(-1, hidden.shape[-1])
        grpo = _bound_grpo(self, hidden, rows.shape[0])
        if grpo is not None:
            from octopus_amd.head_op import compact_rows, grpo_bound_head
            kw = {}
            if self.octopus_scored is not None:
                kw["idx"], kw["count"] = compact_rows(self.octopus_scored)
            out = grpo_bound_head(rows, self.weight, self.octopus_labels, self.octopus_temperature, grpo,
                                  post=_fused_post(self.octopus_post), w_scale=getattr(self, "octopus_w_scale", None),
                                  **kw)
        else:
            out = _scored_rows(self, rows, self.octopus_labels)
        out = out.reshape(*hidden.shape[:-1], 2)
    return _skipping(out, len(self.octopus_post))


def bind_head(model, temperature: float):
    """Install the chunked head as the model's lm_head forward at this temperature, with the model's own
    post-head ops applied to the logits before the softmax. Returns the head module.

    Also installs a forward pre-hook on the model (once; a later bind_head replaces it) that binds each call's GRPO
    inputs from its kwargs to head.octopus_grpo (grpo_inputs: None unless the micro-batch carries them), as the
    actor's own pre-hook binds the labels (actor.py:166-171). head.octopus_grpo_step = False keeps the plain route."""
    head = model.get_output_embeddings()
    head.octopus_post = _post_head_ops(model, head)
    head.octopus_temperature = temperature
    head.octopus_scored = None
    head.octopus_grpo = None
    head.forward = types.MethodType(_chunked_head_forward, head)
    old = getattr(head, "_octopus_grpo_hook", None)
    if old is not None:
        old.remove()

    def stash_grpo(_module, _args, kwargs):
        head.octopus_grpo = grpo_inputs(kwargs)

    head._octopus_grpo_hook = model.register_forward_pre_hook(stash_grpo, with_kwargs=True)
    return head
