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

import types

import torch
from torch.utils import _pytree as pytree
from torch.utils.checkpoint import checkpoint

from octopus_amd.rl.prefix_tree import tree_head_output
from octopus_amd.rl.seq_tiles import _fused

CHUNK = 2048  # rows per checkpointed chunk of the CPU composite path (lm_head.py:20)

_LOGITS = object()  # placeholder for the logits inside a recorded post-head op


class _Tail(torch.Tensor):
    """The logits as the model's forward sees them after its lm_head.

    Probing (`chain` set): every op applied to the newest tail is recorded and yields the next tail; an
    in-place op or an op on an older result cannot be replayed and raises NotImplementedError.
    Bound-head output (`skip` > 0): each op the model applies returns the head's output unchanged, `skip`
    times (the ops already ran inside the head, on each chunk's logits)."""
    chain = None
    skip = 0
    out = None

    @classmethod
    def __torch_function__(cls, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        tail = next(a for a in pytree.tree_leaves((args, kwargs)) if isinstance(a, _Tail))
        with torch._C.DisableTorchFunctionSubclass():
            result = func(*args, **kwargs)
        chain = tail.chain
        if chain is not None and (result is None or tail is not chain["last"]):
            what = "in place" if result is None else "on an earlier result"
            raise NotImplementedError(f"post-head logits: {getattr(func, '__name__', func)} {what} "
                                      "cannot be replayed")
        if not isinstance(result, torch.Tensor):  # metadata queries (shape, dtype, ...)
            return result
        if chain is None:
            return _skipping(tail.out, tail.skip - 1)
        chain["ops"].append(pytree.tree_map(lambda a: _LOGITS if isinstance(a, _Tail) else a, (func, args, kwargs)))
        nxt = result.as_subclass(_Tail)
        nxt.chain = chain
        chain["last"] = nxt
        return nxt


def _skipping(out: torch.Tensor, n: int) -> torch.Tensor:
    """out itself when n == 0, else a tail that swallows the next n post-head ops."""
    if n == 0:
        return out
    tail = out.as_subclass(_Tail)
    tail.out, tail.skip = out, n
    return tail


def _post_head(ops: list, logits: torch.Tensor) -> torch.Tensor:
    """Replay recorded post-head ops on logits."""
    for func, args, kwargs in ops:
        args, kwargs = pytree.tree_map(lambda a: logits if a is _LOGITS else a, (args, kwargs))
        logits = func(*args, **kwargs)
    return logits


def _post_head_ops(model, head) -> list:
    """The ops the model's own forward applies to its lm_head output (Granite's / logits_scaling, Falcon-H1's
    * lm_head_multiplier, Gemma2's tanh soft-cap, ...), found by running that forward once with its other
    children stubbed (zero hidden states) and the head returning a recording tensor. Raises
    NotImplementedError unless the returned logits are the end of one chain of ops on the head output."""
    lm = next(m for m in model.modules() if any(c is head for c in m.children()))
    chain: dict = {"ops": [], "last": None}
    V, H = head.weight.shape

    def recording_head(*_, **__):
        tail = torch.zeros(1, 1, V, dtype=head.weight.dtype).as_subclass(_Tail)
        tail.chain = chain
        chain["last"] = tail
        return tail

    from transformers.modeling_outputs import MoeModelOutputWithPast
    hidden = MoeModelOutputWithPast(last_hidden_state=torch.zeros(1, 1, H, dtype=head.weight.dtype))
    stubs = {c: (lambda *_, **__: hidden) for c in lm.children() if c is not head}
    stubs[head] = recording_head
    saved = {c: vars(c).get("forward") for c in stubs}
    try:
        for c, f in stubs.items():
            c.forward = f
        out = type(lm).forward(lm, input_ids=torch.zeros(1, 1, dtype=torch.long), use_cache=False)
    finally:
        for c, f in saved.items():
            if f is None:
                del c.forward
            else:
                c.forward = f
    if chain["last"] is None or out.logits is not chain["last"]:
        raise NotImplementedError(f"{type(lm).__name__}: its logits are not one chain of ops on its lm_head "
                                  "output; the chunked head cannot reproduce them")
    return chain["ops"]


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


def _chunked_head_forward(self, hidden: torch.Tensor) -> torch.Tensor:
    """[1, T, H] hidden -> [1, T_flat, 2]. The model's own post-head ops then leave the output as it is
    (they ran inside the head). A tree micro-batch (self.octopus_tree) scores its label pairs."""
    if self.octopus_tree is not None:
        out = tree_head_output(_pair_rows(self), hidden, self.octopus_tree)
    else:
        out = _scored_rows(self, hidden.reshape(-1, hidden.shape[-1]), self.octopus_labels).reshape(
            *hidden.shape[:-1], 2)
    return _skipping(out, len(self.octopus_post))


def bind_head(model, temperature: float):
    """Install the chunked head as the model's lm_head forward at this temperature, with the model's own
    post-head ops applied to the logits before the softmax. Returns the head module."""
    head = model.get_output_embeddings()
    head.octopus_post = _post_head_ops(model, head)
    head.octopus_temperature = temperature
    head.octopus_scored = None
    head.forward = types.MethodType(_chunked_head_forward, head)
    return head
