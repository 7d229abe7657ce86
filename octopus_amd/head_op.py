"""PyTorch custom ops over libocto_head.so: the fused LM-head logprob path on HIP tensors.

    octohead::head_fwd / head_bwd      the fused head (GEMM + online softmax epilogue; recompute backward)
    octohead::columns_fwd / columns_bwd  _head_columns over materialised logits
    octohead::pairs_expand / pairs_grad  tree_head_output's pair -> flat expansion
    octohead::grpo_loss                the GRPO objective's value and dL/dlogp per token

Each op is registered for the "cuda" device type only (HIP tensors on ROCm): a CPU tensor has no kernel
here and raises. All work is queued on the current stream; nothing synchronises with the host.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch
from torch import Tensor

from . import _lib

_DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32,
       torch.float8_e4m3fn: _lib.FP8E4M3}


class Post(NamedTuple):
    """Post-head logit transform z' = post * tanh(pre * z) (tanh) or post * pre * z."""
    pre: float = 1.0
    post: float = 1.0
    tanh: bool = False


def _p(t: Optional[Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _dtype_code(t: Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise NotImplementedError(f"octohead: dtype {t.dtype} has no HIP kernel") from None


def _rows2d(x: Tensor) -> Tensor:
    if x.dim() != 2:
        raise ValueError(f"octohead: expected [rows, d], got {tuple(x.shape)}")
    if x.stride(1) != 1 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _index(t: Optional[Tensor]) -> Optional[Tensor]:
    if t is None:
        return None
    return t.to(torch.int64).contiguous()


def _zeros(like: Tensor) -> Tensor:
    """Zeros of like's shape, dtype and device in the contiguous (row-major) layout the library writes, whatever
    like's own strides."""
    return torch.zeros(like.shape, dtype=like.dtype, device=like.device)


def _empty(like: Tensor) -> Tensor:
    return torch.empty(like.shape, dtype=like.dtype, device=like.device)


def _workspace(nbytes: int, like: Tensor) -> Tensor:
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=like.device)


# Bytes of workspace head_bwd gives the library (None: the size octo_head_workspace_bytes returns, the plan at a
# 2 GiB staging budget). The backward runs the largest plan of row passes and vocabulary chunks that fits it.
BWD_WORKSPACE_BYTES: Optional[int] = None


# ---- fused head ---------------------------------------------------------------------------------

def _gather_flag(rows: Tensor, idx: Optional[Tensor]) -> int:
    """OCTO_WS_GATHER when rows are read through idx from a matrix of 2 GiB or more: the library then gathers the
    compact rows into its workspace (its GEMMs address mapped rows with 32-bit offsets)."""
    if idx is None:
        return 0
    return _lib.WS_GATHER if rows.shape[0] * rows.stride(0) * rows.element_size() >= 0x7fffffff else 0


@torch.library.custom_op("octohead::head_fwd", mutates_args=(), device_types="cuda")
def head_fwd(rows: Tensor, weight: Tensor, w_scale: Optional[Tensor], labels: Tensor, idx: Optional[Tensor],
             count: Optional[Tensor], inv_T: float, pre: float, post: float, use_tanh: bool,
             labels_via_idx: bool, scatter: bool) -> tuple[Tensor, Tensor]:
    """(out, lse): out [n, 2] fp32 = (logprob, entropy) per compact row (n = len(idx) or rows), or
    [rows, 2] with each compact row written at idx[r] and zeros elsewhere (scatter); lse [n, 2] fp32, the
    backward's row state (m2, l2S) with lse = (m2 + l2S) ln 2 (OCTO_LSE_PAIR)."""
    rows, weight = _rows2d(rows), _rows2d(weight)
    labels, idx = _index(labels), _index(idx)
    n_max = idx.numel() if idx is not None else rows.shape[0]
    V, d = weight.shape
    flags = (_lib.ROWS_VIA_IDX if labels_via_idx else 0) | (_lib.OUT_SCATTER if scatter else 0) | _lib.LSE_PAIR
    out = torch.zeros(rows.shape[0] if scatter else n_max, 2, dtype=torch.float32, device=rows.device)
    lse = torch.zeros(n_max, 2, dtype=torch.float32, device=rows.device)
    if n_max == 0:
        return out, lse
    w_code = _dtype_code(weight)
    ws = _workspace(_lib.workspace_bytes(n_max, d, V, w_code, _gather_flag(rows, idx)), rows)
    _lib.call("octo_head_fwd", _p(rows), rows.shape[0], rows.stride(0), _dtype_code(rows),
              _p(weight), weight.stride(0), w_code, _p(w_scale), _p(labels), _p(idx), _p(count),
              n_max, d, V, flags, inv_T, pre, post, int(use_tanh),
              None, None, _p(lse), _p(out), 2, _p(ws), ws.numel(), _stream(rows))
    return out, lse


@head_fwd.register_fake
def _(rows, weight, w_scale, labels, idx, count, inv_T, pre, post, use_tanh, labels_via_idx, scatter):
    n_max = idx.shape[0] if idx is not None else rows.shape[0]
    out = rows.new_empty(rows.shape[0] if scatter else n_max, 2, dtype=torch.float32)
    return out, rows.new_empty(n_max, 2, dtype=torch.float32)


@torch.library.custom_op("octohead::head_fwd_grpo", mutates_args=(), device_types="cuda")
def head_fwd_grpo(rows: Tensor, weight: Tensor, w_scale: Optional[Tensor], labels: Tensor, idx: Optional[Tensor],
                  count: Optional[Tensor], inv_T: float, pre: float, post: float, use_tanh: bool,
                  labels_via_idx: bool, scatter: bool, prox: Optional[Tensor], old: Optional[Tensor], adv: Tensor,
                  mask: Tensor, eps_lo: float, eps_hi: float,
                  reject_upper: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """head_fwd plus the GRPO weight of each compact row (octo_head_fwd_grpo): (out, lse, g, loss) with
    g [n] fp32 = dL/dlogprob of compact row r's token (idx[r], or r), in compact order, ready for head_bwd;
    prox, old, adv, mask are per flat token, as grpo_loss takes them."""
    rows, weight = _rows2d(rows), _rows2d(weight)
    labels, idx = _index(labels), _index(idx)
    n_max = idx.numel() if idx is not None else rows.shape[0]
    V, d = weight.shape
    flags = (_lib.ROWS_VIA_IDX if labels_via_idx else 0) | (_lib.OUT_SCATTER if scatter else 0) | _lib.LSE_PAIR
    out = torch.zeros(rows.shape[0] if scatter else n_max, 2, dtype=torch.float32, device=rows.device)
    lse = torch.zeros(n_max, 2, dtype=torch.float32, device=rows.device)
    g = torch.zeros(n_max, dtype=torch.float32, device=rows.device)
    loss = torch.zeros((), dtype=torch.float32, device=rows.device)
    if n_max == 0:
        return out, lse, g, loss
    f = lambda t: None if t is None else t.float().contiguous().reshape(-1)  # noqa: E731
    prox_, old_, adv_, mask_ = f(prox), f(old), f(adv), f(mask)
    tail = _lib.GrpoTail(_p(prox_), _p(old_), _p(adv_), _p(mask_), adv_.numel(), eps_lo, eps_hi, reject_upper,
                         _p(g), _p(loss))
    w_code = _dtype_code(weight)
    ws = _workspace(_lib.workspace_bytes(n_max, d, V, w_code, _gather_flag(rows, idx)), rows)
    _lib.call("octo_head_fwd_grpo", _p(rows), rows.shape[0], rows.stride(0), _dtype_code(rows),
              _p(weight), weight.stride(0), w_code, _p(w_scale), _p(labels), _p(idx), _p(count),
              n_max, d, V, flags, inv_T, pre, post, int(use_tanh),
              None, None, _p(lse), _p(out), 2, ctypes.byref(tail), _p(ws), ws.numel(), _stream(rows))
    return out, lse, g, loss


@head_fwd_grpo.register_fake
def _(rows, weight, w_scale, labels, idx, count, inv_T, pre, post, use_tanh, labels_via_idx, scatter, prox, old, adv,
      mask, eps_lo, eps_hi, reject_upper):
    n_max = idx.shape[0] if idx is not None else rows.shape[0]
    out = rows.new_empty(rows.shape[0] if scatter else n_max, 2, dtype=torch.float32)
    return (out, rows.new_empty(n_max, 2, dtype=torch.float32), rows.new_empty(n_max, dtype=torch.float32),
            rows.new_empty((), dtype=torch.float32))


@torch.library.custom_op("octohead::head_bwd", mutates_args=(), device_types="cuda")
def head_bwd(rows: Tensor, weight: Tensor, w_scale: Optional[Tensor], labels: Tensor, idx: Optional[Tensor],
             count: Optional[Tensor], lse: Tensor, g: Tensor, inv_T: float, pre: float, post: float,
             use_tanh: bool, labels_via_idx: bool, need_rows: bool, need_weight: bool) -> tuple[Tensor, Tensor]:
    """(grad_rows [rows, d] in rows' dtype, grad_weight [V, d] in weight's dtype) for g = dL/dlogprob per
    compact row; an output not asked for is an empty tensor."""
    rows2, weight2 = _rows2d(rows), _rows2d(weight)
    labels, idx = _index(labels), _index(idx)
    n_max = idx.numel() if idx is not None else rows2.shape[0]
    V, d = weight2.shape
    grad_rows = _zeros(rows) if need_rows else rows.new_empty(0)
    grad_w = weight.new_empty(0)
    if n_max == 0 or not (need_rows or need_weight):
        if need_weight:
            grad_w = _zeros(weight)
        return grad_rows, grad_w
    w_code = _dtype_code(weight2)
    flags = (_lib.ROWS_VIA_IDX if labels_via_idx else 0) | _lib.LSE_PAIR
    ws_flags = (_lib.WS_BACKWARD | (0 if need_weight else _lib.WS_NO_GRADW) | (0 if need_rows else _lib.WS_NO_GRADH)
                | _gather_flag(rows2, idx))
    nbytes = _lib.workspace_bytes(n_max, d, V, w_code, ws_flags)
    if BWD_WORKSPACE_BYTES is not None:
        nbytes = int(BWD_WORKSPACE_BYTES)
    ws = _workspace(nbytes, rows2)
    gh = None
    if need_rows:
        # compact-order rows; scattered (runs of equal idx summed) into grad_rows below
        gh = grad_rows if idx is None else torch.empty(n_max, d, dtype=rows2.dtype, device=rows2.device)
    if need_weight:  # written in the weight's dtype (summed in fp32 inside, rounded once)
        grad_w = torch.empty(V, d, dtype=weight.dtype, device=rows2.device)
    lse_c, g_c = lse.contiguous(), g.contiguous()  # kept alive until the call has queued its kernels
    _lib.call("octo_head_bwd", _p(rows2), rows2.shape[0], rows2.stride(0), _dtype_code(rows2),
              _p(weight2), weight2.stride(0), w_code, _p(w_scale), _p(labels), _p(idx), _p(count),
              n_max, d, V, flags, inv_T, pre, post, int(use_tanh), _p(lse_c),
              _p(g_c), _p(gh), d, _dtype_code(rows2) if need_rows else _lib.F32,
              _p(grad_w if need_weight else None), _dtype_code(grad_w) if need_weight else _lib.F32,
              _p(ws), ws.numel(), _stream(rows2))
    if need_rows and idx is not None:
        _lib.call("octo_rows_scatter", _p(gh), d, _dtype_code(gh), _p(idx), _p(count), n_max, d,
                  _p(grad_rows), grad_rows.stride(0), _dtype_code(grad_rows), 0, _stream(rows2))
    return grad_rows, grad_w


@head_bwd.register_fake
def _(rows, weight, w_scale, labels, idx, count, lse, g, inv_T, pre, post, use_tanh, labels_via_idx,
      need_rows, need_weight):
    return (_empty(rows) if need_rows else rows.new_empty(0),
            _empty(weight) if need_weight else weight.new_empty(0))


# Bytes of workspace head_step_grpo gives the library (None: octo_head_workspace_bytes with OCTO_WS_STEP, the plan at
# a 2 GiB staging budget).
STEP_WORKSPACE_BYTES: Optional[int] = None


@torch.library.custom_op("octohead::head_step_grpo", mutates_args=(), device_types="cuda")
def head_step_grpo(rows: Tensor, weight: Tensor, w_scale: Optional[Tensor], labels: Tensor, idx: Optional[Tensor],
                   count: Optional[Tensor], inv_T: float, pre: float, post: float, use_tanh: bool,
                   labels_via_idx: bool, scatter: bool, prox: Optional[Tensor], old: Optional[Tensor], adv: Tensor,
                   mask: Tensor, eps_lo: float, eps_hi: float, reject_upper: float, need_rows: bool,
                   need_weight: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The GRPO step of the head in one call (octo_head_step_grpo): head_fwd_grpo's (out, lse, g, loss), then
    head_bwd's (grad_rows, grad_weight) of that loss, with the logits computed once per row pass. grad_rows is
    [rows, d] in rows' dtype (compact rows scattered to idx, as head_bwd), grad_weight [V, d] in weight's dtype; an
    output not asked for is an empty tensor."""
    rows2, weight2 = _rows2d(rows), _rows2d(weight)
    labels, idx = _index(labels), _index(idx)
    n_max = idx.numel() if idx is not None else rows2.shape[0]
    V, d = weight2.shape
    dev = rows2.device
    flags = (_lib.ROWS_VIA_IDX if labels_via_idx else 0) | (_lib.OUT_SCATTER if scatter else 0) | _lib.LSE_PAIR
    out = torch.zeros(rows2.shape[0] if scatter else n_max, 2, dtype=torch.float32, device=dev)
    lse = torch.zeros(n_max, 2, dtype=torch.float32, device=dev)
    g = torch.zeros(n_max, dtype=torch.float32, device=dev)
    loss = torch.zeros((), dtype=torch.float32, device=dev)
    grad_rows = _zeros(rows) if need_rows else rows.new_empty(0)
    grad_w = (_zeros(weight) if n_max == 0 else _empty(weight)) if need_weight \
        else weight.new_empty(0)
    if n_max == 0:
        return out, lse, g, loss, grad_rows, grad_w
    f = lambda t: None if t is None else t.float().contiguous().reshape(-1)  # noqa: E731
    prox_, old_, adv_, mask_ = f(prox), f(old), f(adv), f(mask)
    tail = _lib.GrpoTail(_p(prox_), _p(old_), _p(adv_), _p(mask_), adv_.numel(), eps_lo, eps_hi, reject_upper,
                         _p(g), _p(loss))
    w_code = _dtype_code(weight2)
    if need_rows or need_weight:
        ws_flags = (_lib.WS_STEP | (0 if need_weight else _lib.WS_NO_GRADW) | (0 if need_rows else _lib.WS_NO_GRADH)
                    | _gather_flag(rows2, idx))
    else:  # no gradient: the library runs the forward with its GRPO tail, in the forward's workspace
        ws_flags = _gather_flag(rows2, idx)
    nbytes = _lib.workspace_bytes(n_max, d, V, w_code, ws_flags)
    if STEP_WORKSPACE_BYTES is not None and (need_rows or need_weight):
        nbytes = int(STEP_WORKSPACE_BYTES)
    ws = _workspace(nbytes, rows2)
    gh = None
    if need_rows:  # compact-order rows; scattered into grad_rows below
        gh = grad_rows if idx is None else torch.empty(n_max, d, dtype=rows2.dtype, device=dev)
    _lib.call("octo_head_step_grpo", _p(rows2), rows2.shape[0], rows2.stride(0), _dtype_code(rows2),
              _p(weight2), weight2.stride(0), w_code, _p(w_scale), _p(labels), _p(idx), _p(count),
              n_max, d, V, flags, inv_T, pre, post, int(use_tanh),
              None, None, _p(lse), _p(out), 2, ctypes.byref(tail),
              _p(gh), d, _dtype_code(rows2) if need_rows else _lib.F32,
              _p(grad_w if need_weight else None), _dtype_code(grad_w) if need_weight else _lib.F32,
              _p(ws), ws.numel(), _stream(rows2))
    if need_rows and idx is not None:
        _lib.call("octo_rows_scatter", _p(gh), d, _dtype_code(gh), _p(idx), _p(count), n_max, d,
                  _p(grad_rows), grad_rows.stride(0), _dtype_code(grad_rows), 0, _stream(rows2))
    return out, lse, g, loss, grad_rows, grad_w


@head_step_grpo.register_fake
def _(rows, weight, w_scale, labels, idx, count, inv_T, pre, post, use_tanh, labels_via_idx, scatter, prox, old, adv,
      mask, eps_lo, eps_hi, reject_upper, need_rows, need_weight):
    n_max = idx.shape[0] if idx is not None else rows.shape[0]
    out = rows.new_empty(rows.shape[0] if scatter else n_max, 2, dtype=torch.float32)
    return (out, rows.new_empty(n_max, 2, dtype=torch.float32), rows.new_empty(n_max, dtype=torch.float32),
            rows.new_empty((), dtype=torch.float32),
            _empty(rows) if need_rows else rows.new_empty(0),
            _empty(weight) if need_weight else weight.new_empty(0))


@torch.library.custom_op("octohead::head_step_grpo_pairs", mutates_args=(), device_types="cuda")
def head_step_grpo_pairs(rows: Tensor, weight: Tensor, w_scale: Optional[Tensor], pair_label: Tensor,
                         pair_pos: Tensor, pair_count: Optional[Tensor], flat_pair: Tensor, inv_T: float, pre: float,
                         post: float, use_tanh: bool, prox: Optional[Tensor], old: Optional[Tensor], adv: Tensor,
                         mask: Tensor, eps_lo: float, eps_hi: float, reject_upper: float, need_rows: bool,
                         need_weight: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """head_step_grpo over a prefix tree's pair rows (octo_head_step_grpo_pairs): row r is rows[pair_pos[r]] with
    label pair_label[r]; flat token t reads pair row flat_pair[t] (none when negative or at or past the row count);
    prox, old, adv, mask are per flat token. Returns (out [T_flat, 2] per flat token, lse [P, 2], g [P] per pair row,
    loss, grad_rows [rows, d] (pair rows summed into their tree positions), grad_weight)."""
    rows2, weight2 = _rows2d(rows), _rows2d(weight)
    pair_label, pair_pos, flat_pair = _index(pair_label), _index(pair_pos), _index(flat_pair)
    n_pairs = pair_pos.numel()
    n_flat = flat_pair.numel()
    V, d = weight2.shape
    dev = rows2.device
    out = torch.zeros(n_flat, 2, dtype=torch.float32, device=dev)
    lse = torch.zeros(n_pairs, 2, dtype=torch.float32, device=dev)
    g = torch.zeros(n_pairs, dtype=torch.float32, device=dev)
    loss = torch.zeros((), dtype=torch.float32, device=dev)
    grad_rows = _zeros(rows) if need_rows else rows.new_empty(0)
    grad_w = (_zeros(weight) if n_pairs == 0 else _empty(weight)) if need_weight \
        else weight.new_empty(0)
    f = lambda t: None if t is None else t.float().contiguous().reshape(-1)  # noqa: E731
    prox_, old_, adv_, mask_ = f(prox), f(old), f(adv), f(mask)
    tail = _lib.GrpoTail(_p(prox_), _p(old_), _p(adv_), _p(mask_), adv_.numel(), eps_lo, eps_hi, reject_upper,
                         _p(g), _p(loss))
    w_code = _dtype_code(weight2)
    ws_flags = (_lib.WS_STEP | (0 if need_weight else _lib.WS_NO_GRADW) | (0 if need_rows else _lib.WS_NO_GRADH)
                | _gather_flag(rows2, pair_pos))
    nbytes = _lib.workspace_bytes(n_pairs, d, V, w_code, ws_flags)
    if STEP_WORKSPACE_BYTES is not None:
        nbytes = int(STEP_WORKSPACE_BYTES)
    ws = _workspace(nbytes, rows2)
    gh = torch.empty(n_pairs, d, dtype=rows2.dtype, device=dev) if need_rows and n_pairs else None
    _lib.call("octo_head_step_grpo_pairs", _p(rows2), rows2.shape[0], rows2.stride(0), _dtype_code(rows2),
              _p(weight2), weight2.stride(0), w_code, _p(w_scale), _p(pair_label), _p(pair_pos), _p(pair_count),
              n_pairs, d, V, _lib.LSE_PAIR, inv_T, pre, post, int(use_tanh), _p(lse), _p(flat_pair), n_flat,
              _p(out), 2, ctypes.byref(tail), _p(gh), d, _dtype_code(rows2) if need_rows else _lib.F32,
              _p(grad_w if need_weight else None), _dtype_code(grad_w) if need_weight else _lib.F32,
              _p(ws), ws.numel(), _stream(rows2))
    if gh is not None:  # pair rows of one tree position (pair_pos ascending) summed into that position
        _lib.call("octo_rows_scatter", _p(gh), d, _dtype_code(gh), _p(pair_pos), _p(pair_count), n_pairs, d,
                  _p(grad_rows), grad_rows.stride(0), _dtype_code(grad_rows), 0, _stream(rows2))
    return out, lse, g, loss, grad_rows, grad_w


@head_step_grpo_pairs.register_fake
def _(rows, weight, w_scale, pair_label, pair_pos, pair_count, flat_pair, inv_T, pre, post, use_tanh, prox, old, adv,
      mask, eps_lo, eps_hi, reject_upper, need_rows, need_weight):
    n_pairs = pair_pos.shape[0]
    return (rows.new_empty(flat_pair.shape[0], 2, dtype=torch.float32),
            rows.new_empty(n_pairs, 2, dtype=torch.float32), rows.new_empty(n_pairs, dtype=torch.float32),
            rows.new_empty((), dtype=torch.float32),
            _empty(rows) if need_rows else rows.new_empty(0),
            _empty(weight) if need_weight else weight.new_empty(0))


def _step_setup(ctx, inputs, output):
    _out, _lse, _g, _loss, grad_rows, grad_w = output
    # Held on ctx as detached aliases, not saved: an activation-offload pack hook (saved_tensors_hooks) would otherwise
    # copy the [V, d] weight gradient to the host and back, and the aliases carry no grad_fn back to this node.
    ctx.grads = (grad_rows.detach(), grad_w.detach())
    ctx.need = (inputs[-2], inputs[-1])  # need_rows, need_weight: the ops' last two arguments
    ctx.n_inputs = len(inputs)


def _step_backward(ctx, _gout, _glse, _gg, gloss, _ggr, _ggw):
    """The loss is the only differentiable output: its gradients were computed by the forward call, scaled here by
    the incoming gradient of the loss (1 for loss.backward())."""
    grad_rows, grad_w = ctx.grads
    need_rows, need_weight = ctx.need
    # the product in fp32, rounded once to the gradient's dtype (a scale such as 1/3 is not exact in bf16)
    scale = gloss.float()
    gr = (grad_rows.float() * scale).to(grad_rows.dtype) if need_rows and ctx.needs_input_grad[0] else None
    gw = (grad_w.float() * scale).to(grad_w.dtype) if need_weight and ctx.needs_input_grad[1] else None
    return (gr, gw) + (None,) * (ctx.n_inputs - 2)


torch.library.register_autograd("octohead::head_step_grpo", _step_backward, setup_context=_step_setup)
torch.library.register_autograd("octohead::head_step_grpo_pairs", _step_backward, setup_context=_step_setup)


def _head_setup(ctx, inputs, output):
    rows, weight, w_scale, labels, idx, count, inv_T, pre, post, use_tanh, labels_via_idx, scatter = inputs
    # The weight is held by reference, not saved: the backward reads the weight the module holds, as the reference's
    # checkpoint recompute reads self.weight (lm_head.py:116-117), and an activation-offload pack hook
    # (saved_tensors_hooks) never copies the [V, d] matrix to the host and back.
    ctx.weight = weight
    ctx.save_for_backward(rows, w_scale, labels, idx, count, output[1])
    ctx.params = (inv_T, pre, post, use_tanh, labels_via_idx, scatter)


def _head_backward(ctx, gout, _glse):
    rows, w_scale, labels, idx, count, lse = ctx.saved_tensors
    weight = ctx.weight
    inv_T, pre, post, use_tanh, labels_via_idx, scatter = ctx.params
    need_rows, need_weight = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    if need_weight and weight.dtype == torch.float8_e4m3fn:
        raise NotImplementedError("octohead: no gradient for fp8 weights")
    gout = gout.float()
    if scatter:  # g of compact row r is the output gradient at its hidden row idx[r]
        col = gout[:, 0].contiguous()
        idx64 = idx.to(torch.int64).contiguous()
        g = torch.empty(idx.numel(), dtype=torch.float32, device=gout.device)
        _lib.call("octo_gather_f32", _p(col), 1, _p(idx64), _p(count), idx.numel(), _p(g), _stream(gout))
    else:
        g = gout[:, 0].contiguous()
    grad_rows, grad_w = head_bwd(rows, weight, w_scale, labels, idx, count, lse, g, inv_T, pre, post, use_tanh,
                                 labels_via_idx, need_rows, need_weight)
    return (grad_rows if need_rows else None, grad_w if need_weight else None,
            None, None, None, None, None, None, None, None, None, None)


torch.library.register_autograd("octohead::head_fwd", _head_backward, setup_context=_head_setup)


def fused_head(rows: Tensor, weight: Tensor, labels: Tensor, temperature: float, post: Post = Post(), *,
               idx: Optional[Tensor] = None, count: Optional[Tensor] = None, labels_via_idx: bool = False,
               scatter: bool = False, w_scale: Optional[Tensor] = None) -> Tensor:
    """[n, 2] (logprob, entropy) of rows[idx] (or all rows) against weight, differentiable in rows and weight;
    with scatter, a [rows, 2] tensor holding each compact row at idx[r] and 0 elsewhere."""
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    out, _ = head_fwd(rows, weight, w_scale, labels, idx, count, 1.0 / float(temperature), float(post.pre),
                      float(post.post), bool(post.tanh), labels_via_idx, scatter)
    return out


def fused_grpo_head(rows: Tensor, weight: Tensor, labels: Tensor, temperature: float, adv: Tensor, mask: Tensor, *,
                    prox: Optional[Tensor] = None, old: Optional[Tensor] = None, post: Post = Post(),
                    idx: Optional[Tensor] = None, count: Optional[Tensor] = None, labels_via_idx: bool = False,
                    scatter: bool = False, w_scale: Optional[Tensor] = None, eps_lo: float = 0.2,
                    eps_hi: float = 0.28, reject_upper: float = 5.0) -> tuple[Tensor, Tensor]:
    """(loss, out): the GRPO objective (grpo_loss's, on the head's logprobs) and fused_head's [n, 2] (logprob,
    entropy) columns, from one octo_head_step_grpo call that also computes the loss's gradients with respect to rows
    and weight (each when it requires grad and grad mode is on); loss.backward() then only scales them. The columns
    carry no gradient: for losses other than this objective, use fused_head. prox, old, adv, mask are per flat
    token (row of `rows`), as grpo_loss takes them. The gradients are held from this call to the backward."""
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    grad_on = torch.is_grad_enabled()
    need_rows = grad_on and rows.requires_grad
    need_weight = grad_on and weight.requires_grad
    out, _lse, _g, loss, _gr, _gw = head_step_grpo(
        rows, weight, w_scale, labels, idx, count, 1.0 / float(temperature), float(post.pre), float(post.post),
        bool(post.tanh), labels_via_idx, scatter, prox, old, adv, mask, float(eps_lo), float(eps_hi),
        float(reject_upper), need_rows, need_weight)
    return loss, out.detach()


def fused_grpo_tree_head(hidden: Tensor, weight: Tensor, meta, temperature: float, adv: Tensor, mask: Tensor, *,
                         prox: Optional[Tensor] = None, old: Optional[Tensor] = None, post: Post = Post(),
                         w_scale: Optional[Tensor] = None, eps_lo: float = 0.2, eps_hi: float = 0.28,
                         reject_upper: float = 5.0) -> tuple[Tensor, Tensor]:
    """fused_grpo_head over a prefix tree (the tree_head_output form, prefix_tree.py:416-421): hidden [1, T_tree, H]
    or [T_tree, H], the head run on the tree's deduplicated (position, label) pair rows of `meta` (a TreeMeta, pairs
    built on the host or on the device), the GRPO objective over the flat tokens (prox, old, adv, mask per flat
    token). Returns (loss, out [1, T_flat, 2]): each flat token's (logprob, entropy), 0 where it has no pair,
    detached; loss.backward() gives hidden and weight their gradients (a pair row's summed over its flat tokens)."""
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    rows = hidden[0] if hidden.dim() == 3 else hidden
    grad_on = torch.is_grad_enabled()
    need_rows = grad_on and hidden.requires_grad
    need_weight = grad_on and weight.requires_grad
    out, _lse, _g, loss, _gr, _gw = head_step_grpo_pairs(
        rows, weight, w_scale, meta.pair_label, meta.pair_pos, meta.pair_count, meta.flat_pair,
        1.0 / float(temperature), float(post.pre), float(post.post), bool(post.tanh), prox, old, adv, mask,
        float(eps_lo), float(eps_hi), float(reject_upper), need_rows, need_weight)
    return loss, out.detach().unsqueeze(0)


# ---- the bound GRPO step: the fused step behind the head's ordinary columns ---------------------------------

# The part of the incoming dL/dlogprob that is not a multiple of the bound step's own GRPO weight, relative (L2) to
# the whole, at or below which the backward only scales the gradients its forward computed. The gradients are linear
# in dL/dlogprob, so leaving that part out changes them by about the same relative amount: 1e-5, far below bf16's
# 2^-9 rounding of dz. Two fp32 evaluations of one objective in a different operation order differ by a few ulp
# (about 1e-7 relative).
SPEC_TOL = 1e-5


class GrpoInputs(NamedTuple):
    """The micro-batch's GRPO inputs per flat position (the head's rows): advantages, behaviour logprobs (`old`),
    proximal logprobs (`prox`; None: the head's own logprobs, reuse_train_logp) and the loss mask, with AReaL's
    constants (grpo.yaml:103-118)."""
    adv: Tensor
    old: Optional[Tensor]
    prox: Optional[Tensor]
    mask: Tensor
    eps_lo: float = 0.2
    eps_hi: float = 0.28
    reject_upper: float = 5.0


def _fit(src: Tensor, idx: Optional[Tensor], g_head: Tensor, count: Optional[Tensor]):
    """(c, rest, count_rest, skip) from octo_grpo_fit: the incoming dL/dlogprob per compact row, a[r] = src[idx[r], 0]
    (src[r, 0] without idx; 0 past the count), fitted as c times the head's own GRPO weight g_head (least squares);
    rest = a - c g_head; count_rest = 0 and skip [1] int32 = 1 when the rest is negligible (SPEC_TOL), else the count
    and 0, so that the residual backward's kernels end at once. One kernel; everything stays on the device."""
    n = g_head.numel()
    dev = g_head.device
    c = torch.empty(1, dtype=torch.float32, device=dev)
    rest = torch.empty(n, dtype=torch.float32, device=dev)
    count_rest = torch.empty(1, dtype=torch.int32, device=dev)
    skip = torch.empty(1, dtype=torch.int32, device=dev)
    src = src.float().contiguous()
    g_head = g_head.float().contiguous()
    idx_c = None if idx is None else _index(idx)
    _lib.call("octo_grpo_fit", _p(src), src.stride(0), _p(idx_c), _p(g_head), n, _p(count), SPEC_TOL, _p(c),
              _p(rest), _p(count_rest), _p(skip), _stream(g_head))
    return c, rest, count_rest, skip


def _scale_add(held: Tensor, rest: Optional[Tensor], c: Tensor, skip: Optional[Tensor]) -> Tensor:
    """held = c held + rest in place (rest None, or not read while skip is set: held = c held); returns held."""
    if held.numel():
        rest = None if rest is None else rest.contiguous()
        _lib.call("octo_scale_add", _p(held), _p(rest), _dtype_code(held), held.numel(), _p(c), _p(skip),
                  _stream(held))
    return held


class _GrpoBound(torch.autograd.Function):
    """The head's (logprob, entropy) columns from octo_head_step_grpo (or _pairs), which also computes the gradients
    of the GRPO objective on them; the backward fits the incoming dL/dlogprob as c times the step's own weight g
    (_fit), scales the held gradients by c and adds octo_head_bwd's gradients of the rest, whose kernels end at
    once when the rest is negligible. A loss that is the objective (times any constant) costs the forward's one pass
    over the logits; any other loss on the logprob column still gets its exact gradients, at the cost of the
    recompute backward. The entropy column carries no gradient (lm_head.py:111)."""

    @staticmethod
    def forward(ctx, rows, weight, w_scale, labels, idx, count, flat_pair, inv_T, post, grpo):
        need_rows, need_weight = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        pre, pst, tanh = float(post.pre), float(post.post), bool(post.tanh)
        if flat_pair is None:  # compact rows: row r is rows[idx[r]] (or r), out scattered to the rows
            out, lse, g, _loss, grad_rows, grad_w = head_step_grpo(
                rows, weight, w_scale, labels, idx, count, inv_T, pre, pst, tanh, idx is not None, idx is not None,
                grpo.prox, grpo.old, grpo.adv, grpo.mask, grpo.eps_lo, grpo.eps_hi, grpo.reject_upper, need_rows,
                need_weight)
        else:  # tree pair rows: row r is rows[idx[r]] with label labels[r]; out per flat token
            out, lse, g, _loss, grad_rows, grad_w = head_step_grpo_pairs(
                rows, weight, w_scale, labels, idx, count, flat_pair, inv_T, pre, pst, tanh, grpo.prox, grpo.old,
                grpo.adv, grpo.mask, grpo.eps_lo, grpo.eps_hi, grpo.reject_upper, need_rows, need_weight)
        # the gradients are held on ctx, not saved: an activation-offload pack hook would copy [V, d] to the host
        ctx.held = (grad_rows.detach(), grad_w.detach())
        ctx.weight = weight
        ctx.save_for_backward(rows, w_scale, labels, idx, count, flat_pair, lse, g)
        ctx.params = (inv_T, pre, pst, tanh)
        return out

    @staticmethod
    def backward(ctx, gout):
        rows, w_scale, labels, idx, count, flat_pair, lse, g_head = ctx.saved_tensors
        inv_T, pre, pst, tanh = ctx.params
        if ctx.held is None:  # the held gradients were scaled in place and handed to autograd by the first backward
            raise RuntimeError("the bound GRPO head's backward runs once per forward (retain_graph is not supported)")
        grad_rows, grad_w = ctx.held
        ctx.held = None
        need_rows, need_weight = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        n = g_head.numel()
        gout = gout.float().contiguous()
        if flat_pair is not None:  # per pair row: the sum over its flat tokens
            c, rest, count_rest, skip = _fit(pairs_grad(gout, flat_pair, n), None, g_head, count)
        else:  # per compact row: the output gradient at its row idx[r] (row r without idx; 0 past the count)
            c, rest, count_rest, skip = _fit(gout, idx, g_head, count)
        # the held gradients times c (no work at all when c is 1), then the rest's gradients added into them by the
        # recompute backward (its kernels end at once, and add nothing, when the rest is negligible)
        if need_weight:
            _scale_add(grad_w, None, c, None)
        if need_rows:
            _scale_add(grad_rows, None, c, None)
        _rest_backward(rows, ctx.weight, w_scale, labels, idx, count_rest, lse, rest, inv_T, pre, pst, tanh,
                       idx is not None and flat_pair is None, grad_rows if need_rows else None,
                       grad_w if need_weight else None, skip)
        return (grad_rows if need_rows else None, grad_w if need_weight else None,
                None, None, None, None, None, None, None, None)


def _rest_backward(rows, weight, w_scale, labels, idx, count, lse, g, inv_T, pre, post, use_tanh, labels_via_idx,
                   grad_rows, grad_w, skip):
    """octo_head_bwd of g over the compact rows below the device count, ADDED into grad_rows ([rows, d], compact
    rows scattered to idx) and grad_w ([V, d], OCTO_GRADW_ACCUMULATE); either may be None. With a count of 0 the
    kernels end at once and nothing is added (skip [1] int32 = 1 then: the scatter's row-wise add reads nothing)."""
    rows2, weight2 = _rows2d(rows), _rows2d(weight)
    labels, idx = _index(labels), _index(idx)
    n_max = idx.numel() if idx is not None else rows2.shape[0]
    V, d = weight2.shape
    need_rows, need_weight = grad_rows is not None, grad_w is not None
    if n_max == 0 or not (need_rows or need_weight):
        return
    w_code = _dtype_code(weight2)
    flags = ((_lib.ROWS_VIA_IDX if labels_via_idx else 0) | _lib.LSE_PAIR
             | (_lib.GRADW_ACCUMULATE if need_weight else 0))
    ws_flags = (_lib.WS_BACKWARD | (0 if need_weight else _lib.WS_NO_GRADW) | (0 if need_rows else _lib.WS_NO_GRADH)
                | _gather_flag(rows2, idx))
    nbytes = _lib.workspace_bytes(n_max, d, V, w_code, ws_flags)
    if BWD_WORKSPACE_BYTES is not None:
        nbytes = int(BWD_WORKSPACE_BYTES)
    ws = _workspace(nbytes, rows2)
    gh = None
    if need_rows:  # compact rows; without idx, rows past the count are added as they are: zeros
        gh = (torch.empty if idx is not None else torch.zeros)(n_max, d, dtype=rows2.dtype, device=rows2.device)
    lse_c, g_c = lse.contiguous(), g.contiguous()
    _lib.call("octo_head_bwd", _p(rows2), rows2.shape[0], rows2.stride(0), _dtype_code(rows2),
              _p(weight2), weight2.stride(0), w_code, _p(w_scale), _p(labels), _p(idx), _p(count),
              n_max, d, V, flags, inv_T, pre, post, int(use_tanh), _p(lse_c),
              _p(g_c), _p(gh), d, _dtype_code(rows2) if need_rows else _lib.F32,
              _p(grad_w), _dtype_code(grad_w) if need_weight else _lib.F32,
              _p(ws), ws.numel(), _stream(rows2))
    if need_rows:
        if idx is not None:  # rows of one idx summed in fp32, added to grad_rows; nothing past the count
            _lib.call("octo_rows_scatter", _p(gh), d, _dtype_code(gh), _p(idx), _p(count), n_max, d,
                      _p(grad_rows), grad_rows.stride(0), _dtype_code(grad_rows), 1, _stream(rows2))
        else:  # compact row r is row r: grad_rows += gh (gh not read while skip is set)
            one = torch.ones(1, dtype=torch.float32, device=rows2.device)
            _scale_add(grad_rows, gh, one, skip)


def grpo_bound_head(rows: Tensor, weight: Tensor, labels: Tensor, temperature: float, grpo: GrpoInputs, *,
                    post: Post = Post(), idx: Optional[Tensor] = None, count: Optional[Tensor] = None,
                    w_scale: Optional[Tensor] = None) -> Tensor:
    """fused_head's columns (with idx: [rows, 2], each compact row r at idx[r], 0 elsewhere; labels per row of
    `rows`), computed by the fused GRPO step on grpo's per-row inputs: a loss that is the GRPO objective on the
    logprob column, times any constant, gets its gradients from that one call; any other loss gets them from the
    recompute backward of the difference (_GrpoBound)."""
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    return _GrpoBound.apply(rows, weight, w_scale, labels, idx, count, None, 1.0 / float(temperature), post, grpo)


def grpo_bound_tree_head(hidden: Tensor, weight: Tensor, meta, temperature: float, grpo: GrpoInputs, *,
                         post: Post = Post(), w_scale: Optional[Tensor] = None) -> Tensor:
    """tree_head_output's [1, T_flat, 2] columns over a prefix tree's pair rows (meta: a TreeMeta) from the fused GRPO
    step over those rows (octo_head_step_grpo_pairs), grpo's inputs per flat token; the backward as grpo_bound_head's,
    with each pair row's dL/dlogprob summed over its flat tokens."""
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    rows = hidden[0] if hidden.dim() == 3 else hidden
    out = _GrpoBound.apply(rows, weight, w_scale, meta.pair_label, meta.pair_pos, meta.pair_count, meta.flat_pair,
                           1.0 / float(temperature), post, grpo)
    return out.unsqueeze(0)


# ---- _head_columns over materialised logits ------------------------------------------------------

@torch.library.custom_op("octohead::columns_fwd", mutates_args=(), device_types="cuda")
def columns_fwd(logits: Tensor, labels: Tensor, inv_T: float) -> tuple[Tensor, Tensor]:
    logits = _rows2d(logits)
    labels = _index(labels)
    n, V = logits.shape
    out = torch.empty(n, 2, dtype=torch.float32, device=logits.device)
    lse = torch.empty(n, 2, dtype=torch.float32, device=logits.device)  # row state (m2, l2S)
    _lib.call("octo_columns_fwd", _p(logits), logits.stride(0), _dtype_code(logits), _p(labels), n, V, inv_T,
              _p(out), _p(lse), _stream(logits))
    return out, lse


@columns_fwd.register_fake
def _(logits, labels, inv_T):
    return logits.new_empty(logits.shape[0], 2, dtype=torch.float32), logits.new_empty(logits.shape[0], 2,
                                                                                        dtype=torch.float32)


@torch.library.custom_op("octohead::columns_bwd", mutates_args=(), device_types="cuda")
def columns_bwd(logits: Tensor, labels: Tensor, inv_T: float, lse: Tensor, g: Tensor) -> Tensor:
    logits = _rows2d(logits)
    labels = _index(labels)
    n, V = logits.shape
    dl = torch.empty_like(logits)
    lse, g = lse.contiguous(), g.contiguous()  # bound here: a temporary's block could be reused before the call
    for r0 in range(0, n, 65535):
        r1 = min(n, r0 + 65535)
        _lib.call("octo_columns_bwd", _p(logits[r0:r1]), logits.stride(0), _dtype_code(logits), _p(labels[r0:r1]),
                  r1 - r0, V, inv_T, _p(lse[r0:r1]), _p(g[r0:r1]), _p(dl[r0:r1]), dl.stride(0), _stream(logits))
    return dl


@columns_bwd.register_fake
def _(logits, labels, inv_T, lse, g):
    return torch.empty_like(logits)


def _columns_setup(ctx, inputs, output):
    logits, labels, inv_T = inputs
    ctx.save_for_backward(logits, labels, output[1])
    ctx.inv_T = inv_T


def _columns_backward(ctx, gout, _glse):
    logits, labels, lse = ctx.saved_tensors
    g = gout[:, 0].float().contiguous()  # the entropy column is detached
    return columns_bwd(logits, labels, ctx.inv_T, lse, g), None, None


torch.library.register_autograd("octohead::columns_fwd", _columns_backward, setup_context=_columns_setup)


def head_columns(logits: Tensor, temperature: float, labels: Tensor) -> Tensor:
    return columns_fwd(logits, labels, 1.0 / float(temperature))[0]


# ---- pair expansion ------------------------------------------------------------------------------

@torch.library.custom_op("octohead::pairs_expand", mutates_args=(), device_types="cuda")
def pairs_expand(pairs: Tensor, flat_pair: Tensor) -> Tensor:
    pairs = pairs.float().contiguous()
    fp = _index(flat_pair)
    P, C = pairs.shape
    out = torch.empty(fp.numel(), C, dtype=torch.float32, device=pairs.device)
    _lib.call("octo_pairs_expand", _p(pairs), P, C, _p(fp), fp.numel(), _p(out), _stream(pairs))
    return out


@pairs_expand.register_fake
def _(pairs, flat_pair):
    return pairs.new_empty(flat_pair.shape[0], pairs.shape[1], dtype=torch.float32)


@torch.library.custom_op("octohead::pairs_grad", mutates_args=(), device_types="cuda")
def pairs_grad(grad: Tensor, flat_pair: Tensor, P: int) -> Tensor:
    grad = grad.float().contiguous()
    fp = _index(flat_pair)
    T, C = grad.shape
    out = torch.empty(P, C, dtype=torch.float32, device=grad.device)
    _lib.call("octo_pairs_grad", _p(grad), T, C, _p(fp), P, _p(out), _stream(grad))
    return out


@pairs_grad.register_fake
def _(grad, flat_pair, P):
    return grad.new_empty(P, grad.shape[1], dtype=torch.float32)


def _pairs_setup(ctx, inputs, output):
    pairs, flat_pair = inputs
    ctx.save_for_backward(flat_pair)
    ctx.P = pairs.shape[0]


def _pairs_backward(ctx, gout):
    (flat_pair,) = ctx.saved_tensors
    return pairs_grad(gout, flat_pair, ctx.P), None


torch.library.register_autograd("octohead::pairs_expand", _pairs_backward, setup_context=_pairs_setup)


# ---- masked-row compaction -----------------------------------------------------------------------

def label_pairs(flat: Tensor, cu: Tensor, flat_to_tree: Tensor, T_tree: int, scored: Optional[Tensor] = None,
                none_as_count: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The label pairs of prefix_tree.py:156-166 on the device: (pair_pos [T_flat], pair_label [T_flat],
    flat_pair [T_flat], count [2] int32), with count[0] = P pairs in pair_pos / pair_label[:P], sorted by
    (tree position, label); flat_pair = -1 (none_as_count: P) where a position has no pair; count[1] = asks
    whose tree position lay outside [0, T_tree) (0 for a valid tree). No host synchronisation."""
    dev = flat.device
    flat = _index(flat.reshape(-1))
    f2t = _index(flat_to_tree.reshape(-1))
    cu = _index(cu.reshape(-1).to(dev))
    T = flat.numel()
    if f2t.numel() != T:
        raise ValueError(f"label_pairs: flat_to_tree has {f2t.numel()} entries for {T} flat positions")
    sc = None
    if scored is not None:
        sc = scored.reshape(-1)
        if sc.numel() != T:
            raise ValueError(f"label_pairs: scored has {sc.numel()} entries for {T} flat positions")
        sc = (sc != 0).contiguous().view(torch.uint8) if sc.dtype != torch.uint8 else sc.contiguous()
    nbytes = ctypes.c_size_t(0)
    _lib.call("octo_label_pairs_workspace_bytes", T, int(T_tree), ctypes.byref(nbytes))
    ws = _workspace(nbytes.value, flat)
    pair_pos = torch.empty(T, dtype=torch.int64, device=dev)
    pair_label = torch.empty(T, dtype=torch.int64, device=dev)
    flat_pair = torch.empty(T, dtype=torch.int64, device=dev)
    count = torch.empty(2, dtype=torch.int32, device=dev)
    _lib.call("octo_label_pairs", _p(flat), T, _p(cu), cu.numel() - 1, _p(f2t), int(T_tree), _p(sc), _p(pair_pos),
              _p(pair_label), _p(flat_pair), _p(count), _lib.PAIRS_NONE_AS_COUNT if none_as_count else 0, _p(ws),
              ws.numel(), _stream(flat))
    return pair_pos, pair_label, flat_pair, count


def quantise_fp8_rows(weight: Tensor) -> tuple[Tensor, Tensor]:
    """(q [V, d] torch.float8_e4m3fn, scale [V] fp32) of a [V, d] bf16 / f16 / fp32 weight: the head's fp8 weight
    format, scale = max(row absmax / 448, 1e-12), q = the quotient weight / scale rounded to e4m3 (nearest even)."""
    w = weight.contiguous()
    V, d = w.shape
    q = torch.empty(V, d, dtype=torch.float8_e4m3fn, device=w.device)
    scale = torch.empty(V, dtype=torch.float32, device=w.device)
    _lib.call("octo_quantise_fp8_rows", _p(w), w.stride(0), _dtype_code(w), V, d, _p(q), d, _p(scale), _stream(w))
    return q, scale


def compact_rows(mask: Tensor) -> tuple[Tensor, Tensor]:
    """(idx [n] int64, count [1] int32): idx[:count] = positions of the true entries, ascending, as
    mask.nonzero()[:, 0]; count stays on the device (no host synchronisation)."""
    m = mask.reshape(-1)
    if m.dtype != torch.bool and m.dtype != torch.uint8:
        m = m != 0
    m = m.contiguous().view(torch.uint8)
    idx = torch.empty(m.numel(), dtype=torch.int64, device=m.device)
    count = torch.empty(1, dtype=torch.int32, device=m.device)
    _lib.call("octo_compact_rows", _p(m), m.numel(), _p(idx), _p(count), _stream(m))
    return idx, count


# ---- GRPO objective ------------------------------------------------------------------------------

@torch.library.custom_op("octohead::grpo_loss", mutates_args=(), device_types="cuda")
def grpo_loss(logp: Tensor, prox: Optional[Tensor], old: Optional[Tensor], adv: Tensor, mask: Tensor,
              eps_lo: float, eps_hi: float, reject_upper: float) -> tuple[Tensor, Tensor]:
    """(loss [] fp32, g [n] fp32 = dloss/dlogp)."""
    f = lambda t: None if t is None else t.float().contiguous().reshape(-1)  # noqa: E731
    logp_, prox_, old_, adv_, mask_ = f(logp), f(prox), f(old), f(adv), f(mask)
    n = logp_.numel()
    g = torch.empty(n, dtype=torch.float32, device=logp.device)
    loss = torch.empty((), dtype=torch.float32, device=logp.device)
    ws = _workspace(_lib.grpo_workspace_bytes(), logp_)
    _lib.call("octo_grpo_grad", _p(logp_), _p(prox_), _p(old_), _p(adv_), _p(mask_), n, eps_lo, eps_hi,
              reject_upper, _p(g), _p(loss), _p(ws), ws.numel(), _stream(logp_))
    return loss, g.reshape(logp.shape)


@grpo_loss.register_fake
def _(logp, prox, old, adv, mask, eps_lo, eps_hi, reject_upper):
    return logp.new_empty((), dtype=torch.float32), torch.empty_like(logp, dtype=torch.float32)


def _grpo_setup(ctx, inputs, output):
    ctx.save_for_backward(output[1])
    ctx.dtype = inputs[0].dtype


def _grpo_backward(ctx, gloss, _gg):
    (g,) = ctx.saved_tensors
    return (g * gloss).to(ctx.dtype), None, None, None, None, None, None, None


torch.library.register_autograd("octohead::grpo_loss", _grpo_backward, setup_context=_grpo_setup)
