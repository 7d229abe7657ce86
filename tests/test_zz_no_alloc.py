"""octo_head_fwd_noalloc, the forward that allocates nothing (its workspace is a device array inside the library),
through the C ABI against octo_head_fwd with a caller workspace on the same inputs: two calls in a row, the second
smaller and through the compaction map, must give the same bits; a size beyond the array's 64 MiB is refused
before anything is queued; and the second call changes the device's free memory by nothing."""

import ctypes

import pytest
import torch

from octopus_amd import _lib, head_op
from oracle import head as ohead

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _inputs(n, d, V, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g)
    h = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    W = (torch.randn(V, d, generator=g) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, V, (n,), generator=g)
    return h.to(DEV), W.to(DEV), y.to(DEV)


def _args(h, W, y, idx, count, n_max, flags, inv_T, lse, out):
    V, d = W.shape
    return (_ptr(h), h.shape[0], h.stride(0), _lib.BF16, _ptr(W), W.stride(0), _lib.BF16, None, _ptr(y), _ptr(idx),
            _ptr(count), n_max, d, V, flags, inv_T, 1.0, 1.0, 0, None, None, _ptr(lse), _ptr(out), 2)


def _both(h, W, y, inv_T, idx=None, count=None):
    """(out, lse) of octo_head_fwd with a torch workspace, then of octo_head_fwd_noalloc, on the same inputs."""
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    n_max = idx.numel() if idx is not None else h.shape[0]
    V, d = W.shape
    flags = _lib.LSE_PAIR | ((_lib.ROWS_VIA_IDX | _lib.OUT_SCATTER) if idx is not None else 0)
    rows_out = h.shape[0]
    res = []
    for noalloc in (False, True):
        out = torch.zeros(rows_out, 2, device=DEV)
        lse = torch.zeros(n_max, 2, device=DEV)
        args = _args(h, W, y, idx, count, n_max, flags, inv_T, lse, out)
        if noalloc:
            free0 = torch.cuda.mem_get_info()[0]
            _lib.call("octo_head_fwd_noalloc", *args, st)
            torch.cuda.synchronize()
            free1 = torch.cuda.mem_get_info()[0]
        else:
            ws = torch.empty(_lib.workspace_bytes(n_max, d, V, _lib.BF16, 0), dtype=torch.uint8, device=DEV)
            _lib.call("octo_head_fwd", *args, _ptr(ws), ws.numel(), st)
            torch.cuda.synchronize()
        res.append((out.cpu(), lse.cpu()))
    return res[0], res[1], free0, free1


def test_noalloc_forward_matches_the_workspace_forward_on_two_calls():
    # first call: 4,000 rows, d 1024, V 50,000 (12.5 MB of scratch)
    h, W, y = _inputs(4000, 1024, 50000, seed=91)
    (o_ws, l_ws), (o_na, l_na), _, _ = _both(h, W, y, 1.0 / 0.7)
    assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na)
    lp, ent, _ = ohead.head_forward(h[:64].cpu(), W.cpu(), y[:64].cpu(), 0.7)
    assert (o_na[:64, 0].double() - lp).abs().max() <= 2e-3 and (o_na[:64, 1].double() - ent).abs().max() <= 2e-3
    # second call, smaller: 1,500 of 2,500 rows through the compaction map, d 512, V 20,000, outputs scattered
    h2, W2, y2 = _inputs(2500, 512, 20000, seed=92)
    mask = torch.rand(2500, generator=torch.Generator().manual_seed(93)) < 0.6
    idx, count = head_op.compact_rows(mask.to(DEV))
    (o_ws, l_ws), (o_na, l_na), free0, free1 = _both(h2, W2, y2, 1.0, idx=idx, count=count)
    assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na)
    assert (o_na[~mask] == 0).all() and (o_na[mask] != 0).any(dim=1).all()
    assert free1 == free0  # the call allocated no device memory


def test_noalloc_forward_refuses_sizes_beyond_its_scratch():
    # 8,000 rows at V = 151,936 need 8,000 x 594 x 16 B = 76 MB of partials, above the 64 MiB array
    V, d, n = 151936, 256, 8000
    h = torch.zeros(n, d, dtype=torch.bfloat16, device=DEV)
    W = torch.zeros(V, d, dtype=torch.bfloat16, device=DEV)
    y = torch.zeros(n, dtype=torch.int64, device=DEV)
    out = torch.full((n, 2), 7.0, device=DEV)
    lse = torch.full((n, 2), 7.0, device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("octo_head_fwd_noalloc", *_args(h, W, y, None, None, n, _lib.LSE_PAIR, 1.0, lse, out), st)
    torch.cuda.synchronize()
    assert (out == 7.0).all() and (lse == 7.0).all()  # nothing was queued
