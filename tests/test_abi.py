"""The C ABI without a GPU: the library loads, exports every function include/octo_head.h declares, the
ctypes table binds exactly those, and argument checks return their status before anything is queued."""

import ctypes
import os
import re

import pytest

from octopus_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "octo_head.h")


def _declared():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return set(re.findall(r"^\s*(?:int|const char \*)\s*(octo_\w+)\s*\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    assert lib.octo_version().startswith(b"octo_head")


def test_workspace_query():
    V, d = 151936, 2560
    fwd = _lib.workspace_bytes(32768, d, V, _lib.BF16, 0)
    assert fwd >= 32768 * ((V + 255) // 256) * 16
    Vp = (V + 255) // 256 * 256
    # 16-bit, V a multiple of 64 and d of 256: h^T [d, P] and dz token-major [P, V_pad] (grad_W reads it K-major,
    # grad_h reads W K-major as stored)
    bwd = _lib.workspace_bytes(32768, d, V, _lib.BF16, _lib.WS_BACKWARD)
    no_gw = _lib.workspace_bytes(32768, d, V, _lib.BF16, _lib.WS_BACKWARD | _lib.WS_NO_GRADW)
    assert bwd >= (32768 * Vp + d * 32768) * 2 and bwd < (32768 * Vp + d * 32768) * 2 + (1 << 20)
    # without grad_W: dz only
    assert no_gw >= 32768 * Vp * 2 and no_gw < 32768 * Vp * 2 + (1 << 20)
    # other shapes stage W^T [d, V_pad] for grad_h as well
    for V2, d2 in ((151937, 2560), (151936, 2304 + 64)):
        Vp2 = (V2 + 255) // 256 * 256
        bwd2 = _lib.workspace_bytes(32768, d2, V2, _lib.BF16, _lib.WS_BACKWARD)
        full = (d2 * Vp2 + 32768 * Vp2 + d2 * 32768) * 2
        assert full <= bwd2 < full + (1 << 20)
    # OCTO_WS_GATHER adds a contiguous copy of the n_max rows read through idx (hidden of 2 GiB or more)
    for flags in (0, _lib.WS_BACKWARD):
        plain = _lib.workspace_bytes(32768, d, V, _lib.BF16, flags)
        assert _lib.workspace_bytes(32768, d, V, _lib.BF16, flags | _lib.WS_GATHER) >= plain + 32768 * d * 2
    assert _lib.workspace_bytes(1000, 4096, V, _lib.FP8E4M3, _lib.WS_GATHER) >= \
        _lib.workspace_bytes(1000, 4096, V, _lib.FP8E4M3, 0) + 1000 * 4096 * 2  # bf16 rows under fp8 weights
    # one pass takes 65,536 rows; two passes of a 16-bit grad_W keep fp32 partial sums
    one = _lib.workspace_bytes(65536, d, V, _lib.BF16, _lib.WS_BACKWARD)
    two = _lib.workspace_bytes(65536 + 256, d, V, _lib.BF16, _lib.WS_BACKWARD)
    assert two >= one + V * d * 4
    # fp32: W^T [d, V_pad], h^T [d, P] and dz in both layouts
    f32 = _lib.workspace_bytes(32768, d, V, _lib.F32, _lib.WS_BACKWARD)
    assert f32 >= (d * Vp + 2 * 32768 * Vp + d * 32768) * 4
    with pytest.raises(ValueError):
        _lib.workspace_bytes(-1, d, V, _lib.BF16, 0)


P = ctypes.c_void_p(256)  # never dereferenced: every call below fails its host-side checks first


def _fwd(**kw):
    a = dict(h=P, h_rows=10, ldh=64, h_dtype=_lib.BF16, w=P, ldw=64, w_dtype=_lib.BF16, w_scale=None, labels=P,
             idx=None, count=None, n_max=10, d=64, V=100, flags=0, inv_T=1.0, pre=1.0, post=1.0, tanh=0,
             ws=None, ws_bytes=0)
    a.update(kw)
    _lib.call("octo_head_fwd", a["h"], a["h_rows"], a["ldh"], a["h_dtype"], a["w"], a["ldw"], a["w_dtype"],
              a["w_scale"], a["labels"], a["idx"], a["count"], a["n_max"], a["d"], a["V"], a["flags"], a["inv_T"],
              a["pre"], a["post"], a["tanh"], None, None, None, None, 2, a["ws"], a["ws_bytes"], None)


@pytest.mark.parametrize("kw,exc", [
    (dict(d=60, ldh=60, ldw=60), ValueError),                      # d not a multiple of 8
    (dict(h_dtype=_lib.F16), NotImplementedError),                 # hidden / weight dtypes differ
    (dict(w_dtype=_lib.FP8E4M3, h_dtype=_lib.F32), NotImplementedError),
    (dict(w_dtype=_lib.FP8E4M3), ValueError),                      # fp8 without scales
    (dict(inv_T=0.0), ValueError),
    (dict(pre=-1.0), ValueError),
    (dict(flags=_lib.OUT_SCATTER), ValueError),                    # scatter without idx
    (dict(h_rows=5), ValueError),                                  # fewer hidden rows than n_max
    (dict(), ValueError),                                          # no workspace
    (dict(h_dtype=7, w_dtype=7), NotImplementedError),
], ids=["d", "dtypes", "fp8-f32", "fp8-noscale", "T", "scale", "scatter", "rows", "workspace", "dtype"])
def test_head_fwd_argument_checks(kw, exc):
    with pytest.raises(exc):
        _fwd(**kw)
    assert _lib.last_error()


def test_small_entry_point_checks():
    with pytest.raises(ValueError):
        _lib.call("octo_compact_rows", P, -1, P, P, None)
    with pytest.raises(ValueError):
        _lib.call("octo_columns_fwd", P, 10, _lib.BF16, P, 4, 100, 1.0, P, None, None)  # ld < V
    with pytest.raises(ValueError):
        _lib.call("octo_grpo_grad", P, None, None, P, P, 4, 0.2, 0.28, 5.0, P, None, None, 0, None)
    assert _lib.grpo_workspace_bytes() >= 4
    nbytes = ctypes.c_size_t(0)
    _lib.call("octo_label_pairs_workspace_bytes", 131072, 114688, ctypes.byref(nbytes))
    assert nbytes.value >= 131072 * 13 + 114688 * 20
    with pytest.raises(ValueError):
        _lib.call("octo_label_pairs_workspace_bytes", 1 << 31, 5, ctypes.byref(nbytes))
    with pytest.raises(ValueError):  # unknown flag
        _lib.call("octo_label_pairs", P, 7, P, 2, P, 5, None, P, P, P, P, 8, P, 1 << 20, None)
    with pytest.raises(ValueError):  # no workspace
        _lib.call("octo_label_pairs", P, 7, P, 2, P, 5, None, P, P, P, P, 0, None, 0, None)
    fwd = (P, 10, 64, _lib.BF16, P, 64, _lib.BF16, None, P, None, None, 10, 64, 100, 0, 1.0, 1.0, 1.0, 0,
           None, None, None, None, 2)
    with pytest.raises(ValueError):  # no GRPO tail
        _lib.call("octo_head_fwd_grpo", *fwd, None, P, 1 << 30, None)
    tail = _lib.GrpoTail(None, None, None, P, 10, 0.2, 0.28, 5.0, P, None)
    with pytest.raises(ValueError):  # no advantages
        _lib.call("octo_head_fwd_grpo", *fwd, ctypes.byref(tail), P, 1 << 30, None)


def test_timing_hook_without_launches():
    """The timing hook records nothing until a GEMM is launched, and reading an unknown name is not an error."""
    _lib.call("octo_timing_enable", 1)
    assert _lib.timing_read("gemm_stats") == (0, 0.0)
    assert _lib.timing_read("no_such_kernel") == (0, 0.0)
    _lib.call("octo_timing_enable", 0)
    with pytest.raises(ValueError):
        _lib.call("octo_timing_read", None, None, None)
