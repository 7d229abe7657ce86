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


def test_ctypes_constants_match_the_header():
    """Every numeric #define OCTO_<NAME> of the header (status codes, element types, flags) has the same value as
    the binding's <NAME>, so no flag reaches the library with another meaning."""
    defines = dict(re.findall(r"^#define\s+OCTO_(\w+)\s+(-?\d+)", open(HEADER).read(), flags=re.M))
    assert len(defines) >= 19
    for name, value in defines.items():
        assert getattr(_lib, name) == int(value), name


GIB = 1 << 30
BUDGET = 2 * GIB  # the backward's default staging budget


def _rows(n):
    """Rows per pass the backward takes for n rows: at most 32,768, balanced over the passes, a multiple of 256."""
    passes = -(-n // 32768)
    return -(-(-(-n // passes)) // 256) * 256


def test_forward_workspace_query():
    V, d = 151936, 2560
    fwd = _lib.workspace_bytes(32768, d, V, _lib.BF16, 0)
    assert 32768 * ((V + 255) // 256) * 16 <= fwd < 32768 * ((V + 255) // 256) * 16 + (1 << 20)
    # fp8 weights are widened to bf16 one vocabulary chunk of at most 256 MiB at a time
    f8 = _lib.workspace_bytes(32768, d, V, _lib.FP8E4M3, 0)
    assert fwd < f8 <= fwd + (256 << 20) + (1 << 20)
    # OCTO_WS_GATHER adds a contiguous copy of the n_max rows read through idx (hidden of 2 GiB or more)
    for flags in (0, _lib.WS_BACKWARD):
        plain = _lib.workspace_bytes(32768, d, V, _lib.BF16, flags)
        assert _lib.workspace_bytes(32768, d, V, _lib.BF16, flags | _lib.WS_GATHER) >= plain + 32768 * d * 2
    assert _lib.workspace_bytes(1000, 4096, V, _lib.FP8E4M3, _lib.WS_GATHER) >= \
        _lib.workspace_bytes(1000, 4096, V, _lib.FP8E4M3, 0) + 1000 * 4096 * 2  # bf16 rows under fp8 weights
    with pytest.raises(ValueError):
        _lib.workspace_bytes(-1, d, V, _lib.BF16, 0)


@pytest.mark.parametrize("n,d,V,w,flags", [
    (24576, 2560, 151936, _lib.BF16, 0),                    # 24,576 scored of 32,768 packed tokens, grad_h + grad_W
    (29491, 4096, 128256, _lib.BF16, 0),                    # d 4096, V 128,256
    (32768, 2560, 151936, _lib.BF16, 0),                    # every one of 32,768 rows scored
    (114688, 2560, 151936, _lib.FP8E4M3, _lib.WS_NO_GRADW),  # fp8 weights, grad_h only, four passes
    (24576, 2560, 151937, _lib.BF16, 0),                    # V not a multiple of 64: W^T staged per chunk
    (24576, 2560, 151936, _lib.F32, 0),                     # fp32: dz in both layouts
])
def test_backward_workspace_stays_within_the_staging_budget(n, d, V, w, flags):
    """The backward's workspace at the default plan is the 2 GiB staging budget (dz of one row pass and vocabulary
    chunk, fp32 grad_h partials across chunks, the chunk's W^T or widened fp8 rows) plus h^T of a pass, the label
    entries, and over several passes with a 16-bit grad_W its fp32 partials [V, d]; no [rows, V] dz exists."""
    ws = _lib.workspace_bytes(n, d, V, w, _lib.WS_BACKWARD | flags)
    P, passes, Vc, chunks = _lib.bwd_plan(n, d, V, w, flags, ws)
    Vp = (V + 255) // 256 * 256
    esz = 4 if w == _lib.F32 else 2
    assert P == _rows(n) and passes == -(-n // P)
    assert Vc % 256 == 0 and chunks == -(-Vp // Vc) and (chunks - 1) * Vc < Vp
    need_gw = not flags & _lib.WS_NO_GRADW
    extra = (d * P * esz if need_gw else 0) + P * 4 + (V * d * 4 if need_gw and passes > 1 and esz == 2 else 0)
    assert ws <= BUDGET + extra + (1 << 20), (ws, extra)
    whole_dz = n * Vp * esz
    assert ws < whole_dz  # the [rows, V] staging of a whole pass would not fit
    # the staging of a chunk fits the budget; the chunk count is the fewest that fit or, with grad_W, up to 3 more when
    # that takes grad_W fewer rounds of tiles
    per_col = P * esz * (1 + (esz == 4 and need_gw)) + (d * esz if (V % 64 or d % 256 or esz == 4) else 0) + \
        (d * 2 if w == _lib.FP8E4M3 else 0)
    assert per_col * Vc + (P * d * 4 if chunks > 1 else 0) <= BUDGET

    def width(c):
        return -(-(-(-Vp // c)) // 256) * 256

    fewest = next(c for c in range(1, Vp // 256 + 1)
                  if per_col * width(c) + (P * d * 4 if c > 1 else 0) <= BUDGET)
    if need_gw:
        assert fewest <= chunks <= fewest + 3
        assert _gradw_rounds(Vp, d, Vc) <= _gradw_rounds(Vp, d, width(fewest))
    else:
        assert chunks == fewest


def _gradw_rounds(Vp, d, Vc):
    """Rounds of 32 tiles per XCD (tiles dealt evenly to 8 XCDs) of grad_W = dz^T . h over the vocabulary chunks."""
    nd = -(-d // 256)
    return sum(-(-(-(-(min(Vc, Vp - v0) // 256) * nd // 8)) // 32) for v0 in range(0, Vp, Vc))


def test_backward_plan_follows_the_workspace():
    """A larger workspace runs fewer chunks, a smaller one more (down to 256-column chunks and 256-row passes);
    below the smallest plan the query refuses with EWORKSPACE."""
    n, d, V = 3000, 256, 5120
    for flags in (0, _lib.WS_NO_GRADW):
        big = _lib.workspace_bytes(n, d, V, _lib.BF16, _lib.WS_BACKWARD | flags)
        assert _lib.bwd_plan(n, d, V, _lib.BF16, flags, big) == (3072, 1, 5120, 1)  # small enough for one chunk
        seen, last = set(), (1, 0)
        for ws in (big, big // 2, big // 4, big // 6, big // 8, 3 << 20, 2 << 20):
            try:
                P, passes, Vc, chunks = _lib.bwd_plan(n, d, V, _lib.BF16, flags, ws)
            except ValueError:  # with grad_W, several passes add fp32 partials [V, d]: nothing fits below one pass
                assert flags == 0 and ws < big // 4
                continue
            assert P * passes >= n > P * (passes - 1) and Vc * chunks >= 5120 > Vc * (chunks - 1)
            assert (passes, chunks) >= last or passes > last[0]  # a smaller workspace never runs fewer pieces
            last = (passes, chunks)
            seen.add((passes > 1, chunks > 1))
        assert (False, True) in seen
        if flags:
            assert (True, True) in seen
    with pytest.raises(ValueError):
        _lib.bwd_plan(n, d, V, _lib.BF16, 0, 1 << 16)


def _gradh_rounds(n, d, p_tiles):
    """grad_h rounds (one long tile per CU, 256 CUs) over the passes of p_tiles x 256 rows covering n rows."""
    nt, nd = -(-n // 256), -(-d // 256)
    passes = -(-nt // p_tiles)
    last = nt - (passes - 1) * p_tiles
    return (passes - 1) * -(-(p_tiles * nd) // 256) + -(-(last * nd) // 256)


@pytest.mark.parametrize("n,d,V,w,flags", [
    (32768, 2560, 151936, _lib.BF16, 0),                     # 32,768 packed rows, grad_h + grad_W: six passes
    (65536, 4096, 128256, _lib.BF16, 0),                     # d 4096, V 128,256: eight passes of 8,192
    (131072, 2560, 151936, _lib.FP8E4M3, _lib.WS_NO_GRADW),  # fp8 weights, grad_h only
    (32768, 2560, 151937, _lib.F16, _lib.WS_NO_GRADW),       # V not a multiple of 64: W^T staged once
])
def test_step_workspace_stays_within_the_staging_budget(n, d, V, w, flags):
    """The fused step's workspace at the default plan: one pass's [rows, V_pad] exponentials (then dz) within the
    2 GiB staging budget, plus that pass's statistics, h^T and label entries, each row's columns (for pair rows), the
    row offsets of the bf16 exponentials with their target dots, dz scales and flagged rows,
    fp32 grad_W partials over several passes (tile-blocked over V rounded up to 256 rows when d is a multiple of 256),
    and once per call the widened fp8 weights and W^T (where grad_h cannot
    read W as stored, or grad_h alone over 16,384 rows or more). Rows per pass: the size up to what the budget holds
    whose passes take the fewest grad_h rounds."""
    ws = _lib.workspace_bytes(n, d, V, w, _lib.WS_STEP | flags)
    P, passes, Vp, one = _lib.bwd_plan(n, d, V, w, _lib.WS_STEP | flags, ws)
    assert Vp == (V + 255) // 256 * 256 and one == 1
    assert P % 256 == 0 and P * Vp * 2 <= BUDGET and passes == -(-n // P)
    need_gw = not flags & _lib.WS_NO_GRADW
    pmax = min(32768, BUDGET // (Vp * 2) // 256 * 256)
    top = min(pmax // 256, -(-n // 256))
    best = min(_gradh_rounds(n, d, p) for p in range(1, top + 1))
    assert _gradh_rounds(n, d, P // 256) == best
    assert all(_gradh_rounds(n, d, p) > best for p in range(P // 256 + 1, top + 1))
    extra = (P * ((V + 255) // 256) * 16 + P * 4 + n * 8 + (d * P * 2 if need_gw else 0) +
             n * 8 + P * 12 + passes * 4 +  # bf16 row offsets: offset and target dot per row, per pass row 3 words
             ((Vp if d % 256 == 0 else V) * d * 4 if need_gw and passes > 1 else 0) +
             (V * d * 2 if w == _lib.FP8E4M3 else 0) +
             (d * Vp * 2 if V % 64 or d % 256 or (not need_gw and n >= 16384) else 0))
    assert P * Vp * 2 <= ws <= P * Vp * 2 + extra + (1 << 20), (ws, extra)
    if n == 131072:
        assert (P, passes) == (6400, 21)  # 21 grad_h rounds, against 38 for 27 x 256 rows
    if (n, d) == (32768, 2560):
        assert (P, passes) == (6400, 6)  # 250 grad_h tiles a pass: one round each


@pytest.mark.parametrize("grads", ["both", "grad_h", "grad_W"])
def test_queried_size_runs_the_default_plan_for_each_gradient_set(grads):
    """The size the query returns for a set of gradients runs that set's plan at the 2 GiB staging budget (not a
    smaller budget's): the step and the backward, at 32,768 rows of d 2560, V 151,936."""
    n, d, V = 32768, 2560, 151936
    Vp = (V + 255) // 256 * 256
    flags = {"both": 0, "grad_h": _lib.WS_NO_GRADW, "grad_W": _lib.WS_NO_GRADH}[grads]
    ws = _lib.workspace_bytes(n, d, V, _lib.BF16, _lib.WS_STEP | flags)
    P, passes, _, _ = _lib.bwd_plan(n, d, V, _lib.BF16, _lib.WS_STEP | flags, ws)
    pmax = BUDGET // (Vp * 2) // 256 * 256
    if grads == "grad_W":  # rows balanced over the fewest passes that fit
        k = -(-n // pmax)
        assert (P, passes) == (-(-(-(-n // k)) // 256) * 256, k) == (6656, 5)
    else:  # the fewest grad_h rounds
        assert (P, passes) == (6400, 6)
    # the backward: the queried size is the least that runs its plan
    bw = _lib.workspace_bytes(n, d, V, _lib.BF16, _lib.WS_BACKWARD | flags)
    plan = _lib.bwd_plan(n, d, V, _lib.BF16, flags, bw)
    assert plan[0] * plan[1] >= n and _lib.bwd_plan(n, d, V, _lib.BF16, flags, bw - 256) != plan


def test_step_plan_follows_the_workspace_and_fp32_falls_back():
    n, d, V = 3000, 256, 5120
    big = _lib.workspace_bytes(n, d, V, _lib.BF16, _lib.WS_STEP)
    assert _lib.bwd_plan(n, d, V, _lib.BF16, _lib.WS_STEP, big) == (3072, 1, 5120, 1)
    last = 1
    for ws in (big, big // 2, big // 4, 8 << 20):
        P, passes, _, _ = _lib.bwd_plan(n, d, V, _lib.BF16, _lib.WS_STEP, ws)
        assert P * passes >= n > P * (passes - 1) and passes >= last
        last = passes
    assert last > 1
    # several passes add the fp32 grad_W partials [V, d] (5 MiB here): below them nothing fits
    with pytest.raises(ValueError):
        _lib.bwd_plan(n, d, V, _lib.BF16, _lib.WS_STEP, 4 << 20)
    assert _lib.bwd_plan(n, d, V, _lib.BF16, _lib.WS_STEP | _lib.WS_NO_GRADW, 4 << 20)[1] > 1
    # fp32 operands run the forward and then the backward in the same workspace
    f32 = _lib.workspace_bytes(n, d, V, _lib.F32, _lib.WS_STEP)
    assert f32 == max(_lib.workspace_bytes(n, d, V, _lib.F32, 0),
                      _lib.workspace_bytes(n, d, V, _lib.F32, _lib.WS_BACKWARD))


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


def test_step_dispatch_checks_before_queueing():
    """octo_head_step_grpo on the host: without a gradient it is the forward (whose workspace check answers), with
    one it needs the step's plan; a missing GRPO tail or lse is refused; nothing is queued in any of these."""
    tail = _lib.GrpoTail(P, None, P, P, 10, 0.2, 0.28, 5.0, P, None)

    def step(gh, gw, ws_bytes=0, tail_=tail, lse=P):
        _lib.call("octo_head_step_grpo", P, 10, 64, _lib.BF16, P, 64, _lib.BF16, None, P, None, None, 10, 64, 100,
                  _lib.LSE_PAIR, 1.0, 1.0, 1.0, 0, None, None, lse, None, 2,
                  ctypes.byref(tail_) if tail_ is not None else None, gh, 64, _lib.BF16, gw, _lib.BF16, None,
                  ws_bytes, None)

    with pytest.raises(ValueError, match="head_fwd: workspace"):
        step(None, None)
    for gh, gw in ((P, None), (None, P), (P, P)):
        with pytest.raises(ValueError, match="head_step_grpo: workspace"):
            step(gh, gw)
    with pytest.raises(ValueError, match="null grpo"):
        step(P, P, tail_=None)
    with pytest.raises(ValueError, match="null lse"):
        step(P, P, lse=None)


def test_step_pairs_checks_before_queueing():
    """octo_head_step_grpo_pairs on the host: labels are per pair row (no idx-based flags), 16-bit operands only, the
    flat-token arrays must be there, and the workspace is the step's; nothing is queued in any of these."""
    tail = _lib.GrpoTail(P, None, P, P, 10, 0.2, 0.28, 5.0, P, None)

    def step(flags=_lib.LSE_PAIR, dtype=_lib.BF16, flat=P, out=P, ld_out=2, pos=P):
        _lib.call("octo_head_step_grpo_pairs", P, 10, 64, dtype, P, 64, dtype, None, P, pos, None, 10, 64, 100, flags,
                  1.0, 1.0, 1.0, 0, P, flat, 10, out, ld_out, ctypes.byref(tail), P, 64, dtype, P, dtype, None, 0,
                  None)

    with pytest.raises(ValueError, match="per pair row"):
        step(flags=_lib.LSE_PAIR | _lib.ROWS_VIA_IDX)
    with pytest.raises(ValueError, match="flat_pair, out_flat or ld_out"):
        step(flat=None)
    with pytest.raises(ValueError, match="flat_pair, out_flat or ld_out"):
        step(ld_out=1)
    with pytest.raises(ValueError, match="null pair_pos"):
        step(pos=None)
    with pytest.raises(NotImplementedError):
        step(dtype=_lib.F32)
    with pytest.raises(ValueError, match="head_step_grpo: workspace"):
        step()


def test_timing_hook_without_launches():
    """The timing hook records nothing until a GEMM is launched, and reading an unknown name is not an error."""
    _lib.call("octo_timing_enable", 1)
    assert _lib.timing_read("gemm_stats") == (0, 0.0)
    assert _lib.timing_read("no_such_kernel") == (0, 0.0)
    _lib.call("octo_timing_enable", 0)
    with pytest.raises(ValueError):
        _lib.call("octo_timing_read", None, None, None)


def test_step_plan_keeps_its_passes_when_the_workspace_lacks_the_optional_w_transpose():
    """grad_h alone over 16,384 rows or more stages W^T by choice; a workspace short of exactly that W^T gets the same
    rows per pass without it, not smaller passes."""
    n, d, V, w, fl = 131072, 2560, 151936, _lib.FP8E4M3, _lib.WS_STEP | _lib.WS_NO_GRADW
    ws = _lib.workspace_bytes(n, d, V, w, fl)
    Vp = (V + 255) // 256 * 256
    full = _lib.bwd_plan(n, d, V, w, fl, ws)
    assert _lib.bwd_plan(n, d, V, w, fl, ws - d * Vp * 2) == full
    small = _lib.workspace_bytes(8192, d, V, w, fl)  # below 16,384 rows: no W^T
    assert _lib.workspace_bytes(16384, d, V, w, fl) - small >= d * Vp * 2
