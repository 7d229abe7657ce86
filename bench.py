"""Benchmark of the fused LM-head logprob path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg3] [--no-cpu-baseline]

A step is one pass of the path over one packed micro-batch, inputs resident in HBM: compaction of the scored rows,
then the head's GRPO step in one call (octo_head_step_grpo), row pass by row pass: the logits GEMM with the softmax
statistics and each element's tile-relative exponential in its epilogue; the merge (logprob, entropy, target gather,
GRPO weight g and loss); the exponentials scaled into dz; the grad_hidden and grad_W GEMMs; row scatter, grad_W to
bf16. --two-call runs the forward and the backward as the autograd route calls them instead (octo_head_fwd_grpo,
then octo_head_bwd, which recomputes the logits); the default run also times that route for context.
Default workload cfg3: N = 32,768 packed tree tokens (an 8,192-token root shared by 12 branches of 2,048,
root masked: 24,576 scored rows), d = 2560, V = 151,936, bf16, T = 1.0 (octopus_amd.workloads).
Prints one JSON line: packed tokens/s; per GEMM kernel, its average launch time from HIP events recorded around
each launch over the timed steps (the library's timing hook) and the MFMA roofline of the dominant one; and the
reference algorithm timed on the host CPU beside it.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import platform
import sys
import time

import numpy as np
import torch

PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s (AMD public spec)
PEAK_F32 = 157.3e12
PEAK_HBM = 8.0e12


def _cpu_model() -> str:
    """The host CPU's model name as lscpu reports it (/proc/cpuinfo when lscpu is missing)."""
    import subprocess
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, scored_rows: int, target_s: float = 4.0) -> dict:
    """The reference algorithm on the host (oracle.baseline: CHUNK-row checkpointed chunks, bf16 GEMMs, fp32
    softmax, checkpoint-recompute backward) with os.cpu_count() threads: one chunk timed first, then k whole
    2048-row chunks (about target_s seconds each run) timed three times, the median scaled to the step's scored rows
    (chunks are independent, so the scaling is linear)."""
    from oracle import baseline
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    one = baseline.time_chunks(cfg.d, cfg.V, 1, cfg.temperature, repeats=1)
    n_chunks = max(1, min(scored_rows // baseline.CHUNK, int(round(target_s / max(one["seconds"], 1e-3)))))
    r = baseline.time_chunks(cfg.d, cfg.V, n_chunks, cfg.temperature, repeats=3)
    step_s = r["seconds"] * scored_rows / r["rows"]
    model = _cpu_model()
    return {"value": cfg.N / step_s, "unit": "tokens/s", "cores": r["threads"], "kind": "port",
            "os_cpu_count": os.cpu_count(), "cpu_model": model,
            "sample": f"{n_chunks} x 2048-row chunks fwd+bwd (bf16, d={cfg.d}, V={cfg.V}), median of 3 runs "
                      f"{r['seconds']:.2f} s, scaled x{scored_rows / r['rows']:.2f} to the step's {scored_rows} "
                      f"scored rows (extrapolated); {r['threads']} threads = os.cpu_count(); host: {model}"}


GEMM_KERNELS = ("gemm_stats", "gemm_dz", "gemm_store_grad_h", "gemm_store_grad_w", "gemm_grads", "dz_scale",
                "ex_fix")
PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def recorded_traffic(kernel: str, workload: str, fused: bool = False, key: str = "traffic"):
    """HBM bytes per launch of `kernel` at `workload` as recorded from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    (line `traffic <kernel>: <bytes>`; with key, `<key> <kernel>: <bytes>`) in profiles/step_kernels_<workload>.md for
    the fused step's launches, in profiles/gemm_kernels_<workload>_counters.md for the two-call route's; None when not
    recorded."""
    path = os.path.join(PROFILES, f"step_kernels_{workload}.md" if fused else f"gemm_kernels_{workload}_counters.md")
    key = f"{key} {kernel}:"
    try:
        for line in open(path):
            if line.startswith(key):
                return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def library_gemms(workload: str, reps: int = 5) -> dict:
    """torch.matmul (hipBLASLt) on the step's four contractions at the workload's scored-row count, bf16 in,
    no epilogue: logits (twice: forward and recompute), dz . W and dz^T . h. Context for the fused kernels'
    MFMA rates; these are not the path."""
    from octopus_amd.workloads import CONFIGS
    cfg = CONFIGS[workload]
    dev = torch.device("cuda", 0)
    n = sum(s for s, scored, _ in cfg.segments if scored)
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(n, cfg.d, device=dev, dtype=torch.bfloat16, generator=g)
    W = torch.randn(cfg.V, cfg.d, device=dev, dtype=torch.bfloat16, generator=g)
    dz = torch.randn(n, cfg.V, device=dev, dtype=torch.bfloat16, generator=g)
    flop = 2 * n * cfg.d * cfg.V
    out = {"workload": workload, "rows": n, "flop_each": flop}
    for name, f in (("logits W.h^T", lambda: W @ h.T), ("grad_h dz.W", lambda: dz @ W),
                    ("grad_W dz^T.h", lambda: dz.T @ h)):
        f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[name] = {"ms": ms, "tflops": flop / ms / 1e9}
    return out


def pairs_bench(workload: str, steps: int, warmup: int) -> dict:
    """The label-pair section of the prefix tree (octo_label_pairs) at a root-plus-branches workload: the
    sequences are root + branch, flattened (T_flat tokens), over the packed tree of N tokens; branch tokens are
    scored. Device time from HIP events over `steps` calls; the host restatement (numpy np.unique, as the
    reference runs it) timed beside it."""
    from octopus_amd import head_op
    from octopus_amd.rl.prefix_tree import build_tree, label_pairs as host_pairs
    from octopus_amd.workloads import CONFIGS
    cfg = CONFIGS[workload]
    root, branches = cfg.segments[0], cfg.segments[1:]
    if root[1] or not all(b[1] for b in branches):
        raise SystemExit(f"--pairs takes a root-plus-branches workload (cfg3, cfg5), not {workload}")
    rng = np.random.default_rng(5)
    r_tok = rng.integers(0, cfg.V, root[0])
    seqs = [np.concatenate([r_tok, rng.integers(0, cfg.V, n)]) for n, _, _ in branches]
    flat = np.concatenate(seqs).astype(np.int64)
    cu = np.array([0, *np.cumsum([len(x) for x in seqs])], dtype=np.int64)
    scored = np.ones(len(flat), dtype=bool)
    for a in cu[:-1]:
        scored[a:a + root[0]] = False
    tree = build_tree(flat, cu, scored=scored)
    dev = torch.device("cuda", 0)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    fd, cud, f2t, sc = t(flat), t(cu), t(tree.flat_to_tree), t(scored)
    T_tree = len(tree.tokens)
    for _ in range(warmup):
        head_op.label_pairs(fd, cud, f2t, T_tree, sc, True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        pos, lab, fp, count = head_op.label_pairs(fd, cud, f2t, T_tree, sc, True)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    P = int(count[0].item())
    assert P == len(tree.pair_pos) and torch.equal(pos[:P].cpu(), torch.from_numpy(tree.pair_pos))
    # algorithmic bytes: flat token, tree position, scored flag read and flat_pair written per flat position;
    # (position, label) written per pair
    T = len(flat)
    alg = T * (8 + 8 + 1 + 8) + P * 16
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < 2.0:
        host_pairs(flat, cu, tree.flat_to_tree, scored)
        reps += 1
    host_s = (time.perf_counter() - t0) / reps
    return {"metric": "label pairs per second (prefix_tree.py:156-166 on the device)", "value": T / (ms / 1e3),
            "unit": "flat tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
            "data": "synthetic (seeded tokens; root prompt unscored, branches scored)",
            "config": {"workload": f"{workload}: {len(seqs)} sequences of root {root[0]} + branch, label pairs",
                       "T_flat": T, "T_tree": T_tree, "pairs": P},
            "roofline": {"kernel": "octo_label_pairs (9 launches)", "bound": "hbm",
                         "achieved": alg / (ms / 1e3) / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                         "frac": alg / (ms / 1e3) / PEAK_HBM, "traffic": None,
                         "per_launch": f"{alg} algorithmic bytes per call (25 B per flat position + 16 B per "
                                       f"pair); the call is launch- and latency-bound at this size"},
            "cpu_baseline": {"value": T / host_s, "unit": "flat tokens/s", "cores": 1, "kind": "port",
                             "sample": f"host label_pairs (numpy np.unique over (position, label)) on the same "
                                       f"{T} flat positions, {reps} runs, {host_s * 1e3:.2f} ms each; host: "
                                       f"{_cpu_model()}"}}


def quantise_bench(workload: str, steps: int, warmup: int) -> dict:
    """The per-row e4m3 weight quantiser (octo_quantise_fp8_rows) on the workload's [V, d] bf16 weight: HIP events
    over `steps` calls, HBM roofline on its algorithmic bytes (weight read once, codes and scales written); the
    torch CPU quantisation of 64 rows timed beside it, scaled to V rows."""
    from octopus_amd import head_op
    from octopus_amd.workloads import CONFIGS, quantise_fp8_rows as torch_quantise
    cfg = CONFIGS[workload]
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(1)
    W = (torch.randn(cfg.V, cfg.d, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    for _ in range(warmup):
        head_op.quantise_fp8_rows(W)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        q, scale = head_op.quantise_fp8_rows(W)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    alg = cfg.V * cfg.d * (2 + 1) + cfg.V * 4
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    sample = W[:4096].cpu()
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < 2.0:
        torch_quantise(sample)
        reps += 1
    host_s = (time.perf_counter() - t0) / reps * cfg.V / sample.shape[0]
    return {"metric": "fp8 e4m3 per-row weight quantisation", "value": cfg.V / (ms / 1e3), "unit": "rows/s",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16 -> e4m3",
            "data": "synthetic (seeded W ~ N(0, 0.02))",
            "config": {"workload": f"{workload} weight [{cfg.V}, {cfg.d}] bf16 -> e4m3 + row scales"},
            "roofline": {"kernel": "quantise_fp8_rows_kernel", "bound": "hbm", "achieved": alg / (ms / 1e3) / 1e9,
                         "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": alg / (ms / 1e3) / PEAK_HBM,
                         "traffic": None,
                         "per_launch": f"{alg} algorithmic bytes (2 B read + 1 B written per weight, 4 B per row "
                                       f"scale)"},
            "cpu_baseline": {"value": cfg.V / host_s, "unit": "rows/s", "cores": threads, "kind": "port",
                             "sample": f"torch CPU quantisation (workloads.quantise_fp8_rows) of 4096 rows, "
                                       f"{reps} runs, scaled to {cfg.V} rows; host: {_cpu_model()}"}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="cfg3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--temperature", type=float, default=0.0,
                    help="run the workload at this temperature instead of its own (low temperatures send most rows "
                         "through the fused step's row-offset rescale)")
    ap.add_argument("--bwd-workspace-mib", type=int, default=0,
                    help="give the backward this much workspace instead of the queried size (its plan of row passes "
                         "and vocabulary chunks follows the workspace)")
    ap.add_argument("--two-call", action="store_true",
                    help="run the forward and the backward as two calls (octo_head_fwd_grpo, octo_head_bwd: the "
                         "autograd route, logits recomputed in the backward) instead of the fused step")
    ap.add_argument("--bound", action="store_true",
                    help="time the bound route instead of the fused step: the head's columns from the fused step "
                         "under autograd, the GRPO objective on them and loss.backward() (the trainer's unchanged call "
                         "path after bind_head)")
    ap.add_argument("--no-context", action="store_true",
                    help="skip the two-call route's timing after the fused step's (profiling runs)")
    ap.add_argument("--hipblaslt", action="store_true",
                    help="only time torch.matmul (hipBLASLt) on the four plain GEMMs of the workload's step, "
                         "without any epilogue, for context; then exit")
    ap.add_argument("--pairs", action="store_true",
                    help="only time the device label-pair section of the prefix tree (octo_label_pairs) at the "
                         "workload's tree against the host numpy restatement; then exit")
    ap.add_argument("--quantise", action="store_true",
                    help="only time the per-row fp8 weight quantiser (octo_quantise_fp8_rows) on the workload's "
                         "weight; then exit")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB three times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against known bytes), then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the LM-head path runs on a single MI355X here (no multi-GPU run)",
              file=sys.stderr)
        return 2
    if args.copy_probe:
        src = torch.ones(args.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_each_way": src.numel() * 4}), flush=True)
        return 0
    if args.quantise:
        print(json.dumps(quantise_bench(args.workload, args.steps, args.warmup)), flush=True)
        return 0
    if args.pairs:
        print(json.dumps(pairs_bench(args.workload, args.steps, args.warmup)), flush=True)
        return 0
    if args.hipblaslt:
        print(json.dumps(library_gemms(args.workload)), flush=True)
        return 0

    from octopus_amd import _lib, head_op
    from octopus_amd.workloads import CONFIGS, make_batch
    if args.bwd_workspace_mib:
        head_op.BWD_WORKSPACE_BYTES = args.bwd_workspace_mib << 20
        head_op.STEP_WORKSPACE_BYTES = args.bwd_workspace_mib << 20

    cfg = CONFIGS[args.workload]
    if args.temperature > 0:
        cfg = dataclasses.replace(cfg, temperature=args.temperature)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.load()
    b = make_batch(cfg, dev)
    h, W, y = b.hidden, b.weight, b.labels
    inv_T = 1.0 / cfg.temperature
    mask_f = b.scored.float()
    need_w = cfg.backward == "full"

    # untimed set-up: the rollout's ("old") logprobs = this policy's + N(0, 0.01)
    idx, count = head_op.compact_rows(b.scored)
    out, _ = head_op.head_fwd(h, W, b.w_scale, y, idx, count, inv_T, 1.0, 1.0, False, True, True)
    old = (out[:, 0] + b.old_noise).contiguous()
    scored_rows = int(count.item())
    torch.cuda.synchronize()

    def forward():
        idx, count = head_op.compact_rows(b.scored)
        out, lse = head_op.head_fwd(h, W, b.w_scale, y, idx, count, inv_T, 1.0, 1.0, False, True, True)
        return idx, count, out, lse

    def forward_grpo():
        # the forward with the GRPO weight dL/dlogprob of each compact row computed in its last kernel (the
        # reference's decoupled objective: proximal logprobs = the forward's own, behaviour weight against the
        # rollout's logprobs, eps 0.2 / 0.28, rejection 5.0), ready for the backward
        idx, count = head_op.compact_rows(b.scored)
        out, lse, g, loss = head_op.head_fwd_grpo(h, W, b.w_scale, y, idx, count, inv_T, 1.0, 1.0, False, True,
                                                  True, None, old, b.adv, mask_f, 0.2, 0.28, 5.0)
        return idx, count, out, lse, g

    def backward(idx, count, lse, g):
        return head_op.head_bwd(h, W, b.w_scale, y, idx, count, lse, g, inv_T, 1.0, 1.0, False, True, True,
                                need_w)

    def two_call():
        idx, count, out, lse, g = forward_grpo()
        return backward(idx, count, lse, g)

    def fused_step():
        # forward, GRPO weight and loss, grad_hidden and grad_W in one call, the logits computed once per row pass
        idx, count = head_op.compact_rows(b.scored)
        return head_op.head_step_grpo(h, W, b.w_scale, y, idx, count, inv_T, 1.0, 1.0, False, True, True, None,
                                      old, b.adv, mask_f, 0.2, 0.28, 5.0, True, need_w)

    # the bound route: the trainer's unchanged call path (bind_head's pre-hook binds the GRPO inputs; AReaL's loss on
    # the head's logprob column; loss.backward()), here the head's forward as the bound model runs it, the objective
    # (grpo_loss, the same reference objective) and autograd's backward, gradients set to None before each step
    hb = h.detach().clone().requires_grad_(True)
    Wb = W.detach().clone().requires_grad_(need_w and not cfg.fp8_weight)
    grpo_in = head_op.GrpoInputs(adv=b.adv, old=old, prox=None, mask=mask_f)

    def bound_step():
        hb.grad, Wb.grad = None, None
        idx, count = head_op.compact_rows(b.scored)
        out = head_op.grpo_bound_head(hb, Wb, y, cfg.temperature, grpo_in, idx=idx, count=count, w_scale=b.w_scale)
        loss, _ = head_op.grpo_loss(out[:, 0], None, old, b.adv, mask_f, 0.2, 0.28, 5.0)
        loss.backward()

    fused = cfg.backward != "none" and not args.two_call

    def step():
        if cfg.backward == "none":  # a forward-only workload: logprob and entropy of every scored row
            return forward()[2]
        if args.bound:
            return bound_step()
        return fused_step() if fused else two_call()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the timed region: each GEMM launch is bracketed by HIP events on its own stream (octo_timing_*)
    _lib.call("octo_timing_enable", 1)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3
    kernels = {}
    for name in GEMM_KERNELS:
        launches, total = _lib.timing_read(name)
        if launches:
            kernels[name] = {"launches_per_step": launches / args.steps, "avg_ms": total / launches,
                             "ms_per_step": total / args.steps}
    _lib.call("octo_timing_enable", 0)

    # per-phase HIP-event timing on the launch stream (torch's current stream carries every launch): the forward
    # and the backward of the two-call route (for the fused step: context beside its own time)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    fwd_ms, bwd_ms, reps = [], [], 0 if fused and args.no_context else 3
    if fused and reps:
        two_call()
        torch.cuda.synchronize()
    for _ in range(reps):
        ev[0].record()
        if cfg.backward == "none":
            forward()
        else:
            idx, count, out, lse, g = forward_grpo()
        ev[1].record()
        ev[2].record()
        if cfg.backward != "none":
            backward(idx, count, lse, g)
        ev[3].record()
        torch.cuda.synchronize()
        fwd_ms.append(ev[0].elapsed_time(ev[1]))
        bwd_ms.append(ev[2].elapsed_time(ev[3]))
    fwd_ms = sorted(fwd_ms)[reps // 2] if reps else None
    bwd_ms = sorted(bwd_ms)[reps // 2] if reps else None
    bound_ms = None
    if fused and reps:  # the bound route, same timing: one warm-up, the median of 3
        bound_step()
        torch.cuda.synchronize()
        runs = []
        for _ in range(3):
            ev[0].record()
            bound_step()
            ev[1].record()
            torch.cuda.synchronize()
            runs.append(ev[0].elapsed_time(ev[1]))
        bound_ms = sorted(runs)[1]

    n, d, V = scored_rows, cfg.d, cfg.V
    alg_flop = {"full": 6, "hidden": 4, "none": 2}[cfg.backward] * n * d * V
    # executed: the fused step computes the logits once (as the forward-only workload), the two-call route twice
    exe_flop = ({"full": 6, "hidden": 4, "none": 2} if fused or cfg.backward == "none"
                else {"full": 8, "hidden": 6})[cfg.backward] * n * d * V
    peak = PEAK_BF16 if cfg.dtype != torch.float32 else PEAK_F32
    step_s = ms / 1e3
    # every GEMM kernel of the path is one dense contraction of 2 * n * d * V FLOP per step: logits
    # (gemm_stats), logits again -> dz (gemm_dz, two-call route only), dz . W (gemm_store_grad_h), dz^T . h
    # (gemm_store_grad_w); a kernel launched in several row passes does 2 * n * d * V / launches per launch on
    # average. dz_scale (fused step) is HBM-bound: 4 bytes per element of the scored rows' [n, V_pad] (an f16
    # exponential read, a 16-bit dz written)
    flop_step = 2 * n * d * V
    V_pad = -(-V // 256) * 256
    for name, k in kernels.items():
        if name == "ex_fix":  # the row-offset exponentials' dz scales (and any flagged row's rescale): time only
            continue
        if name == "dz_scale":
            k["bytes_per_launch"] = 4 * n * V_pad / k["launches_per_step"]
            k["GBps"] = k["bytes_per_launch"] / (k["avg_ms"] / 1e3) / 1e9
            continue
        # gemm_grads (fused step) runs both gradient GEMMs of a row pass in one launch
        k["flop_per_launch"] = flop_step * (2 if name == "gemm_grads" else 1) / k["launches_per_step"]
        k["tflops"] = k["flop_per_launch"] / (k["avg_ms"] / 1e3) / 1e12
    for name, k in kernels.items():  # fabric (HBM side of L2) bytes per launch from the recorded rocprof counters
        t = recorded_traffic(name, cfg.name, fused)
        k["traffic_GBps"] = t / (k["avg_ms"] / 1e3) / 1e9 if t else None
    # the weight stream: the logits GEMM reads W (its MFMA operand: bf16, fp8 weights widened) once per launch that
    # has rows to score. The fused step's launches past the device row count end at once and read nothing, so W is
    # read once per row pass holding scored rows (ceil(n / rows per pass) of them); the forward reads it once.
    w_bytes = V * d * (4 if cfg.dtype == torch.float32 else 2)
    weight_stream = None
    if "gemm_stats" in kernels:
        ks = kernels["gemm_stats"]
        reads = 1
        if fused:
            w_code = _lib.FP8E4M3 if cfg.fp8_weight else {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16,
                                                           torch.float32: _lib.F32}[cfg.dtype]
            fl = _lib.WS_STEP | (0 if need_w else _lib.WS_NO_GRADW)
            ws = head_op.STEP_WORKSPACE_BYTES or _lib.workspace_bytes(cfg.N, d, V, w_code, fl)
            rows_per_pass = _lib.bwd_plan(cfg.N, d, V, w_code, fl, ws)[0]
            reads = -(-n // rows_per_pass)
        weight_stream = {"bytes_per_read": w_bytes, "kernel": "gemm_stats", "reads_per_step": reads,
                         "GBps": w_bytes * reads / (ks["ms_per_step"] / 1e3) / 1e9,
                         "fabric_GBps_all_operands": ks["traffic_GBps"]}
    # fabric traffic of one full row pass (the launches' averages include passes with fewer or no rows) against the
    # bytes the pass must move at least, recorded with the rocprof counters
    for name, k in kernels.items():
        full = recorded_traffic(name, cfg.name, fused, key="traffic_full_pass")
        alg = recorded_traffic(name, cfg.name, fused, key="algorithmic_full_pass")
        if full and alg:
            k["traffic_full_pass"] = full
            k["algorithmic_full_pass"] = alg
            k["traffic_ratio_full_pass"] = full / alg
    # The roofline kernel: the one with the most time per step among those whose FLOP are algorithmic work of the
    # metric (the forward logits GEMM and the two gradient GEMMs); gemm_dz recomputes the logits (executed, not
    # algorithmic work) and is never credited. The whole path's algorithmic and executed fractions sit beside it.
    algorithmic = [k for k in ("gemm_stats", "gemm_store_grad_h", "gemm_store_grad_w", "gemm_grads") if k in kernels]
    dom = max(algorithmic, key=lambda k: kernels[k]["ms_per_step"])
    flop_launch = kernels[dom]["flop_per_launch"]
    dom_achieved = flop_launch / (kernels[dom]["avg_ms"] / 1e3)
    result = {
        "metric": "packed tokens/sec fwd+bwd logprob @ d=2560,V=151936 bf16; % MFMA peak",
        "value": cfg.N / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else str(cfg.dtype).replace("torch.", ""),
        "data": "synthetic (seeded: hidden N(0,1) RMS-normalised, W N(0,0.02), Zipf(1.1) targets)",
        "config": {"workload": f"{cfg.name}: packed tree micro-batch, "
                               + ("bound GRPO head (fused step behind the columns, loss.backward())" if fused and
                                  args.bound else
                                  "fused fwd+bwd GRPO logprob head (one call)" if fused else
                                  "GRPO logprob head, forward then backward (two calls)" if cfg.backward != "none"
                                  else "logprob head forward"),
                   "N_packed": cfg.N, "scored_rows": n, "d": d, "V": V, "temperature": cfg.temperature,
                   "backward": cfg.backward, "weight": "fp8 e4m3 + row scales" if cfg.fp8_weight else "as hidden",
                   "parallelism": "single GPU"},
        "mfma_frac_algorithmic": alg_flop / step_s / peak,
        "mfma_frac_executed": exe_flop / step_s / peak,
        "phase_ms": ({"two_call_forward": fwd_ms, "two_call_backward": bwd_ms, "two_call_step": fwd_ms + bwd_ms,
                      "bound_step": bound_ms}
                     if fused and reps else {} if fused else {"forward": fwd_ms, "backward": bwd_ms}),
        "kernels": kernels,
        "weight_stream": weight_stream,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": dom_achieved / 1e12, "peak": peak / 1e12,
                     "unit": "TFLOP/s", "frac": dom_achieved / peak,
                     "traffic": recorded_traffic(dom, cfg.name, fused),
                     "per_launch": f"{'4' if dom == 'gemm_grads' else '2'}*n*d*V / launches = {flop_launch:.4g} "
                                   f"algorithmic FLOP (n={n} scored rows, "
                                   f"{kernels[dom]['launches_per_step']:g} launches per step), HIP events "
                                   f"around each launch over the timed steps",
                     "path_frac_algorithmic": alg_flop / step_s / peak,
                     "path_frac_executed": exe_flop / step_s / peak},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, n)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
