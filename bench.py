#!/usr/bin/env python
"""SandMuon optimizer step on one MI355X: BASELINE cfg4 (103M GPT, 54 matrices).

One "step" is the optimizer's whole hot path for one effective batch:
the statistics hooks of 8 microbatches (16 x 1024 tokens each) followed by
step() (finish statistics, AdamW on the 39.5M auxiliary parameters, and for
the 54 matrices momentum -> whiten -> S8 -> mapback -> graft -> update).

The hook bodies are driven directly with synthetic activations and
cotangents of the shapes and dtypes a bf16-autocast GPT forward/backward
hands them (LayerNorm-fed q/c_fc inputs in fp32, attention/GELU outputs and
every cotangent in bf16), rotating over two sets of 4 GB so HBM, not the
256 MB MALL, serves them.  Gradients are synthetic fp32.  No model forward
or backward is timed.

Prints one JSON line (driver contract) with `roofline` (dominant kernel) and
`cpu_baseline` (the CPU oracle on a bounded sample, rank 0, N=1 only).
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import torch

METRIC = "optimizer step ms (103M GPT, 54 mats) + S8 GEMM MFMA %peak, 1 GPU"
HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15         # dense BF16 MFMA, FLOP/s
FP32_PEAK = 157.3e12       # FP32 MFMA, FLOP/s


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="gpt103m", choices=["gpt103m", "gpt2048"])
    ap.add_argument("--s8-mode", default="comp_bf16", choices=["comp_bf16", "mixed", "fp32"])
    ap.add_argument("--no-alt-mode", action="store_true",
                    help="skip the second measurement of the other BF16-class S8 mode (comp_bf16 <-> mixed) "
                         "that the line carries under `alt_mode`")
    ap.add_argument("--no-peak-probe", action="store_true", help="skip the MFMA peak probe of the line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: all cores in the affinity mask")
    ap.add_argument("--train", action="store_true",
                    help="time whole training steps instead (model forward/backward of 8 microbatches under bf16 "
                         "autocast + step()), with the hook statistics, with the fused statistics, and with "
                         "no statistics; prints its own JSON line")
    ap.add_argument("--mfma-peak", action="store_true",
                    help="only run the MFMA peak probe (dense BF16, FP16 and FP32 MFMAs from registers on every "
                         "SIMD; sustained TFLOP/s and the engine clock held) and exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="only run 3 plain device copies of MB megabytes (the known-size reference for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    g = ap.add_argument_group("profile summaries (no GPU: text summaries of rocprofv3 --output-format csv runs "
                              "of this script, as committed under profiles/)")
    g.add_argument("--summarize", choices=["trace", "counters", "traffic"],
                   help="trace: a --kernel-trace run; counters: a --pmc run; traffic: the FETCH_SIZE and "
                        "WRITE_SIZE runs of the workload and of --copy-calibration (four --prof-dir, in that order)")
    g.add_argument("--prof-dir", action="append", default=[], help="rocprofv3 output directory (-d)")
    g.add_argument("--prof-command", action="append", default=[],
                   help="the command that made each --prof-dir (quoted in the summary)")
    g.add_argument("--title", default="", help="first line of the summary")
    g.add_argument("--run-steps", type=int, default=3,
                   help="optimizer steps in the profiled run (per-step figures = run totals / this)")
    g.add_argument("--copy-mb", type=int, default=512, help="the --copy-calibration size of the traffic runs")
    g.add_argument("--out", help="summary text file (default: stdout)")
    g.add_argument("--json-out", help="traffic: the per-kernel bytes as JSON (bench.py reads profiles/traffic_cfg4.json)")
    return ap.parse_args()


def copy_calibration(mb):
    """Three plain copies of `mb` MB (reads and writes mb*2^20 bytes each),
    the known-size reference for the rocprofv3 byte counters, then the rate
    of 20 more: the device's read+write streaming ceiling, against which the
    elementwise kernels of the step (read+write mixes) are judged."""
    n = mb * (1 << 20) // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(20):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / 20 * 1e3
    print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 3, "timed_copies": 20, "us_per_copy": round(us, 1),
                      "read_write_tb_s": round(2 * n * 4 / us / 1e6, 3)}), flush=True)


def mfma_peak_probe(device) -> dict:
    """Sustained dense MFMA rates (smx_mfma_peak: 4 blocks of 8 waves per CU,
    register operands, about 30 ms per dtype) and the clock held: the
    measured denominators beside the nominal 2.5 PFLOP/s (BF16/FP16) and
    157.3 TFLOP/s (FP32) peaks, which assume 2.4 GHz."""
    from sandmuon_amd import _native
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return {name: _native.mfma_peak(dt, iters, device, blocks=4 * cus)
            for name, dt, iters in (("bf16", torch.bfloat16, 40000), ("fp16", torch.float16, 40000),
                                    ("fp32", torch.float32, 20000))}


# ------------------------------------------------------------ workload ---
def build(cfg_name, mode, device):
    from sandmuon_amd import RankOneAWeightedPE
    from sandmuon_amd.workloads import GPT, GPT_103M, GPT_2048, transformer_filter
    cfg = GPT_103M if cfg_name == "gpt103m" else GPT_2048
    micro, mb_batch = (8, 16) if cfg_name == "gpt103m" else (4, 8)
    model = GPT(cfg).to(device)
    model.init_weights(1337)
    opt = RankOneAWeightedPE(model, lr=1e-2, module_filter=transformer_filter, s8_mode=mode)
    g = torch.Generator(device=device).manual_seed(1337)
    for p in model.parameters():
        p.grad = torch.randn(p.shape, generator=g, device=device) * 1e-3
    rows = mb_batch * cfg.ctx
    w, m = cfg.width, cfg.mlp
    sets = []
    for s in range(2):
        a, b = [], []
        for blk in model.transformer.h:
            # Hook inputs under bf16 autocast: LayerNorm outputs stay fp32,
            # the attention output and the GELU output are bf16.
            a.append((blk.attn.q_proj.weight, torch.randn(rows, w, generator=g, device=device)))
            a.append((blk.attn.c_proj.weight, torch.randn(rows, w, generator=g, device=device).bfloat16()))
            a.append((blk.mlp.c_fc.weight, torch.randn(rows, w, generator=g, device=device)))
            a.append((blk.mlp.c_proj.weight, torch.randn(rows, m, generator=g, device=device).bfloat16()))
            for lin, width in ((blk.attn.q_proj, w), (blk.attn.k_proj, w), (blk.attn.v_proj, w),
                               (blk.attn.c_proj, w), (blk.mlp.c_fc, m), (blk.mlp.c_proj, w)):
                b.append((lin.weight, (torch.randn(rows, width, generator=g, device=device) * 1e-3).bfloat16()))
        sets.append((a, b))
    stat_bytes = sum(t.numel() * t.element_size() for _, t in sets[0][0] + sets[0][1]) * micro
    return model, opt, sets, micro, stat_bytes


def run_hooks(opt, sets, micro):
    """The hook bodies of `micro` microbatches, then the launch of whatever
    the hooks left queued, so the hook phase holds every statistics launch."""
    for k in range(micro):
        a, b = sets[k % 2]
        for p, x in a:
            opt._accumulate_a(p, x)
        for p, d in b:
            opt._accumulate_b(p, d)
    opt._flush_stats()


def summarize_s8(runs, launches, steps):
    """Per-step S8 time and issued MFMA FLOPs from the whole-run records of
    the timed steps (first launch to last, so the time includes the stage-1
    polynomial pass and the gaps between launches), and per-phase launch
    averages from the per-launch records of one further, untimed step."""
    assert [p for _, p, _ in runs] == ["run"] * len(runs) and len(runs) % steps == 0
    ms = sum(r[0] for r in runs) / steps
    flops = sum(r[2] for r in runs) / steps
    per = {}
    for t, phase, fl in launches:
        d = per.setdefault(phase, [0, 0.0])
        d[0] += 1
        d[1] += t
    phases = {p: {"launches_per_step": per[p][0], "avg_us": round(per[p][1] / per[p][0] * 1e3, 1)}
              for p in per if p != "run"}
    return ms, flops, phases


def logical_s8_flops(opt):
    """Logical S8 FLOPs per step: 5 (4 r^2 c + 2 r^3) per oriented r x c matrix."""
    total = 0
    for p in opt.named_matrices.values():
        r, c = sorted(p.shape)
        total += 5 * (4 * r * r * c + 2 * r ** 3)
    return total


def vendor_gemm_rate(opt, device, reps=20):
    """Plain BF16 batched GEMMs of one S8 stage's shapes through torch.bmm
    (hipBLASLt), FP32 accumulation, one product each: per shape class of
    oriented r x c, the Gram X X^T, the square G G and the apply P X.  Dense
    FLOPs (the Gram and square in full) / time: the vendor library's rate on
    the S8's shapes on this box, a reference for the S8 kernel's own rate.
    Every operand is contiguous (no transposed views into bmm)."""
    classes = {}
    for p in opt.named_matrices.values():
        r, c = sorted(p.shape)
        classes[(r, c)] = classes.get((r, c), 0) + 1
    g = torch.Generator(device=device).manual_seed(7)
    work = []
    for (r, c), n in classes.items():
        x = torch.randn(n, r, c, generator=g, device=device).bfloat16()
        xt = x.transpose(1, 2).contiguous()
        gm = torch.randn(n, r, r, generator=g, device=device).bfloat16()
        work += [(x, xt, 2 * n * r * r * c), (gm, gm, 2 * n * r * r * r), (gm, x, 2 * n * r * r * c)]
    flops = sum(f for _, _, f in work)
    for a, b, _ in work:
        torch.bmm(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for a, b, _ in work:
            torch.bmm(a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "frac": round(flops / (ms * 1e-3) / BF16_PEAK, 4),
            "ms_per_stage": round(ms, 3), "flops_per_stage": flops,
            "what": "torch.bmm bf16 (hipBLASLt) on one S8 stage's shapes: Gram X X^T, square G G, apply P X, "
                    "one product each, dense"}


def committed_traffic():
    """HBM bytes per launch of the dominant kernels, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None if absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic_cfg4.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


# -------------------------------------------------------- CPU baseline ---
def _median_of_3(fn):
    """One warm-up call, then three timed calls: (median, min, max) seconds."""
    fn()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[1], times[0], times[2]


def cpu_baseline(cfg_name, threads):
    """The CPU oracle (the eager FP32 restatement of the reference) timed on
    this host's cores: step() on a deep copy of a pre-filled state (one
    microbatch of statistics and synthetic gradients for every matrix), and
    the hook bodies on one full microbatch of every hooked class (shape,
    dtype, side), each with one warm-up and the median of three, scaled by
    the number of such calls per step."""
    import copy
    from oracle import sandmuon_oracle as O
    from sandmuon_amd.workloads import GPT, GPT_103M, GPT_2048, transformer_filter
    torch.set_num_threads(threads)
    cfg = GPT_103M if cfg_name == "gpt103m" else GPT_2048
    micro, rows = (8, 16 * 1024) if cfg_name == "gpt103m" else (4, 8 * 1024)
    model = GPT(cfg)
    model.init_weights(1337)
    ora = O.OracleOptimizer(model, 1e-2, rank_one_a=True, module_filter=transformer_filter, hooks=False)
    g = torch.Generator().manual_seed(7)
    for p in model.parameters():
        p.grad = torch.randn(p.shape, generator=g) * 1e-3
    w, m = cfg.width, cfg.mlp
    # Hook classes of one transformer block under bf16 autocast: A (sum x^2
    # and sum x) of the LayerNorm-fed q and c_fc inputs in fp32 and of the
    # attention and GELU outputs in bf16; B (sum d^2) of the six cotangents.
    classes = {("a", w, torch.float32): 2, ("a", w, torch.bfloat16): 1, ("a", m, torch.bfloat16): 1,
               ("b", w, torch.bfloat16): 5, ("b", m, torch.bfloat16): 1}
    per_step = {"median": 0.0, "min": 0.0, "max": 0.0}
    for (side, width, dtype), calls in classes.items():
        x = torch.randn(rows, width, generator=g).to(dtype)
        sq = torch.zeros(width)
        first = torch.zeros(width) if side == "a" else None
        med, lo, hi = _median_of_3(lambda: O.accumulate_rows(x, sq, first))
        n = calls * cfg.layers * micro
        per_step["median"] += med * n
        per_step["min"] += lo * n
        per_step["max"] += hi * n
    # step(): statistics of one microbatch per matrix so that every factor
    # is defined; the state is deep-copied before each timed call.
    for name, p in ora.matrices.items():
        own = ora.a_source[id(p)] is p
        ora.feed(name, x=torch.randn(256, p.shape[1], generator=g) if own else None,
                 delta=torch.randn(256, p.shape[0], generator=g))
    filled = copy.deepcopy(ora.state)
    params = {id(p): p.detach().clone() for p in model.parameters()}

    def step_once():
        ora.state = copy.deepcopy(filled)
        with torch.no_grad():
            for p in model.parameters():
                p.copy_(params[id(p)])
        ora.step()

    step_med, step_lo, step_hi = _median_of_3(step_once)
    sample = (f"oracle step() on all {len(ora.matrices)} matrices and the AdamW parameters (1 warm-up, median of 3, "
              f"state deep-copied per call) + the hook bodies on one {rows}-row microbatch of each of the "
              f"{len(classes)} hooked classes (1 warm-up, median of 3), scaled x{cfg.layers * micro} per class "
              f"count ({micro} microbatches of {cfg.layers} blocks)")
    spread = {"step_ms": [round(step_lo * 1e3, 1), round(step_hi * 1e3, 1)],
              "hooks_ms": [round(per_step["min"] * 1e3, 1), round(per_step["max"] * 1e3, 1)]}
    return (per_step["median"] + step_med) * 1e3, per_step["median"] * 1e3, step_med * 1e3, sample, spread


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def quiet_gc():
    """Collect once and freeze the surviving objects before a timed region,
    as long training loops do: a full collection of the ~270K objects torch
    and the harness hold takes ~70 ms of host time, and when one falls inside
    the timed steps the GPU idles behind it.  Objects created later are
    still collected."""
    gc.collect()
    gc.freeze()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def train_bench(args, device):
    """Whole training steps of the cfg4 GPT: 8 microbatches of 16 x 1024
    random tokens, forward and backward under bf16 autocast, then step().
    Four variants on the same model and optimizer: the statistics in the
    hooks (the reference's design); fused into the Linear's input cast and
    bias-gradient passes (sandmuon_amd.fused); those and the MLP's GELU
    (the model passed to fuse_statistics); and none at all (hooks removed,
    forward/backward only) as the floor they are measured against."""
    from sandmuon_amd import RankOneAWeightedPE
    from sandmuon_amd.fused import fuse_statistics
    from sandmuon_amd.workloads import GPT, GPT_103M, transformer_filter
    model = GPT(GPT_103M).to(device)
    model.init_weights(1337)
    opt = RankOneAWeightedPE(model, lr=1e-4, module_filter=transformer_filter, s8_mode=args.s8_mode)
    g = torch.Generator(device=device).manual_seed(1337)
    micro = [(torch.randint(0, GPT_103M.vocab, (16, 1024), generator=g, device=device),
              torch.randint(0, GPT_103M.vocab, (16, 1024), generator=g, device=device)) for _ in range(8)]

    def fwd_bwd():
        for idx, tgt in micro:
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = model(idx, tgt) / len(micro)
            loss.backward()

    def timed(with_step):
        def once(ev=None):
            opt.zero_grad(set_to_none=True)
            if ev:
                ev[0].record()
            fwd_bwd()
            if ev:
                ev[1].record()
            if with_step:
                opt.step()
            if ev:
                ev[2].record()
        for _ in range(args.warmup):
            once()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
        torch.cuda.synchronize()
        quiet_gc()
        for k in range(args.steps):
            once(evs[k])
        torch.cuda.synchronize()
        fb = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
        st = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
        return round(fb + st, 3), round(fb, 3), round(st, 3)

    log("train: hook statistics")
    hooks = timed(True)
    log(f"train: hooks {hooks}")
    handle = fuse_statistics(opt)
    log(f"train: fused statistics ({len(handle.fused_names)} layers)")
    fused = timed(True)
    log(f"train: fused {fused}")
    handle.close()
    handle = fuse_statistics(opt, model)
    log("train: fused statistics and GELU")
    fused_gelu = timed(True)
    gelu_per_step = handle.gelu_taken / (args.warmup + args.steps)
    log(f"train: fused with GELU {fused_gelu} ({gelu_per_step:.0f} GELU outputs' statistics taken per step)")
    handle.close()
    opt.close()
    log("train: no statistics (forward/backward only)")
    floor = timed(False)
    log(f"train: floor {floor}")
    out = {
        "metric": "training step ms (103M GPT: 8 x 16x1024-token microbatches fwd+bwd under bf16 autocast + "
                  "SandMuon step), 1 GPU",
        "value": fused[0], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": fused[0], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg4 training step with fused statistics", "s8_mode": args.s8_mode,
                   "matrices": len(opt.named_matrices), "microbatches": len(micro)},
        "variants_ms": {"hooks": {"total": hooks[0], "fwd_bwd": hooks[1], "step": hooks[2]},
                        "fused": {"total": fused[0], "fwd_bwd": fused[1], "step": fused[2]},
                        "fused_with_gelu": {"total": fused_gelu[0], "fwd_bwd": fused_gelu[1], "step": fused_gelu[2],
                                            "gelu_outputs_per_step": gelu_per_step},
                        "no_statistics_fwd_bwd": floor[1]},
        "statistics_cost_ms": {"hooks": round(hooks[1] - floor[1], 3), "fused": round(fused[1] - floor[1], 3),
                               "fused_with_gelu": round(fused_gelu[1] - floor[1], 3)},
    }
    print(json.dumps(out), flush=True)


# ------------------------------------------------------- profile summaries ---
# Text summaries of the rocprofv3 runs of this script (CSV output), the form
# committed under profiles/.  Counter values are per dispatch, summed over
# the hardware instances by rocprofv3 (SQ counters over the shader engines,
# GRBM counters over the 8 XCDs).
S8_PHASE_NAMES = {"0": "gram", "1": "square", "2": "apply", "5": "sym"}


def _prof_rows(d, stem):
    import csv
    import glob
    import gzip
    files = sorted(glob.glob(os.path.join(d, "**", f"*{stem}.csv"), recursive=True) +
                   glob.glob(os.path.join(d, "**", f"*{stem}.csv.gz"), recursive=True))
    if not files:
        sys.exit(f"no *{stem}.csv(.gz) under {d}")
    rows = []
    for f in files:
        with (gzip.open(f, "rt") if f.endswith(".gz") else open(f)) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def _kname(name):
    """Kernel name without namespace and argument list, template arguments kept."""
    n = name.replace("void ", "").replace("smx::", "").replace("(anonymous namespace)::", "")
    if n.startswith("Cijk_"):  # hipBLASLt: its macro tile names the kernel
        tile = [t for t in n.split("_") if t.startswith("MT")]
        return "hipBLASLt " + (tile[0] if tile else n[:24])
    return n.split("(")[0] if "(" in n else n


def _git_head():
    import subprocess
    try:
        here = os.path.dirname(os.path.abspath(__file__))
        return subprocess.run(["git", "-C", here, "rev-parse", "--short", "HEAD"], capture_output=True,
                              text=True, check=True).stdout.strip()
    except Exception:
        return "unknown"


def _header(args, lines):
    out = [f"# {args.title}" if args.title else "# rocprofv3 summary", ""]
    cmds = args.prof_command or []
    out.append("command:" if len(cmds) == 1 else "commands:")
    out += [f"  {c}" for c in cmds]
    out.append(f"summary: python bench.py --summarize {args.summarize} " +
               " ".join(f"--prof-dir {d}" for d in args.prof_dir) + f" --run-steps {args.run_steps}")
    out.append(f"code: git {_git_head()}")
    out.append("")
    return out + lines + [""]


def _steps_of(trace):
    """Start indices of step(): the first finish-fold launch after any other kernel."""
    fin = lambda n: "finish_fold" in n or "finish_kernel" in n or "finish_table_kernel" in n
    return [i for i, r in enumerate(trace) if "finish_fold" in r["name"] and (i == 0 or not fin(trace[i - 1]["name"]))]


def summarize_trace(args):
    rows = _prof_rows(args.prof_dir[0], "kernel_trace")
    trace = sorted(({"name": r["Kernel_Name"], "q": int(r["Queue_Id"]), "t0": int(r["Start_Timestamp"]),
                     "t1": int(r["End_Timestamp"])} for r in rows), key=lambda r: r["t0"])
    agg = {}
    for r in trace:
        a = agg.setdefault(_kname(r["name"]), [0, 0.0])
        a[0] += 1
        a[1] += (r["t1"] - r["t0"]) / 1e3
    total = sum(v[1] for v in agg.values())
    lines = ["Durations are rocprofv3 per-dispatch GPU times over the whole run (warm-up, timed and per-launch",
             "timing steps of bench.py, plus the synthetic-input setup: at::native kernels).  The S8 launches",
             "run as two chains on two streams (two HW queues), so their durations overlap in time.", "",
             f"{'kernel':<60}{'calls':>7}{'total_ms':>11}{'avg_us':>10}{'pct':>7}"]
    for n, (c, us) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        lines.append(f"{n[:59]:<60}{c:>7}{us / 1e3:>11.2f}{us / c:>10.1f}{100 * us / total:>7.2f}")
    st = _steps_of(trace)
    lines += ["", "## Statistics launches before each step()"]
    prev = 0
    for i in st:
        lines.append(f"  {sum('stats_accumulate_kernel' in r['name'] for r in trace[prev:i])} launches")
        prev = i
    if len(st) >= 2:
        # the last timed step (the run's last step carries per-launch timing events)
        a, b = st[-2], st[-1]
        b = next((k for k in range(a + 1, b) if "stats_accumulate_kernel" in trace[k]["name"]), b)
        step = trace[a:b]
        t0 = step[0]["t0"]
        span = (max(r["t1"] for r in step) - t0) / 1e3
        lines += ["", f"## One timed step(), in launch order (start offset, duration, HW queue): span {span:.1f} us"]
        for r in step:
            lines.append(f"  {(r['t0'] - t0) / 1e3:9.1f} us {(r['t1'] - r['t0']) / 1e3:8.1f} us  q{r['q']}  "
                         f"{_kname(r['name'])}")
        per = {}
        for r in step:
            per[_kname(r["name"])] = per.get(_kname(r["name"]), 0.0) + (r["t1"] - r["t0"]) / 1e3
        lines += ["", "## GPU time of that step() by kernel (us; the two S8 chains overlap)"]
        for n, us in sorted(per.items(), key=lambda kv: -kv[1]):
            lines.append(f"  {us:9.1f}  {n}")
    return "\n".join(_header(args, lines))


def _dispatches(d):
    """{dispatch id: {"name", "dur_ns", counter: value}} of a --pmc run."""
    out = {}
    for r in _prof_rows(d, "counter_collection"):
        e = out.setdefault(r["Dispatch_Id"], {"name": r["Kernel_Name"],
                                              "dur_ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
        e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def summarize_counters(args):
    disp = _dispatches(args.prof_dir[0])
    groups = {}
    for e in disp.values():
        groups.setdefault(_kname(e["name"]), []).append(e)
    counters = sorted({k for e in disp.values() for k in e if k not in ("name", "dur_ns")})
    lines = ["Per kernel: launches in the profiled run, average launch time (counter runs serialise the",
             "launches, so the two S8 chains do not overlap here) and the run totals of each counter per launch.",
             "Derived, where the counters are present:",
             "  clock_GHz = GRBM_GUI_ACTIVE / 8 XCDs / launch time (launches under 30 us: '-', their counter",
             "  window is longer than the launch);",
             "  issued TFLOP/s = SQ_VALU_MFMA_BUSY_CYCLES x 1024 FLOP / launch time, %nom against 2.5 PFLOP/s,",
             "  %clk against 2.5 PFLOP/s x clock / 2.4 GHz;",
             "  fractions of SQ_WAVE_CYCLES: wait_issue = SQ_WAIT_INST_ANY (waiting to issue the next",
             "  instruction), wait_any = SQ_WAIT_ANY (memory counters, barriers), wait_lds = SQ_WAIT_INST_LDS,",
             "  valu / lds = SQ_ACTIVE_INST_VALU / _LDS, vmem_cyc = SQ_INST_CYCLES_VMEM;",
             "  MOPS/LDS = (SQ_INSTS_VALU_MFMA_MOPS_BF16 + _F16) per SQ_INSTS_LDS (one MOP = 512 FLOP).", ""]
    hdr = f"{'kernel':<44}{'calls':>6}{'avg_us':>9}"
    have = set(counters)
    if "GRBM_GUI_ACTIVE" in have:
        hdr += f"{'clk_GHz':>9}"
    if "SQ_VALU_MFMA_BUSY_CYCLES" in have:
        hdr += f"{'TFLOP/s':>9}{'%nom':>7}{'%clk':>7}"
    labels = {"SQ_WAIT_INST_ANY": "wait_issue", "SQ_WAIT_ANY": "wait_any", "SQ_WAIT_INST_LDS": "wait_lds",
              "SQ_ACTIVE_INST_VALU": "valu", "SQ_ACTIVE_INST_LDS": "lds", "SQ_INST_CYCLES_VMEM": "vmem_cyc"}
    waits = [c for c in labels if c in have and "SQ_WAVE_CYCLES" in have]
    hdr += "".join(f"{labels[c]:>11}" for c in waits)
    lds = "SQ_INSTS_LDS" in have
    if lds:
        hdr += f"{'LDS_insts':>11}{'conflict':>11}{'MOPS/LDS':>9}"
    lines.append(hdr)
    for n, es in sorted(groups.items(), key=lambda kv: -sum(e["dur_ns"] for e in kv[1])):
        if n.startswith("at::") or n.startswith("__amd"):
            continue
        c = len(es)
        dur = sum(e["dur_ns"] for e in es)
        tot = lambda k: sum(e.get(k, 0.0) for e in es)
        row = f"{n[:43]:<44}{c:>6}{dur / c / 1e3:>9.1f}"
        clk = None
        if "GRBM_GUI_ACTIVE" in have:
            if dur / c >= 30e3:
                clk = tot("GRBM_GUI_ACTIVE") / 8 / dur
                row += f"{clk:>9.2f}"
            else:
                row += f"{'-':>9}"
        if "SQ_VALU_MFMA_BUSY_CYCLES" in have:
            tf = tot("SQ_VALU_MFMA_BUSY_CYCLES") * 1024 / dur / 1e3
            row += f"{tf:>9.1f}{100 * tf / 2500:>7.1f}"
            row += f"{100 * tf / (2500 * clk / 2.4):>7.1f}" if clk else f"{'':>7}"
        wc = tot("SQ_WAVE_CYCLES") if waits else 0.0
        row += "".join(f"{tot(w) / wc:>11.3f}" if wc else f"{'':>11}" for w in waits)
        if lds:
            li = tot("SQ_INSTS_LDS")
            mops = tot("SQ_INSTS_VALU_MFMA_MOPS_BF16") + tot("SQ_INSTS_VALU_MFMA_MOPS_F16")
            row += f"{li / c:>11.3g}{tot('SQ_LDS_BANK_CONFLICT') / c:>11.3g}" + (f"{mops / li:>9.1f}" if li else "")
        lines.append(row)
    return "\n".join(_header(args, lines))


def summarize_traffic(args):
    fetch, write, cfetch, cwrite = (_dispatches(d) for d in args.prof_dir[:4])
    copy_bytes = args.copy_mb * (1 << 20)

    def copies(disp, counter):
        v = [e[counter] for e in disp.values() if "copyBuffer" in e["name"] and e.get(counter)]
        v.sort()
        return v[len(v) // 2]  # the median copy of the calibration run (KiB)

    cf, cw = copies(cfetch, "FETCH_SIZE"), copies(cwrite, "WRITE_SIZE")
    fscale, wscale = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)

    def group(name):
        k = _kname(name)
        if k.startswith("s8_stage_kernel<"):
            return ["s8_stage_kernel", "s8_stage_kernel " + S8_PHASE_NAMES.get(k.split("<")[1].split(",")[1].strip(), "?")]
        return [k.split("<")[0]]

    per = {}
    for disp, key, scale, counter in ((fetch, "hbm_read_bytes_per_step", fscale, "FETCH_SIZE"),
                                      (write, "hbm_write_bytes_per_step", wscale, "WRITE_SIZE")):
        for e in disp.values():
            if e["name"].startswith("void at::") or "__amd" in e["name"] or "Cijk" in e["name"]:
                continue
            for g in group(e["name"]):
                d = per.setdefault(g, {"launches_per_step": 0.0, "hbm_read_bytes_per_step": 0.0,
                                       "hbm_write_bytes_per_step": 0.0})
                d[key] += e.get(counter, 0.0) * 1024 * scale / args.run_steps
                if counter == "FETCH_SIZE":
                    d["launches_per_step"] += 1 / args.run_steps
    for d in per.values():
        d["hbm_bytes_per_step"] = d["hbm_read_bytes_per_step"] + d["hbm_write_bytes_per_step"]
        for k in d:
            d[k] = round(d[k], 2) if k == "launches_per_step" else int(d[k])
    js = {"calibration": {"copy_bytes": copy_bytes, "FETCH_SIZE_KiB": cf, "WRITE_SIZE_KiB": cw,
                          "fetch_scale": fscale, "write_scale": wscale},
          "commands": args.prof_command, "code": _git_head(), **per}
    lines = [f"Calibration: a plain device copy of {copy_bytes} bytes reads FETCH_SIZE = {cf:.0f} KiB and "
             f"WRITE_SIZE = {cw:.0f} KiB per dispatch,",
             f"so fetch counts are scaled by {fscale:.3f} and write counts by {wscale:.3f}.",
             f"Per step = counter totals of the profiled run / {args.run_steps} steps.", "",
             f"{'kernel':<32}{'launches/step':>14}{'read GB':>10}{'write GB':>10}{'total GB':>10}"]
    for n, d in sorted(per.items(), key=lambda kv: -kv[1]["hbm_bytes_per_step"]):
        lines.append(f"{n:<32}{d['launches_per_step']:>14.2f}{d['hbm_read_bytes_per_step'] / 1e9:>10.3f}"
                     f"{d['hbm_write_bytes_per_step'] / 1e9:>10.3f}{d['hbm_bytes_per_step'] / 1e9:>10.3f}")
    return "\n".join(_header(args, lines)), js


def summarize(args):
    need = 4 if args.summarize == "traffic" else 1
    if len(args.prof_dir) != need:
        sys.exit(f"--summarize {args.summarize} takes {need} --prof-dir")
    js = None
    if args.summarize == "trace":
        text = summarize_trace(args)
    elif args.summarize == "counters":
        text = summarize_counters(args)
    else:
        text, js = summarize_traffic(args)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text)
    else:
        print(text)
    if js is not None and args.json_out:
        with open(args.json_out, "w") as f:
            json.dump(js, f, indent=1)
            f.write("\n")


# ---------------------------------------------------------------- main ---
def main():
    args = parse()
    if args.summarize:
        summarize(args)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.mfma_peak:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        print(json.dumps({"mfma_peak_probe": mfma_peak_probe(torch.device("cuda", 0))}), flush=True)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: the optimizer step is run and reported "
                                   "on a single MI355X (multi-GPU sharding is a design note, not built)",
                          "n_gpus_requested": args.gpus}))
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from sandmuon_amd import _native
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.train:
        if args.config != "gpt103m":
            sys.exit("--train runs the cfg4 (gpt103m) model only")
        train_bench(args, device)
        return
    log(f"building {args.config} ({args.s8_mode})")
    model, opt, sets, micro, stat_bytes = build(args.config, args.s8_mode, device)
    log(f"built: {len(opt.named_matrices)} matrices, {stat_bytes / 1e9:.2f} GB of hook input per step")

    def one_step(ev=None):
        if ev:
            ev[0].record()
        run_hooks(opt, sets, micro)
        if ev:
            ev[1].record()
        opt.step()
        if ev:
            ev[2].record()

    def timed_steps(steps):
        """`steps` timed steps: total ms per step, hook-phase and step() ms,
        host wall ms, and the library's whole-run S8 records."""
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        _native.s8_timing(True, runs_only=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for k in range(steps):
            one_step(evs[k])
        end.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        _native.s8_timing(False)
        runs = _native.s8_timing_read()
        ms = start.elapsed_time(end) / steps
        hooks_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
        step_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
        return ms, hooks_ms, step_ms, wall, runs

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    quiet_gc()
    log("warmup done")
    # Timed region: K steps between two events; inside it, event pairs around
    # the hook phase and step() of every step, and the library records an
    # event pair around each step's whole S8 run on the stream it uses.
    ms, hooks_ms, step_ms, wall, runs = timed_steps(args.steps)
    # One more step, untimed, with an event pair around every S8 launch for
    # the per-phase breakdown.
    _native.s8_timing(True)
    one_step()
    _native.s8_timing(False)
    launches = _native.s8_timing_read()
    s8_ms, s8_issued, s8_phases = summarize_s8(runs, launches, args.steps)
    s8_logical = logical_s8_flops(opt)
    log(f"timed {args.steps} steps: {ms:.3f} ms/step (hooks {hooks_ms:.3f}, step {step_ms:.3f}, "
        f"S8 GEMM launches {s8_ms:.3f})")

    peak_mfma = FP32_PEAK if args.s8_mode == "fp32" else BF16_PEAK  # FP16 and BF16 MFMA share the peak
    stats_gbs = stat_bytes / (hooks_ms * 1e-3) / 1e9
    s8_tfs = s8_issued / (s8_ms * 1e-3) / 1e12
    # The committed counter summary covers the cfg4 step in comp_bf16 mode;
    # other workloads and modes carry no traffic figure.
    traffic = (committed_traffic() or {}) if (args.config, args.s8_mode) == ("gpt103m", "comp_bf16") else {}
    roof_stats = {"bound": "hbm", "achieved": round(stats_gbs, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                  "frac": round(stats_gbs / (HBM_PEAK / 1e9), 4),
                  "traffic": traffic.get("stats_accumulate_kernel", {}).get("hbm_bytes_per_step"),
                  "kernel": "stats_accumulate_kernel (every statistics launch of the step's hooks: queued hook inputs, "
                            "up to 1 GiB of them per launch)",
                  "bytes_per_step": stat_bytes, "ms_per_step": round(hooks_ms, 3)}
    roof_s8 = {"bound": "mfma", "achieved": round(s8_tfs, 1), "peak": peak_mfma / 1e12, "unit": "TFLOP/s",
               "frac": round(s8_tfs / (peak_mfma / 1e12), 4),
               "traffic": traffic.get("s8_stage_kernel", {}).get("hbm_bytes_per_step"),
               "kernel": "s8_stage_kernel (Gram/square/apply launches of step(); time = span of the S8 run)",
               "issued_flops_per_step": s8_issued, "logical_flops_per_step": s8_logical,
               "logical_tflops": round(s8_logical / (s8_ms * 1e-3) / 1e12, 1), "ms_per_step": round(s8_ms, 3),
               "phases": s8_phases}
    roof_s8["vendor_bf16_gemm"] = vendor_gemm_rate(opt, device)
    alt = None
    alt_mode = {"comp_bf16": "mixed", "mixed": "comp_bf16"}.get(args.s8_mode)
    if alt_mode and not args.no_alt_mode:
        # The same workload and optimizer with the other BF16-class S8 mode:
        # one warm-up step, then the same number of timed steps.
        log(f"alternate mode {alt_mode}")
        opt.s8_mode = alt_mode
        one_step()
        a_ms, a_hooks, a_step, _, a_runs = timed_steps(args.steps)
        opt.s8_mode = args.s8_mode
        a_s8 = sum(r[0] for r in a_runs) / args.steps
        a_issued = sum(r[2] for r in a_runs) / args.steps
        a_tfs = a_issued / (a_s8 * 1e-3) / 1e12
        alt = {"s8_mode": alt_mode, "ms_per_step": round(a_ms, 4),
               "phases_ms": {"hooks": round(a_hooks, 3), "step": round(a_step, 3)},
               "s8": {"ms_per_step": round(a_s8, 3), "achieved_tflops": round(a_tfs, 1),
                      "frac": round(a_tfs / (BF16_PEAK / 1e12), 4), "issued_flops_per_step": a_issued,
                      "logical_tflops": round(s8_logical / (a_s8 * 1e-3) / 1e12, 1)}}
    if not args.no_peak_probe:
        probe = mfma_peak_probe(device)
        roof_s8["mfma_peak_probe"] = probe
        key = {"fp32": "fp32", "mixed": "fp16"}.get(args.s8_mode, "bf16")
        roof_s8["frac_of_probe"] = round(s8_tfs / probe[key]["tflops"], 4)
        if alt:
            akey = "fp16" if alt["s8_mode"] == "mixed" else "bf16"
            alt["s8"]["frac_of_probe"] = round(alt["s8"]["achieved_tflops"] / probe[akey]["tflops"], 4)
    dominant = roof_stats if hooks_ms >= s8_ms else roof_s8
    out = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": {"comp_bf16": "bf16", "mixed": "bf16+fp16", "fp32": "fp32"}[args.s8_mode], "data": "synthetic",
        "config": {"workload": ("cfg4: 103M GPT SandMuon step = hook statistics of 8 microbatches x 16x1024 tokens + "
                                "step() on 54 matrices + AdamW on 39.5M params") if args.config == "gpt103m" else
                   "cfg5: 2048-wide 24-layer GPT, 144 matrices, 4 microbatches x 8x1024 tokens",
                   "s8_mode": args.s8_mode, "matrices": len(opt.named_matrices), "microbatches": micro},
        "roofline": dominant,
        "roofline_stats": roof_stats,
        "roofline_s8": roof_s8,
        "phases_ms": {"hooks": round(hooks_ms, 3), "step": round(step_ms, 3), "host_wall_per_step": round(wall, 3)},
    }
    if alt:
        out["alt_mode"] = alt
    if not args.no_cpu_baseline:
        log("cpu baseline")
        threads = args.cpu_threads or len(os.sched_getaffinity(0))
        total, hooks, step, sample, spread = cpu_baseline(args.config, threads)
        out["cpu_baseline"] = {"value": round(total, 1), "unit": "ms", "cores": threads, "kind": "port",
                               "sample": sample, "hooks_ms": round(hooks, 1), "step_ms": round(step, 1),
                               "spread_min_max": spread, "cpu": cpu_model_name()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
