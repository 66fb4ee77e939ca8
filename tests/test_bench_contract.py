"""bench.py keeps the driver's contract: one JSON line with the metric of
BASELINE.json, the timing fields, the config and the roofline objects; a
request for more than one GPU is refused with a message (this build measures
one GPU).  The GPU case runs a short bench as a child process."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "bench.py"


def run_bench(*args, timeout=600):
    env = dict(os.environ)
    env.pop("WORLD_SIZE", None)
    return subprocess.run([sys.executable, str(BENCH), *args], capture_output=True, text=True, timeout=timeout,
                          cwd=str(ROOT), env=env)


def test_more_than_one_gpu_is_refused():
    res = run_bench("--gpus", "2")
    assert res.returncode == 2
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert line["n_gpus_requested"] == 2 and "one GPU" in line["error"]


@pytest.mark.gpu
def test_bench_line_has_the_contract_fields(device):
    res = run_bench("--steps", "2", "--warmup", "1", "--no-cpu-baseline")
    assert res.returncode == 0, res.stderr[-2000:]
    line = json.loads(res.stdout.strip().splitlines()[-1])
    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    assert line["metric"] == baseline["metric"]
    assert line["n_gpus"] == 1 and line["steps"] == 2 and line["warmup"] == 1
    assert line["unit"] == "ms" and line["higher_is_better"] is False and line["scaling"] == "weak"
    assert line["value"] == line["ms_per_step"] > 0
    assert line["vs_baseline"] is None and line["data"] == "synthetic" and line["dtype"] == "bf16"
    assert line["config"]["workload"].startswith("cfg4") and line["config"]["matrices"] == 54
    phases = line["phases_ms"]
    # the timed step is the hook phase and step(), nothing skipped
    assert abs(phases["hooks"] + phases["step"] - line["ms_per_step"]) < 0.05 * line["ms_per_step"]
    for key in ("roofline", "roofline_stats", "roofline_s8"):
        roof = line[key]
        assert roof["bound"] in ("hbm", "mfma")
        assert roof["unit"] in ("GB/s", "TFLOP/s")
        assert 0 < roof["frac"] <= 1 and abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
        assert "traffic" in roof
    assert line["roofline_stats"]["peak"] == 8000.0 and line["roofline_s8"]["peak"] == 2500.0
    s8 = line["roofline_s8"]
    assert s8["logical_flops_per_step"] == 1223059046400
    assert 0 < s8["ms_per_step"] < phases["step"]
    assert set(s8["phases"]) >= {"gram", "square", "apply"}
    # the same run's second BF16-class mode and the MFMA peak probe
    alt = line["alt_mode"]
    assert alt["s8_mode"] == "mixed" and 0 < alt["s8"]["ms_per_step"] < alt["phases_ms"]["step"]
    probe = s8["mfma_peak_probe"]
    for dt in ("bf16", "fp16", "fp32"):
        assert probe[dt]["finite"] and probe[dt]["tflops"] > 0 and 1.0 < probe[dt]["clock_ghz"] < 3.0
        assert probe[dt]["tflops"] <= 1.02 * probe[dt]["nominal_tflops_at_clock"]
    assert 0 < s8["frac_of_probe"] <= 1


def _write_csv(path, header, rows):
    import csv
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(header)
        w.writerows(rows)


def test_profile_summaries_of_synthetic_rocprof_output(tmp_path):
    """bench.py --summarize on hand-made rocprofv3 CSVs: a kernel trace of
    two steps, a counter run, and the four traffic runs, whose figures are
    known in closed form."""
    trace = ["Kind", "Agent_Id", "Queue_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    rows, t = [], 0
    for step in range(3):
        for name, us in (("smx::stats_accumulate_kernel(smx::StatsPack)", 100), ("smx::finish_fold_kernel(x)", 5),
                         ("smx::finish_kernel(x)", 5), ("void smx::s8_stage_kernel<1, 2, 256, 256>(smx::StageArgs)", 40)):
            rows.append(["KERNEL_DISPATCH", "Agent 1", 1, name, t, t + us * 1000])
            t += us * 1000 + 1000
    _write_csv(tmp_path / "tr" / "run_kernel_trace.csv", trace, rows)
    res = run_bench("--summarize", "trace", "--prof-dir", str(tmp_path / "tr"), "--prof-command", "cmd-t")
    assert res.returncode == 0, res.stderr
    out = res.stdout
    assert "cmd-t" in out and "s8_stage_kernel<1, 2, 256, 256>" in out
    stats = [l.split() for l in out.splitlines() if l.startswith("stats_accumulate_kernel")][0]
    assert stats[1:4] == ["3", "0.30", "100.0"], stats
    assert out.count("1 launches") == 3 and "span 52.0 us" in out  # fold 5 + 1 + finish 5 + 1 + S8 40

    cc = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    # a 100 us launch: 8 XCDs x 2.0 GHz, and 1.0e8 MFMA-busy cycles -> 1024 TFLOP/s
    _write_csv(tmp_path / "pmc" / "run_counter_collection.csv", cc,
               [[1, "void smx::s8_stage_kernel<1, 0, 128, 128>(smx::StageArgs)", "GRBM_GUI_ACTIVE", 8 * 2.0e5, 0,
                 100000],
                [1, "void smx::s8_stage_kernel<1, 0, 128, 128>(smx::StageArgs)", "SQ_VALU_MFMA_BUSY_CYCLES", 1.0e8, 0,
                 100000]])
    res = run_bench("--summarize", "counters", "--prof-dir", str(tmp_path / "pmc"), "--prof-command", "cmd-c")
    assert res.returncode == 0, res.stderr
    row = [l for l in res.stdout.splitlines() if l.startswith("s8_stage_kernel<1, 0, 128, 128>")][0].split()
    assert row[-6:] == ["1", "100.0", "2.00", "1024.0", "41.0", "49.2"], row

    # traffic: the copy of 1 MiB reads 512 KiB and writes 1024 KiB per dispatch
    for d, counter, name, kib in (("f", "FETCH_SIZE", "smx::adamw_kernel(smx::AdamPack)", 300.0),
                                  ("w", "WRITE_SIZE", "smx::adamw_kernel(smx::AdamPack)", 600.0),
                                  ("cf", "FETCH_SIZE", "__amd_rocclr_copyBuffer", 512.0),
                                  ("cw", "WRITE_SIZE", "__amd_rocclr_copyBuffer", 1024.0)):
        _write_csv(tmp_path / d / "run_counter_collection.csv", cc, [[1, name, counter, kib, 0, 1000]])
    js = tmp_path / "t.json"
    args = ["--summarize", "traffic", "--run-steps", "1", "--copy-mb", "1", "--json-out", str(js)]
    for d in ("f", "w", "cf", "cw"):
        args += ["--prof-dir", str(tmp_path / d), "--prof-command", f"cmd-{d}"]
    res = run_bench(*args)
    assert res.returncode == 0, res.stderr
    data = json.loads(js.read_text())
    assert data["calibration"]["fetch_scale"] == 2.0 and data["calibration"]["write_scale"] == 1.0
    assert data["adamw_kernel"] == {"launches_per_step": 1.0, "hbm_read_bytes_per_step": 600 * 1024,
                                    "hbm_write_bytes_per_step": 600 * 1024, "hbm_bytes_per_step": 1200 * 1024}
