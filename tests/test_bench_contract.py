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
