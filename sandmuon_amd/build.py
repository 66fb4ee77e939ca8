"""Build libsandmuon_amd.so (gfx950) in-tree with hipcc.

Usage: python -m sandmuon_amd.build   (or sandmuon_amd.build.build())
Each .hip file under csrc/ is compiled to an object in parallel, then the
objects are linked into sandmuon_amd/libsandmuon_amd.so; the C-ABI example
program examples/abi_example.cpp is linked against it as
sandmuon_amd/abi_example.  The compiler's per-kernel resource report
(VGPRs, spills, scratch bytes per lane, LDS, occupancy) is written to
sandmuon_amd/kernel_resources.json beside the library.
"""
from __future__ import annotations

import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libsandmuon_amd.so"
# A host program that uses the library through the C ABI only (HIP memory
# and streams, no Python); tests/test_gpu_abi_example.py runs it.
EXAMPLE_SRC = HERE / "examples" / "abi_example.cpp"
EXAMPLE = HERE / "abi_example"
ARCH = os.environ.get("SANDMUON_AMD_ARCH", "gfx950")
RESOURCES = HERE / "kernel_resources.json"

# -packed-fp32-ops: keep the compiler from emitting packed FP32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# "remark: Function Name: <symbol>" opens a kernel's record, then one
# "remark:     <key>: <value>" line per resource.
_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z][\w ]*?(?: \[[^\]]*\])?):\s+(\S+)\s+\[-Rpass-analysis")
_KEYS = {"VGPRs": "vgprs", "AGPRs": "agprs", "TotalSGPRs": "sgprs", "ScratchSize [bytes/lane]": "scratch",
         "Occupancy [waves/SIMD]": "occupancy", "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill",
         "LDS Size [bytes/block]": "lds"}


def parse_resources(text: str, src: str) -> dict:
    """Per-kernel resources from hipcc's -Rpass-analysis=kernel-resource-usage
    remarks: {symbol: {"source", "vgprs", "agprs", "sgprs", "scratch",
    "occupancy", "sgpr_spill", "vgpr_spill", "lds"}}."""
    out, cur = {}, None
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {"source": src})
        elif cur is not None and key in _KEYS:
            cur[_KEYS[key]] = int(val)
    return out


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="smx_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]

        def compile_one(pair):
            src, obj = pair
            cmd = [hipcc, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
            res = subprocess.run(cmd, capture_output=True, text=True)
            text = res.stdout + res.stderr
            # the remarks and their source excerpts are kept out of the log
            out = "\n".join(l for l in text.splitlines()
                            if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l
                            and not re.match(r"\s*(\d+ \||\|)", l))
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n{out}")
            if verbose and out.strip():
                print(out, file=sys.stderr)
            return parse_resources(text, src.name)

        workers = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
        with ThreadPoolExecutor(max_workers=workers) as ex:
            resources = {}
            for r in ex.map(compile_one, zip(srcs, objs)):
                resources.update(r)
        tmp_lib = Path(tmp) / LIB.name
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib), *map(str, objs)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
        shutil.move(str(tmp_lib), str(LIB))
        RESOURCES.write_text(json.dumps(dict(sorted(resources.items())), indent=1) + "\n")
        tmp_exe = Path(tmp) / EXAMPLE.name
        cmd = [hipcc, "-O2", "-std=c++17", str(EXAMPLE_SRC), "-o", str(tmp_exe), f"-L{HERE}", "-lsandmuon_amd",
               "-Wl,-rpath,$ORIGIN", "-Wno-unused-command-line-argument"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"example build failed:\n{res.stdout}{res.stderr}")
        shutil.move(str(tmp_exe), str(EXAMPLE))
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
