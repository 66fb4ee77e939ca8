"""The compiler's resource report of every kernel in the library (written by
sandmuon_amd/build.py from hipcc's kernel-resource-usage remarks).

No kernel may use scratch memory or spill registers: a spill or a private
array in the hot kernels costs far more than it shows in a register count.
(A rolled epilogue loop that indexed the GEMM accumulators at run time once
moved all of them to scratch in the 256-row square kernels, 576 bytes per
lane, with no spill reported, and made those launches 60% slower.)
The S8 GEMM kernels must also keep the occupancy their tile plan assumes.
"""
import json

import pytest

from sandmuon_amd import build as B

pytestmark = pytest.mark.skipif(not B.RESOURCES.exists(), reason="library not built (sandmuon_amd.build)")


def report():
    return json.loads(B.RESOURCES.read_text())


def test_report_is_current_and_covers_every_source():
    built = B.RESOURCES.stat().st_mtime
    stale = [s.name for s in B.sources() if s.stat().st_mtime > built]
    assert not stale, f"sources newer than the last build: {stale}"
    r = report()
    with_kernels = {v["source"] for v in r.values()}
    # every source that defines a kernel is in the report
    for s in B.sources():
        if "__global__" in s.read_text():
            assert s.name in with_kernels, s.name


def test_no_kernel_spills_or_uses_scratch():
    bad = {k: v for k, v in report().items() if v["scratch"] or v["vgpr_spill"] or v["sgpr_spill"]}
    assert not bad, bad


def test_s8_gemm_kernels_keep_their_occupancy():
    # 128 x 128 tiles (4 waves): at most 168 VGPRs, three waves per SIMD;
    # 256-row tiles: 256 VGPRs, two waves per SIMD.
    r = {k: v for k, v in report().items() if "s8_stage_kernel" in k}
    assert len(r) >= 30, sorted(r)
    for k, v in r.items():
        small = k.endswith("Li128ELi128EEEvNS_9StageArgsE")
        assert v["occupancy"] >= (3 if small else 2), (k, v)
        assert v["vgprs"] + v["agprs"] <= (168 if small else 256), (k, v)
