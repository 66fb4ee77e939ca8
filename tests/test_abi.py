"""CPU checks of the C ABI: the library loads without a GPU, exports every
function include/sandmuon_amd.h declares, its struct layouts match the
ctypes mirrors, and argument validation fails cleanly before any GPU work."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from sandmuon_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sandmuon_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(smx_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_reports_abi_version():
    lib = _native.lib()
    assert lib.smx_abi_version() == _native.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True).stdout
        exported = set(re.findall(r"\bT (smx_[a-z0-9_]+)", out))
        assert set(names) <= exported


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc missing")
def test_struct_layouts_match_header(tmp_path):
    src = tmp_path / "layout.c"
    fields = {
        "smx_finish_desc": _native.FinishDesc,
        "smx_stats_desc": _native.StatsDesc,
        "smx_adamw_desc": _native.AdamwDesc,
        "smx_matrix_desc": _native.MatrixDesc,
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "sandmuon_amd.h"', "int main(void){"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split("\n") if l)
    for cname, cls in fields.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, (cname, f)


def test_validation_errors_return_before_gpu_work():
    lib = _native.lib()
    # bad dtype
    rc = lib.smx_stats_accumulate(ctypes.c_void_p(16), 9, 4, 4, 4, ctypes.c_void_p(16), None, 1, None)
    assert rc == -3
    assert b"dtype" in lib.smx_last_error()
    # empty input is a no-op even with null pointers
    assert lib.smx_stats_accumulate(None, 0, 0, 4, 4, None, None, 1, None) == 0
    # batched statistics: two descriptors adding into overlapping slot rows
    # are rejected before any launch, and an empty table is a no-op
    S = _native.StatsDesc
    d0 = S(x=16, slots_sq=4096, slots_first=None, rows=4, cols=8, row_stride=8, dtype=0, n_slots=2)
    d1 = S(x=16, slots_sq=4096 + 32, slots_first=None, rows=4, cols=8, row_stride=8, dtype=1, n_slots=2)
    assert lib.smx_stats_accumulate_batch((S * 2)(d0, d1), 2, None) == -1
    assert b"overlap" in lib.smx_last_error()
    d1.slots_sq, d1.slots_first = 1 << 20, 4096 + 60  # first-moment rows overlapping d0's sums
    assert lib.smx_stats_accumulate_batch((S * 2)(d0, d1), 2, None) == -1
    d1.dtype = 7
    assert lib.smx_stats_accumulate_batch((S * 2)(d0, d1), 2, None) == -3
    assert lib.smx_stats_accumulate_batch(None, 0, None) == 0
    # matrix step: workspace too small
    d = _native.MatrixDesc(param=16, grad=16, momentum=16, inv_row=16, inv_col=16, rows=64, cols=32,
                           lr=1e-3, momentum_beta=.8, grad_dtype=0)
    arr = (_native.MatrixDesc * 1)(d)
    assert lib.smx_matrix_step(arr, 1, 1, ctypes.c_void_p(256), 1024, None) == -5
    # rank-one z without kappa
    d.z = 16
    arr = (_native.MatrixDesc * 1)(d)
    assert lib.smx_matrix_step(arr, 1, 1, ctypes.c_void_p(256), 1 << 40, None) == -1
    # unknown S8 mode
    assert lib.smx_s8(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 4, 4, 16, 4, 1, 7, ctypes.c_void_p(256), 1 << 20,
                      None) == -1
    # finish: bad kind
    f = _native.FinishDesc(sum_sq=16, slots_sq=16, ema=16, inv=16, n=4, count=1, n_slots=1, kind=5)
    assert lib.smx_stats_finish((_native.FinishDesc * 1)(f), 1, .97, None) == -1
    # fused statistics: the cast takes f32 input and a bf16/f16 output only
    assert lib.smx_stats_cast(ctypes.c_void_p(16), 1, 4, 4, 4, ctypes.c_void_p(16), None, 1, ctypes.c_void_p(16), 1,
                              4, None) == -3
    assert lib.smx_stats_cast(ctypes.c_void_p(16), 0, 4, 4, 4, ctypes.c_void_p(16), None, 1, ctypes.c_void_p(16), 0,
                              4, None) == -3
    assert lib.smx_stats_cast(None, 0, 0, 4, 4, ctypes.c_void_p(16), None, 1, None, 1, 4, None) == 0
    # relayout statistics: 16-bit input only, aligned strides, no row chunk
    # across a sequence (chunks of 512 rows for 2 x 1024 rows and 128 slots)
    v16 = ctypes.c_void_p(16)
    ok_args = (1, 2, 1024, 12, 64, 12 * 1024 * 64, 64, 1024 * 64, v16, v16, None, 128, None)
    assert lib.smx_stats_relayout(v16, 0, *ok_args[1:]) == -3
    assert lib.smx_stats_relayout(v16, 1, 2, 1024, 12, 60, 12 * 1024 * 60, 60, 1024 * 60, v16, v16, None, 128,
                                  None) == -4
    assert lib.smx_stats_relayout(ctypes.c_void_p(24), *ok_args) == -4
    assert lib.smx_stats_relayout(v16, 1, 2, 768, 12, 64, 12 * 768 * 64, 64, 768 * 64, v16, v16, None, 128,
                                  None) == -2
    assert b"multiple of the row chunk" in lib.smx_last_error()
    assert lib.smx_stats_relayout(v16, 1, 2, 1024, 12, 64, 12 * 1024 * 64, 64, 1024 * 64, v16, None, None, 128,
                                  None) == -1
    need = lib.smx_stats_colsum_workspace_bytes(768, 128)
    assert need >= 128 * 768 * 4 and need % 256 == 0
    assert lib.smx_stats_colsum_workspace_bytes(0, 128) == -1
    assert lib.smx_stats_colsum(ctypes.c_void_p(16), 1, 4, 768, 768, ctypes.c_void_p(16), 128, ctypes.c_void_p(16),
                                ctypes.c_void_p(256), need - 1, None) == -5
    assert lib.smx_stats_colsum(ctypes.c_void_p(16), 1, 4, 768, 768, ctypes.c_void_p(16), 128, ctypes.c_void_p(16),
                                ctypes.c_void_p(16), need, None) == -4
    # adamw: offsets must be prefix sums; the parameter dtype must be known
    a = _native.AdamwDesc(param=16, grad=16, exp_avg=16, exp_avg_sq=16, n=4, offset=3, bias1=.1, bias2=.1)
    assert lib.smx_adamw((_native.AdamwDesc * 1)(a), 1, 4, 1e-3, .9, .999, 1e-8, .01, None) == -2
    a.offset, a.param_dtype = 0, 3
    assert lib.smx_adamw((_native.AdamwDesc * 1)(a), 1, 4, 1e-3, .9, .999, 1e-8, .01, None) == -3
    # staged finish and AdamW: the descriptor checks of the by-value calls,
    # then the size of the device table
    f.kind = 0
    fs = (_native.FinishDesc * 3)(f, f, f)
    assert lib.smx_stats_finish_table_bytes(3) == 3 * ctypes.sizeof(_native.FinishDesc)
    assert lib.smx_stats_finish_table_bytes(0) == 0
    v16 = ctypes.c_void_p(16)
    assert lib.smx_stats_finish_staged(fs, 3, .97, None, 1 << 20, None) == -5
    assert lib.smx_stats_finish_staged(fs, 3, .97, v16, 3 * ctypes.sizeof(_native.FinishDesc) - 1, None) == -5
    f.kind = 5
    assert lib.smx_stats_finish_staged((_native.FinishDesc * 1)(f), 1, .97, v16, 1 << 20, None) == -1
    assert lib.smx_stats_finish_staged(fs, 0, .97, None, 0, None) == 0
    a = _native.AdamwDesc(param=16, grad=16, exp_avg=16, exp_avg_sq=16, n=4, offset=0, bias1=.1, bias2=.1)
    # the table holds the descriptors (each block finds its first tensor)
    assert lib.smx_adamw_table_bytes(1, 4) == ctypes.sizeof(_native.AdamwDesc)
    assert lib.smx_adamw_table_bytes(2, 10 ** 6) == 2 * ctypes.sizeof(_native.AdamwDesc)
    assert lib.smx_adamw_table_bytes(0, 0) == 0
    assert lib.smx_adamw_staged((_native.AdamwDesc * 1)(a), 1, 4, 1e-3, .9, .999, 1e-8, .01, None, 1 << 20,
                                None) == -5
    assert lib.smx_adamw_staged((_native.AdamwDesc * 1)(a), 1, 4, 1e-3, .9, .999, 1e-8, .01, v16,
                                ctypes.sizeof(_native.AdamwDesc) - 1, None) == -5
    a.offset = 3
    assert lib.smx_adamw_staged((_native.AdamwDesc * 1)(a), 1, 4, 1e-3, .9, .999, 1e-8, .01, v16, 1 << 20,
                                None) == -2
    # matrix step: f64 parameters are not a step dtype
    d = _native.MatrixDesc(param=16, grad=16, momentum=16, inv_row=16, inv_col=16, rows=64, cols=32,
                           lr=1e-3, momentum_beta=.8, grad_dtype=0, param_dtype=3)
    assert lib.smx_matrix_step((_native.MatrixDesc * 1)(d), 1, 1, ctypes.c_void_p(256), 1 << 40, None) == -3
    assert b"param dtype" in lib.smx_last_error()
    # helpers: kind, dtype and the rank-one pointers are checked
    v = ctypes.c_void_p(16)
    assert lib.smx_inverse_sqrt(2, 0, v, v, 4, v, v, v, None) == -1
    assert lib.smx_inverse_sqrt(0, 1, v, None, 4, v, None, None, None) == -3
    assert lib.smx_inverse_sqrt(1, 3, v, None, 4, v, None, None, None) == -1
    assert lib.smx_inverse_sqrt(0, 0, v, None, 0, v, None, None, None) == -2
    assert lib.smx_rank1_apply(2, v, ctypes.c_void_p(32), 1, 4, 4, v, v, v, v, v, v, 0, v, None) == -3
    assert lib.smx_rank1_apply(3, v, v, 1, 4, 4, v, v, v, v, v, v, 0, v, None) == -1  # out aliases x
    assert lib.smx_rank1_apply(0, v, ctypes.c_void_p(32), 0, 4, 4, v, v, v, v, v, v, 1, v, None) == 0


def test_compensated_stage_count_setting():
    lib = _native.lib()
    assert lib.smx_s8_comp_stages(7) == -1 and lib.smx_s8_comp_stages(-1) == -1
    assert lib.smx_s8_comp_stages(3) == 5   # the production default is unchanged by the rejected calls
    assert _native.s8_comp_stages(5) == 3
    with pytest.raises(ValueError):
        _native.s8_comp_stages(6)
    assert lib.smx_s8_comp_stages(5) == 5


def test_compensation_mask_setting():
    lib = _native.lib()
    assert lib.smx_s8_comp_mask(0x20) == -1 and lib.smx_s8_comp_mask(-1) == -1
    assert lib.smx_s8_comp_mask(0x15) == 0x1F  # the production default is unchanged by the rejected calls
    assert lib.smx_s8_comp_stages(2) == 1      # leading compensated stages of 0x15: stage 1 only
    assert _native.s8_comp_mask(0x1F) == 0x03
    with pytest.raises(ValueError):
        _native.s8_comp_mask(64)
    assert lib.smx_s8_comp_stages(5) == 5


def test_tile_geometry_setting():
    lib = _native.lib()
    assert lib.smx_s8_tile_geometry(3) == -1 and lib.smx_s8_tile_geometry(-1) == -1
    assert lib.smx_s8_tile_geometry(1) == 0   # the automatic default is unchanged by the rejected calls
    assert _native.s8_tile_geometry(2) == 1
    with pytest.raises(ValueError):
        _native.s8_tile_geometry(4)
    assert lib.smx_s8_tile_geometry(0) == 2


def test_stats_slot_rows():
    # Row chunks hold at least 512 rows and at most n_slots chunks are used.
    lib = _native.lib()
    cases = {0: 0, 1: 1, 512: 1, 513: 2, 16384: 32, 8192: 16, 65536: 128, 70000: 128, 10**7: 128}
    for rows, want in cases.items():
        assert lib.smx_stats_slot_rows(rows, 128) == want, rows
    assert lib.smx_stats_slot_rows(5000, 4) == 4
    assert lib.smx_stats_slot_rows(-1, 128) == -1 and lib.smx_stats_slot_rows(10, 0) == -1


def test_workspace_sizes_are_consistent():
    # 103M GPT matrices: 36 of 768x768 and 18 of 768x3072 (9 of them transposed).
    shapes = [(768, 768)] * 36 + [(3072, 768)] * 9 + [(768, 3072)] * 9
    for mode in (0, 1):
        ws = _native.matrix_step_workspace_bytes(shapes, mode)
        # two iterate buffers of r x c per matrix, one more (the stage-5
        # result in parameter layout) per transposed parameter, two r x r
        # buffers (G, P) per matrix and three more (T and the Q ping-pong)
        # per matrix of the Gram-space class (768 x 3072), 4 bytes per
        # element; and three row-sum partials per 64 elements of r x c
        rc = 36 * 768 * 768 + 18 * 768 * 3072
        dense = ((2 * rc + 9 * 768 * 3072) * 4 + 2 * 54 * 768 * 768 * 4 + 3 * 18 * 768 * 768 * 4
                 + 3 * rc // 64 * 4)
        assert dense <= ws <= dense * 1.01
    assert _native.lib().smx_s8_workspace_bytes(2, 7, 3, 0) > 0


def test_s8_timing_recorder_without_launches():
    lib = _native.lib()
    assert lib.smx_s8_timing(1) == 0
    assert _native.s8_timing_read(16) == []
    assert lib.smx_s8_timing(2) == 0
    assert _native.s8_timing_read(16) == []
    assert lib.smx_s8_timing(0) == 0
    assert lib.smx_s8_timing(3) == -1
    assert lib.smx_s8_timing_read(None, None, None, -1) == -1
