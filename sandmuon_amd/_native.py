"""ctypes binding of libsandmuon_amd.so (the C ABI in include/sandmuon_amd.h).

The library is the only compute path of this package: if it cannot be
loaded, every entry point raises.  There is no CPU or eager-PyTorch fallback.
Device tensors are passed by data pointer; every call enqueues on the
current HIP stream of the tensor's device.
"""
from __future__ import annotations

import ctypes
import functools
import threading
from ctypes import c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path
from typing import List, Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsandmuon_amd.so"
ABI_VERSION = 5

SMX_F32, SMX_BF16, SMX_F16, SMX_F64 = 0, 1, 2, 3
S8_FP32, S8_COMP_BF16, S8_MIXED = 0, 1, 2
S8_MODES = {"fp32": S8_FP32, "comp_bf16": S8_COMP_BF16, "mixed": S8_MIXED}

_DTYPES = {torch.float32: SMX_F32, torch.bfloat16: SMX_BF16, torch.float16: SMX_F16}

_STATUS = {
    -1: "SMX_EINVAL", -2: "SMX_ESHAPE", -3: "SMX_EDTYPE", -4: "SMX_EALIGN",
    -5: "SMX_EWORKSPACE", -6: "SMX_ELAUNCH",
}


class NativeError(RuntimeError):
    """A libsandmuon_amd entry point returned an error status."""


class FinishDesc(ctypes.Structure):
    _fields_ = [("sum_sq", c_void_p), ("slots_sq", c_void_p), ("sum_first", c_void_p),
                ("slots_first", c_void_p), ("ema", c_void_p), ("mean_ema", c_void_p),
                ("inv", c_void_p), ("z", c_void_p), ("kappa", c_void_p),
                ("n", c_int64), ("count", c_int64), ("n_slots", c_int32), ("kind", c_int32),
                ("first", c_int32), ("pad_", c_int32)]


class StatsDesc(ctypes.Structure):
    _fields_ = [("x", c_void_p), ("slots_sq", c_void_p), ("slots_first", c_void_p),
                ("rows", c_int64), ("cols", c_int64), ("row_stride", c_int64),
                ("dtype", c_int32), ("n_slots", c_int32)]


class AdamwDesc(ctypes.Structure):
    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("exp_avg", c_void_p),
                ("exp_avg_sq", c_void_p), ("n", c_int64), ("offset", c_int64),
                ("bias1", c_float), ("bias2", c_float), ("grad_dtype", c_int32), ("param_dtype", c_int32)]


class MatrixDesc(ctypes.Structure):
    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("momentum", c_void_p),
                ("inv_row", c_void_p), ("inv_col", c_void_p), ("z", c_void_p), ("kappa", c_void_p),
                ("rows", c_int64), ("cols", c_int64), ("lr", c_double), ("momentum_beta", c_double),
                ("grad_dtype", c_int32), ("param_dtype", c_int32)]


# name -> (restype, argtypes); every symbol include/sandmuon_amd.h declares.
SIGNATURES = {
    "smx_abi_version": (c_int, []),
    "smx_last_error": (ctypes.c_char_p, []),
    "smx_stats_accumulate": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                     c_int32, c_void_p]),
    "smx_stats_accumulate_batch": (c_int, [ctypes.POINTER(StatsDesc), c_int32, c_void_p]),
    "smx_stats_slot_rows": (c_int32, [c_int64, c_int32]),
    "smx_stats_cast": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int32,
                               c_void_p, c_int, c_int64, c_void_p]),
    "smx_stats_gelu": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                               c_int32, c_void_p]),
    "smx_stats_relayout": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                   c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "smx_stats_add_partials": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "smx_stats_colsum_workspace_bytes": (c_int64, [c_int64, c_int32]),
    "smx_stats_colsum": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_int32, c_void_p,
                                 c_void_p, c_int64, c_void_p]),
    "smx_stats_fold": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "smx_stats_finish": (c_int, [ctypes.POINTER(FinishDesc), c_int32, c_double, c_void_p]),
    "smx_stats_finish_table_bytes": (c_size_t, [c_int32]),
    "smx_stats_finish_staged": (c_int, [ctypes.POINTER(FinishDesc), c_int32, c_double, c_void_p, c_size_t,
                                        c_void_p]),
    "smx_adamw": (c_int, [ctypes.POINTER(AdamwDesc), c_int32, c_int64, c_double, c_double, c_double, c_double,
                          c_double, c_void_p]),
    "smx_adamw_table_bytes": (c_size_t, [c_int32, c_int64]),
    "smx_adamw_staged": (c_int, [ctypes.POINTER(AdamwDesc), c_int32, c_int64, c_double, c_double, c_double,
                                 c_double, c_double, c_void_p, c_size_t, c_void_p]),
    "smx_matrix_step_workspace_bytes": (c_size_t, [ctypes.POINTER(c_int64), ctypes.POINTER(c_int64),
                                                   c_int32, c_int]),
    "smx_matrix_step": (c_int, [ctypes.POINTER(MatrixDesc), c_int32, c_int, c_void_p, c_size_t, c_void_p]),
    "smx_matrix_step_static": (c_int, [ctypes.POINTER(MatrixDesc), c_int32, c_int, c_void_p]),
    "smx_s8_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int]),
    "smx_s8": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int,
                       c_void_p, c_size_t, c_void_p]),
    "smx_inverse_sqrt": (c_int, [c_int, c_int, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                 c_void_p]),
    "smx_rank1_apply": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "smx_graft": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p]),
    "smx_s8_comp_stages": (c_int, [c_int32]),
    "smx_s8_comp_mask": (c_int, [c_int32]),
    "smx_s8_tile_geometry": (c_int, [c_int32]),
    "smx_mfma_peak": (c_int, [c_int32, c_int32, c_int64, c_void_p, c_void_p, c_void_p]),
    "smx_s8_timing": (c_int, [c_int32]),
    "smx_s8_timing_read": (c_int32, [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(c_int32),
                                     ctypes.POINTER(c_double), c_int32]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the library once; raise loudly if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m sandmuon_amd.build` "
                    "(hipcc, gfx950). sandmuon_amd has no fallback path.")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            version = handle.smx_abi_version()
            if version != ABI_VERSION:
                raise ImportError(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}; rebuild it")
            _lib = handle
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().smx_last_error().decode(errors="replace")
        kind = _STATUS.get(rc, str(rc))
        if rc in (-1, -2, -3, -4, -5):
            raise ValueError(f"{what}: {kind}: {msg}")
        raise NativeError(f"{what}: {kind}: {msg}")


def require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what}: sandmuon_amd runs on ROCm GPU tensors only (got {t.device})")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_busy(device: torch.device) -> bool:
    """True while work enqueued on the current stream of `device` has not
    finished (hipStreamQuery through torch).  A stream under graph capture
    cannot be queried and counts as busy."""
    with torch.cuda.device(device):
        if torch.cuda.is_current_stream_capturing():
            return True
        return not torch.cuda.current_stream(device).query()


def stream_of(device: torch.device) -> int:
    """The current stream of `device` (the autograd device stream inside a
    backward hook) as a hipStream_t value."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


_streams = {}  # (raw stream, device index) -> torch stream object


def torch_stream(stream: int, device: torch.device) -> torch.cuda.Stream:
    """The torch stream object of a raw hipStream_t of `device`.  The null
    handle is the default stream: torch.cuda.ExternalStream(0) would hand
    out a new pool stream instead."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (stream, index)
    s = _streams.get(key)
    if s is None:
        dev = torch.device("cuda", index)
        s = torch.cuda.default_stream(dev) if stream == 0 else torch.cuda.ExternalStream(stream, device=dev)
        _streams[key] = s
    return s


def stream_wait(waiter: int, signaler: int, device: torch.device) -> None:
    """Makes stream `waiter` wait for the work enqueued so far on stream
    `signaler` (raw hipStream_t values of `device`)."""
    done = torch.cuda.Event()
    done.record(torch_stream(signaler, device))
    torch_stream(waiter, device).wait_event(done)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------ wrappers ---
def stats_accumulate(rows2d: torch.Tensor, slots_sq: torch.Tensor, slots_first: Optional[torch.Tensor]) -> None:
    rc = lib().smx_stats_accumulate(rows2d.data_ptr(), dtype_code(rows2d.dtype), rows2d.shape[0],
                                    rows2d.shape[1], rows2d.stride(0), slots_sq.data_ptr(),
                                    ptr(slots_first), slots_sq.shape[0], stream_of(rows2d.device))
    _check(rc, "smx_stats_accumulate")
    _record_use(rows2d, stream_of(rows2d.device))


def _record_use(t: torch.Tensor, stream: int) -> None:
    """Tells the caching allocator that `t` is read by work enqueued on
    `stream` (a raw hipStream_t of t's device), which need not be the stream
    t was allocated on: its memory is then not handed to another allocation
    before that work has run."""
    t.record_stream(torch_stream(stream, t.device))


@functools.lru_cache(maxsize=256)
def stats_slot_rows(rows: int, n_slots: int) -> int:
    """Leading slot rows (of n_slots) a statistics call over `rows` rows adds into."""
    n = lib().smx_stats_slot_rows(rows, n_slots)
    _check(min(n, 0), "smx_stats_slot_rows")
    return n


def stats_accumulate_batch(entries, stream: int) -> None:
    """One launch over several hook inputs: entries of (rows2d, slots_sq,
    slots_first) whose slot rows are pairwise distinct."""
    descs = (StatsDesc * len(entries))()
    for d, (rows2d, sq, fs) in zip(descs, entries):
        d.x, d.slots_sq, d.slots_first = rows2d.data_ptr(), sq.data_ptr(), ptr(fs)
        d.rows, d.cols, d.row_stride = rows2d.shape[0], rows2d.shape[1], rows2d.stride(0)
        d.dtype, d.n_slots = dtype_code(rows2d.dtype), sq.shape[0]
    rc = lib().smx_stats_accumulate_batch(descs, len(entries), stream)
    _check(rc, "smx_stats_accumulate_batch")
    for rows2d, _, _ in entries:
        _record_use(rows2d, stream)


def stats_cast(rows2d: torch.Tensor, slots_sq: torch.Tensor, slots_first: Optional[torch.Tensor],
               out2d: torch.Tensor) -> None:
    """A statistic of an fp32 [rows, cols] view plus its bf16/f16 copy in out2d."""
    rc = lib().smx_stats_cast(rows2d.data_ptr(), dtype_code(rows2d.dtype), rows2d.shape[0], rows2d.shape[1],
                              rows2d.stride(0), slots_sq.data_ptr(), ptr(slots_first), slots_sq.shape[0],
                              out2d.data_ptr(), dtype_code(out2d.dtype), out2d.stride(0),
                              stream_of(rows2d.device))
    _check(rc, "smx_stats_cast")


def stats_gelu(rows2d: torch.Tensor, out2d: torch.Tensor, part_sq: torch.Tensor, part_first: Optional[torch.Tensor],
               n_slots: int) -> None:
    """out2d = GELU(rows2d) (bf16/f16) with the per-chunk partial sums of
    out2d's statistic in part_sq / part_first ([chunks, cols] FP32)."""
    rc = lib().smx_stats_gelu(rows2d.data_ptr(), dtype_code(rows2d.dtype), rows2d.shape[0], rows2d.shape[1],
                              rows2d.stride(0), out2d.data_ptr(), out2d.stride(0), part_sq.data_ptr(),
                              ptr(part_first), n_slots, stream_of(rows2d.device))
    _check(rc, "smx_stats_gelu")


def stats_relayout(x4: torch.Tensor, out: torch.Tensor, part_sq: torch.Tensor, part_first: Optional[torch.Tensor],
                   n_slots: int) -> None:
    """out (contiguous, x4's numel) = the row-major copy of the [batch, seq,
    heads, head_dim] view x4 (unit last stride), with the per-chunk partials
    of out's statistic in part_sq / part_first ([chunks, heads*head_dim])."""
    b, t, h, d = x4.shape
    sb, st, sh, sd = x4.stride()
    if sd != 1 and d > 1:
        raise ValueError("stats_relayout: the last dimension must have unit stride")
    rc = lib().smx_stats_relayout(x4.data_ptr(), dtype_code(x4.dtype), b, t, h, d, sb, st, sh, out.data_ptr(),
                                  part_sq.data_ptr(), ptr(part_first), n_slots, stream_of(x4.device))
    _check(rc, "smx_stats_relayout")


def stats_add_partials(slots_sq: torch.Tensor, part_sq: torch.Tensor, slots_first: Optional[torch.Tensor],
                       part_first: Optional[torch.Tensor]) -> None:
    """slots[:chunks] += partials (FP32), chunks = part_sq.shape[0]."""
    rc = lib().smx_stats_add_partials(slots_sq.data_ptr(), part_sq.data_ptr(), ptr(slots_first), ptr(part_first),
                                      part_sq.shape[1], part_sq.shape[0], stream_of(part_sq.device))
    _check(rc, "smx_stats_add_partials")


def stats_colsum_workspace_bytes(cols: int, n_slots: int) -> int:
    n = lib().smx_stats_colsum_workspace_bytes(cols, n_slots)
    _check(min(n, 0), "smx_stats_colsum_workspace_bytes")
    return n


def stats_colsum(rows2d: torch.Tensor, slots_sq: torch.Tensor, colsum: torch.Tensor,
                 workspace: torch.Tensor) -> None:
    """B statistic of a [rows, cols] view plus colsum = its column sums."""
    rc = lib().smx_stats_colsum(rows2d.data_ptr(), dtype_code(rows2d.dtype), rows2d.shape[0], rows2d.shape[1],
                                rows2d.stride(0), slots_sq.data_ptr(), slots_sq.shape[0], colsum.data_ptr(),
                                workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                                stream_of(rows2d.device))
    _check(rc, "smx_stats_colsum")


def stats_fold(sum_sq, slots_sq, sum_first, slots_first) -> None:
    rc = lib().smx_stats_fold(sum_sq.data_ptr(), slots_sq.data_ptr(), ptr(sum_first), ptr(slots_first),
                              sum_sq.numel(), slots_sq.shape[0], stream_of(sum_sq.device))
    _check(rc, "smx_stats_fold")


# Descriptors per launch of the by-value entry points (kernel arguments);
# longer tables go through the staged ones.
FINISH_BATCH = 32
ADAMW_BATCH = 56


class DescriptorStage:
    """Device tables for the staged entry points (smx_stats_finish_staged,
    smx_adamw_staged), each slot with an event recorded on the stream after
    its call.  The library writes a table in order on the call's stream (the
    descriptors travel in kernel arguments), so on one stream a table could
    be reused at once; the events keep a table whose kernels have not run
    from being rewritten by a call on another stream.  A call takes the
    first free slot, or waits for the oldest when all MAX_SLOTS are in
    flight, so several staged calls of one step (the finish, an AdamW call
    per parameter group) never wait on each other.

    The slots are allocated together and all of one size, a power of two of
    at least MIN_BYTES that covers the largest table staged so far, so a
    step whose tables fit allocates nothing.  (Under graph capture, where the
    host cannot wait on an event, the by-value calls are used.)"""

    MAX_SLOTS = 8
    MIN_BYTES = 1 << 16

    def __init__(self, device: torch.device):
        self.device = device
        self.size = 0
        self.slots: List[list] = []  # [device table, event], oldest use first

    def _grow(self, nbytes: int) -> None:
        for sl in self.slots:  # queued kernels still read these tables
            if sl[1] is not None:
                sl[1].synchronize()
        self.size = max(self.MIN_BYTES, 1 << (int(nbytes) - 1).bit_length())
        self.slots = [[torch.empty(self.size, dtype=torch.uint8, device=self.device), None]
                      for _ in range(self.MAX_SLOTS)]

    def take(self, nbytes: int):
        if nbytes > self.size:
            self._grow(nbytes)
        free = [i for i, sl in enumerate(self.slots) if sl[1] is None or sl[1].query()]
        slot = self.slots.pop(free[0] if free else 0)
        if not free:
            slot[1].synchronize()
        self.slots.append(slot)  # most recent use last
        return slot

    def done(self, slot) -> None:
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        slot[1] = ev


def stats_finish(descs: Sequence[FinishDesc], beta: float, device: torch.device,
                 stage: Optional[DescriptorStage] = None) -> None:
    """Finish of every vector: one fold and one finish launch per FINISH_BATCH
    descriptors, or one of each for the whole table through `stage`."""
    if not descs:
        return
    arr = (FinishDesc * len(descs))(*descs)
    if stage is None or len(descs) <= FINISH_BATCH or torch.cuda.is_current_stream_capturing():
        _check(lib().smx_stats_finish(arr, len(descs), beta, stream_of(device)), "smx_stats_finish")
        return
    nbytes = int(lib().smx_stats_finish_table_bytes(len(descs)))
    slot = stage.take(nbytes)
    _check(lib().smx_stats_finish_staged(arr, len(descs), beta, slot[0].data_ptr(), slot[0].numel(),
                                         stream_of(device)), "smx_stats_finish_staged")
    stage.done(slot)


def adamw(descs: Sequence[AdamwDesc], total: int, lr: float, beta1: float, beta2: float, eps: float,
          weight_decay: float, device: torch.device, stage: Optional[DescriptorStage] = None) -> None:
    """AdamW over every tensor: one launch per ADAMW_BATCH descriptors, or one
    for the whole table through `stage`."""
    if not descs:
        return
    arr = (AdamwDesc * len(descs))(*descs)
    if stage is None or len(descs) <= ADAMW_BATCH or torch.cuda.is_current_stream_capturing():
        _check(lib().smx_adamw(arr, len(descs), total, lr, beta1, beta2, eps, weight_decay, stream_of(device)),
               "smx_adamw")
        return
    nbytes = int(lib().smx_adamw_table_bytes(len(descs), total))
    slot = stage.take(nbytes)
    _check(lib().smx_adamw_staged(arr, len(descs), total, lr, beta1, beta2, eps, weight_decay, slot[0].data_ptr(),
                                  slot[0].numel(), stream_of(device)), "smx_adamw_staged")
    stage.done(slot)


def matrix_step_workspace_bytes(shapes: Sequence[tuple], mode: int) -> int:
    n = len(shapes)
    rows = (c_int64 * n)(*[s[0] for s in shapes])
    cols = (c_int64 * n)(*[s[1] for s in shapes])
    return int(lib().smx_matrix_step_workspace_bytes(rows, cols, n, mode))


def matrix_step(descs: Sequence[MatrixDesc], mode: int, workspace: torch.Tensor) -> None:
    if not descs:
        return
    arr = (MatrixDesc * len(descs))(*descs)
    _check(lib().smx_matrix_step(arr, len(descs), mode, workspace.data_ptr(), workspace.numel(),
                                 stream_of(workspace.device)), "smx_matrix_step")


S8_PHASES = {0: "gram", 1: "square", 2: "apply", 3: "poly1", 4: "run", 5: "sym"}


def s8_timing(enable, runs_only: bool = False) -> None:
    """Start (discarding earlier records) or stop the S8 launch recorder.
    With runs_only, only whole S8 runs are recorded (two events per run)."""
    level = 0 if not enable else (2 if runs_only else 1)
    _check(lib().smx_s8_timing(level), "smx_s8_timing")


def s8_timing_read(capacity: int = 4096):
    """Recorded S8 launches as (ms, phase name, issued MFMA FLOPs); waits for them."""
    ms = (ctypes.c_float * capacity)()
    ph = (c_int32 * capacity)()
    fl = (c_double * capacity)()
    n = lib().smx_s8_timing_read(ms, ph, fl, capacity)
    _check(min(n, 0), "smx_s8_timing_read")
    return [(ms[i], S8_PHASES[ph[i]], fl[i]) for i in range(n)]


def s8(x: torch.Tensor, out: torch.Tensor, mode: int) -> None:
    """x, out: [batch, rows, cols] float32 on the GPU (any strides)."""
    b, r, c = x.shape
    nbytes = int(lib().smx_s8_workspace_bytes(b, r, c, mode))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    if out.stride() != x.stride():
        raise ValueError("s8: out must have the strides of x")
    rc = lib().smx_s8(x.data_ptr(), out.data_ptr(), b, r, c, x.stride(0), x.stride(1), x.stride(2), mode,
                      ws.data_ptr(), ws.numel(), stream_of(x.device))
    _check(rc, "smx_s8")


_HELPER_DTYPES = {torch.float32: SMX_F32, torch.float64: SMX_F64}


def helper_dtype_code(dtype: torch.dtype) -> int:
    try:
        return _HELPER_DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported helper dtype {dtype}; expected float32 or float64") from None


def inverse_sqrt(kind: int, second: torch.Tensor, mean: Optional[torch.Tensor], inv: torch.Tensor,
                 z: Optional[torch.Tensor], kappa: Optional[torch.Tensor]) -> None:
    """kind 0: diagonal_inverse_sqrt of `second`; kind 1: rank1_inverse_sqrt
    of (second, mean) into inv, z, kappa.  Contiguous 1-D tensors of one
    dtype (float32 or float64) on the GPU."""
    rc = lib().smx_inverse_sqrt(kind, helper_dtype_code(second.dtype), second.data_ptr(), ptr(mean),
                                second.numel(), inv.data_ptr(), ptr(z), ptr(kappa), stream_of(second.device))
    _check(rc, "smx_inverse_sqrt")


def rank1_apply(x: torch.Tensor, out: torch.Tensor, left, right, order: int) -> None:
    """x, out: contiguous [batch, rows, cols]; left/right: (inv, z, coef) of
    shapes [batch, n], [batch, n], [batch], all of x's dtype."""
    b, r, c = x.shape
    li, lz, lc = left
    ri, rz, rc_ = right
    work = torch.empty(max(b * (r + c), 1), dtype=torch.float64, device=x.device)
    rc = lib().smx_rank1_apply(helper_dtype_code(x.dtype), x.data_ptr(), out.data_ptr(), b, r, c, li.data_ptr(),
                               lz.data_ptr(), lc.data_ptr(), ri.data_ptr(), rz.data_ptr(), rc_.data_ptr(), order,
                               work.data_ptr(), stream_of(x.device))
    _check(rc, "smx_rank1_apply")


def graft(x: torch.Tensor, out: torch.Tensor, output_rows: int) -> None:
    work = torch.empty(1024, dtype=torch.float64, device=x.device)
    rc = lib().smx_graft(x.data_ptr(), out.data_ptr(), x.numel(), output_rows, work.data_ptr(), 1024,
                         stream_of(x.device))
    _check(rc, "smx_graft")


def s8_tile_geometry(policy: int) -> int:
    """Sets the S8 GEMM tile geometry policy (0 automatic, 1 256 x 256 tiles
    for every launch, 2 never 256 x 256; a test aid); returns the old value."""
    prev = lib().smx_s8_tile_geometry(int(policy))
    _check(min(prev, 0), "smx_s8_tile_geometry")
    return prev


def s8_comp_stages(k: int) -> int:
    """Sets how many S8 stages of the compensated-BF16 mode are compensated
    (a measurement aid; 5 is the production recipe); returns the old value."""
    prev = lib().smx_s8_comp_stages(int(k))
    _check(min(prev, 0), "smx_s8_comp_stages")
    return prev


def s8_comp_mask(mask: int) -> int:
    """Sets which S8 stages of the compensated-BF16 mode are compensated (bit
    k-1: stage k; the others are plain BF16 products; a measurement aid,
    0x1f is the production recipe); returns the old mask."""
    prev = lib().smx_s8_comp_mask(int(mask))
    _check(min(prev, 0), "smx_s8_comp_mask")
    return prev


def mfma_peak(dtype: torch.dtype, iters: int, device, blocks: Optional[int] = None) -> dict:
    """The MFMA peak probe (smx_mfma_peak): dense MFMAs from registers on
    every SIMD of the device (blocks = one per CU by default), timed with
    events on the current stream.  Returns the sustained TFLOP/s, the engine
    clock held (GHz, from s_memtime against the 100 MHz s_memrealtime) and
    the nominal rate at that clock (4096 BF16/FP16 or 256 FP32 FLOP per
    clock per CU)."""
    code = {torch.float32: SMX_F32, torch.bfloat16: SMX_BF16, torch.float16: SMX_F16}[dtype]
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks = blocks or cus
    times = torch.zeros(blocks * 4, dtype=torch.int64, device=device)
    sink = torch.empty(blocks * 512, dtype=torch.float32, device=device)
    st = stream_of(device)
    _check(lib().smx_mfma_peak(code, blocks, 1, times.data_ptr(), sink.data_ptr(), st), "smx_mfma_peak")  # warm
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    _check(lib().smx_mfma_peak(code, blocks, int(iters), times.data_ptr(), sink.data_ptr(), st), "smx_mfma_peak")
    b.record()
    torch.cuda.synchronize(device)
    ms = a.elapsed_time(b)
    per_mfma = 4096 if code == SMX_F32 else 32768
    flops = blocks * 8 * 4 * int(iters) * per_mfma
    t = times.view(blocks, 4).cpu().double()
    ghz = float(((t[:, 1] - t[:, 0]) / (t[:, 3] - t[:, 2])).median()) * 0.1
    per_clk = 256 if code == SMX_F32 else 4096
    return {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "clock_ghz": round(ghz, 3),
            "nominal_tflops_at_clock": round(cus * per_clk * ghz * 1e9 / 1e12, 1), "ms": round(ms, 3),
            "blocks": blocks, "iters": int(iters), "finite": bool(torch.isfinite(sink).all())}
