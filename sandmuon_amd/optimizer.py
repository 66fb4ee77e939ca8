"""SandMuon optimizer on MI355X: the public API of sandmuon/optimizer.py with
every tensor operation of the hooks and of step() running in the gfx950 HIP
kernels of libsandmuon_amd.so.

Drop-in surface (sandmuon/optimizer.py:96-328): DiagonalWeightedPE,
RankOneAWeightedPE, module_filter, the forward/cotangent hooks, step(),
state_dict()/load_state_dict() (same state keys and types; the load keeps
the statistics, momentum and moments float32 for 16-bit parameters) and
close().  The module-level helpers imported by the reference tests
(_s8_fp32, diagonal_inverse_sqrt, _graft_direction, rank1_inverse_sqrt,
rank1_mapback, rank1_whiten) are GPU-backed here as well.

Added keywords (defaults keep the production recipe and the reference's
results):
* ``s8_mode`` selects the arithmetic of the S8 products: "comp_bf16"
  (compensated BF16 MFMA in all five stages), "mixed" (compensated BF16
  stages 1-2, FP16 MFMA stages 3-5: about 1e-3 from the FP32 map at a
  quarter less S8 time) or "fp32" (FP32 MFMA);
* ``hook_batch_bytes``: the hooks queue their inputs and take the
  statistics of the queue in one launch once it holds this many bytes (and
  at step(), state_dict() and close()); 0 launches in every hook call.  The
  statistics are bit-identical either way.  A queued input must not be
  modified in place before its launch: the launch checks the tensor's
  version counter and raises RuntimeError if it moved.
"""
from __future__ import annotations

import math
import re
from typing import Callable, Dict, List, Optional, Tuple

import torch
from torch import nn
from torch.optim import Optimizer

from . import _native
from .coefficients import S8_COEFFICIENTS, S8_MARGIN, S8_MULTIPLIER

__all__ = [
    "DiagonalWeightedPE", "RankOneAWeightedPE", "diagonal_inverse_sqrt", "rank1_inverse_sqrt",
    "rank1_whiten", "rank1_mapback", "_graft_direction", "_s8_fp32",
]

# q/k/v activation-statistic sharing rule (sandmuon/optimizer.py:129-135).
_QKV_SHARE = re.compile(r"^(transformer\.h\.\d+\.attn\.)[kv]_proj\.weight$")

_KIND_DIAG_A, _KIND_RANK1_A, _KIND_B = 0, 1, 2


# --------------------------------------------------------------- helpers ---
# The module-level helpers run in float64 when their input is float64 and
# in float32 otherwise, as the reference computes them in the input dtype;
# _graft_direction and _s8_fp32 work in float32, as the reference's do.
def _to_gpu(t, dtype: torch.dtype) -> torch.Tensor:
    t = torch.as_tensor(t)
    if t.device.type != "cuda":
        if not torch.cuda.is_available():
            raise RuntimeError("sandmuon_amd needs a ROCm GPU; none is available")
        t = t.to(torch.device("cuda", torch.cuda.current_device()))
    return t.to(dtype).contiguous()


def _to_gpu_f32(t) -> torch.Tensor:
    return _to_gpu(t, torch.float32)


def _work_dtype(*tensors) -> torch.dtype:
    """float64 if any input is float64, else float32."""
    return torch.float64 if any(torch.as_tensor(t).dtype == torch.float64 for t in tensors) else torch.float32


def diagonal_inverse_sqrt(value: torch.Tensor) -> torch.Tensor:
    """Mean-normalised diagonal inverse square root (sandmuon/optimizer.py:19-24)."""
    dt = _work_dtype(value)
    v = _to_gpu(value, dt).reshape(-1)
    if v.numel() == 0:
        return value.new_empty(value.shape)
    inv = torch.empty_like(v)
    _native.inverse_sqrt(0, v, None, inv, None, None)
    return inv.reshape(value.shape).to(value.device, value.dtype)


def rank1_inverse_sqrt(second: torch.Tensor, mean: torch.Tensor):
    """D^-1/2 and the Sherman-Morrison rank-one (z, kappa) (sandmuon/optimizer.py:27-35)."""
    dt = _work_dtype(second, mean)
    s = _to_gpu(second, dt).reshape(-1)
    m = _to_gpu(mean, dt).reshape(-1)
    inv, z = torch.empty_like(s), torch.empty_like(s)
    kappa = torch.empty((), dtype=dt, device=s.device)
    _native.inverse_sqrt(1, s, m, inv, z, kappa)
    out_dtype = torch.promote_types(second.dtype, mean.dtype)
    out = lambda t: t.to(second.device, out_dtype)
    return out(inv), out(z), out(kappa)


def _batched_factor(f, batch_shape, n, dt):
    vec = _to_gpu(f[0], dt).expand(*batch_shape, n).reshape(-1, n).contiguous()
    z = _to_gpu(f[1], dt).expand(*batch_shape, n).reshape(-1, n).contiguous()
    c = _to_gpu(f[2], dt).expand(torch.Size(batch_shape)).reshape(-1).contiguous()
    return vec, z, c


def _rank1(matrix: torch.Tensor, left, right, order: int) -> torch.Tensor:
    dt = _work_dtype(matrix, *left, *right)
    x = _to_gpu(matrix, dt)
    r, c = x.shape[-2], x.shape[-1]
    batch_shape = x.shape[:-2]
    xb = x.reshape(-1, r, c)
    out = torch.empty_like(xb)
    lf = _batched_factor(left, batch_shape, r, dt)
    rf = _batched_factor(right, batch_shape, c, dt)
    _native.rank1_apply(xb, out, lf, rf, order)
    res = out.reshape(x.shape)
    return res.to(matrix.device, torch.promote_types(matrix.dtype, dt))


def rank1_whiten(matrix: torch.Tensor, left, right) -> torch.Tensor:
    """Dense left/right rank-one whiteners without forming matrices (sandmuon/optimizer.py:38-45)."""
    return _rank1(matrix, left, right, 0)


def rank1_mapback(value: torch.Tensor, left, right) -> torch.Tensor:
    """Rank-one factors, then diagonals (sandmuon/optimizer.py:48-60)."""
    return _rank1(value, left, right, 1)


def _graft_direction(value: torch.Tensor, output_rows: int) -> torch.Tensor:
    """Frobenius graft to sqrt(output_rows) in float32 (sandmuon/optimizer.py:63-66)."""
    v = _to_gpu_f32(value)
    out = torch.empty_like(v)
    _native.graft(v, out, int(output_rows))
    return out.to(value.device)


def _s8_fp32(x: torch.Tensor, mode: str = "fp32") -> torch.Tensor:
    """S8 polar map on [..., rows, cols] (sandmuon/optimizer.py:69-93), FP32 MFMA by default."""
    v = _to_gpu_f32(x)
    r, c = v.shape[-2], v.shape[-1]
    vb = v.reshape(-1, r, c)
    out = torch.empty_like(vb)
    _native.s8(vb, out, _native.S8_MODES[mode])
    return (out.reshape(v.shape) * S8_MULTIPLIER).to(x.device)


_PARAM_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
# Optimizer state kept in float32 whatever the parameter dtype (the kernels
# read and write it as FP32; sandmuon/optimizer.py creates it float32).
_FP32_STATE = ("a_sum", "a_first_sum", "b_sum", "a_ema", "a_mean_ema", "b_ema", "momentum_buffer",
               "exp_avg", "exp_avg_sq")


def _dense(t: torch.Tensor) -> bool:
    """Whether t's elements fill its storage span without gaps or overlap
    (any dimension order), so that an elementwise kernel can walk it flat."""
    if t.is_contiguous():
        return True
    dims = sorted((st, n) for st, n in zip(t.stride(), t.shape) if n != 1)
    expect = 1
    for st, n in dims:
        if st != expect:
            return False
        expect *= n
    return True


def _check_layout(parameter: torch.Tensor, name: str, matrix: bool) -> None:
    """Matrix kernels read parameters as row-major [rows, cols]; the
    elementwise AdamW kernel walks any gap-free layout."""
    if matrix and not parameter.is_contiguous():
        raise ValueError(f"sandmuon_amd needs row-major contiguous matrix parameters; {name} has strides "
                         f"{tuple(parameter.stride())} (call .contiguous() on it before building the optimizer)")
    if not matrix and not _dense(parameter):
        raise ValueError(f"sandmuon_amd needs parameters without gaps or overlap; {name} has strides "
                         f"{tuple(parameter.stride())}")


def _require_f32(t: torch.Tensor, n: int, device, what: str) -> torch.Tensor:
    """A state vector the kernels read and write as n contiguous FP32 values
    on `device`; anything else is refused before a launch gets its pointer."""
    if (not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.numel() != n or
            not t.is_contiguous() or t.device != device):
        desc = (f"{t.dtype}, {t.numel()} elements, contiguous={t.is_contiguous()}, {t.device}"
                if isinstance(t, torch.Tensor) else type(t).__name__)
        raise ValueError(f"optimizer state {what} must be a contiguous float32 tensor of {n} elements on "
                         f"{device} (got {desc})")
    return t


def _like(t: torch.Tensor, parameter: torch.Tensor, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """t (same shape as `parameter`) with the parameter's strides: as it is
    when they already match, else copied into the parameter's layout."""
    if t.stride() == parameter.stride() and (dtype is None or t.dtype == dtype):
        return t
    return torch.empty_like(parameter, dtype=dtype or t.dtype).copy_(t)


def select_matrices(model: nn.Module, module_filter=None):
    """Selected matrices and their modules, in named_modules() order.

    sandmuon/optimizer.py:106-118: every module accepted by the filter
    (default: every nn.Linear) whose `.weight` is a trainable 2-D Parameter.
    """
    choose = module_filter or (lambda name, module: isinstance(module, nn.Linear))
    matrices: Dict[str, nn.Parameter] = {}
    modules: Dict[str, nn.Module] = {}
    for name, module in dict(model.named_modules()).items():
        if name and choose(name, module):
            parameter = getattr(module, "weight", None)
            if isinstance(parameter, nn.Parameter) and parameter.requires_grad and parameter.ndim == 2:
                matrices[name + ".weight"] = parameter
                modules[name + ".weight"] = module
    if not matrices:
        raise ValueError("No eligible trainable linear weights found")
    return matrices, modules


def shared_source(name: str, matrices: Dict[str, nn.Parameter]) -> str:
    """Name of the matrix whose activation statistic `name` uses.

    sandmuon/optimizer.py:128-135: transformer.h.N.attn.{k,v}_proj share the
    statistic of the same block's q_proj when it is selected; every other
    matrix is its own source.
    """
    match = _QKV_SHARE.match(name)
    if match and (match.group(1) + "q_proj.weight") in matrices:
        return match.group(1) + "q_proj.weight"
    return name


def _rows2d(t: torch.Tensor) -> torch.Tensor:
    """[..., d] -> [N, d] view with unit column stride (hook input layout)."""
    _native.require_gpu(t, "statistics hook")
    rows = t.detach().reshape(-1, t.shape[-1])
    if rows.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        rows = rows.float()
    if rows.shape[1] > 1 and rows.stride(1) != 1:
        rows = rows.contiguous()
    return rows


class _StatsQueue:
    """Hook inputs whose statistics are still to be taken, in hook order.

    Every entry adds into its own slot rows (an entry whose slot rows are
    already queued flushes the queue first), so one launch over the whole
    queue adds exactly what one launch per hook call would, in the same
    order per slot row.  The queue keeps its tensors alive until the launch
    is enqueued on the stream current at the first hook call.

    A phase of hooks (from construction or a step to the next step) starts
    by asking whether the stream of its first hook call still has work.
    If it has (the step itself, a forward pass), every launch takes `limit`
    bytes: the GPU is busy while the queue fills.  If the stream is idle,
    the launch threshold ramps up instead: the first launch takes `first`
    bytes and each later one `growth` times more, up to `limit`, so the GPU
    starts reading after a few hook calls rather than after a full batch
    (Python queues hook inputs only somewhat faster than the GPU reads
    them), and the batches still reach the full size.  Small launches
    leave part of the device idle, so the ramp is only taken when it helps.
    """

    __slots__ = ("limit", "first", "growth", "threshold", "fresh", "entries", "slot_ptrs", "nbytes", "stream",
                 "device")

    def __init__(self, limit: int, first: int = 64 << 20, growth: float = 1.6):
        self.limit = int(limit)
        self.first = int(first)
        self.growth = float(growth)
        self.threshold = min(self.limit, self.first)
        self.fresh = True  # the next hook call is the first of a phase
        self.entries: List[Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], int]] = []
        self.slot_ptrs = set()
        self.nbytes = 0
        self.stream = None
        self.device = None

    def grow(self) -> None:
        """The next launch threshold, after a launch."""
        self.threshold = min(self.limit, int(self.threshold * self.growth))

    def restart(self) -> None:
        """A new phase of hooks begins (the statistics were consumed)."""
        self.threshold = min(self.limit, self.first)
        self.fresh = True

    def start_phase(self, busy: bool) -> None:
        """At the phase's first hook call: no ramp when the GPU is busy."""
        self.fresh = False
        if busy:
            self.threshold = self.limit

    def clear(self) -> None:
        self.entries = []
        self.slot_ptrs = set()
        self.nbytes = 0
        self.stream = self.device = None


# ------------------------------------------------------------- optimizer ---
class DiagonalWeightedPE(Optimizer):
    """S8 directions weighted by activation and output-cotangent diagonals.

    Mirrors sandmuon/optimizer.py:96-321.  Statistics are accumulated from
    every forward/backward microbatch between optimizer steps; defaults
    match the 103M run (beta .97, momentum .8, S8 margin 1.35, AdamW LR
    ratio .1 and decay .01).
    """

    # Slot rows per statistics vector: each hook launch spreads its rows over
    # this many row chunks, each chunk owning one slot row.
    STAT_SLOTS = 128
    # Queued hook bytes that trigger a statistics launch.  One launch per
    # hook call pays a fixed start/drain cost that is large against the
    # 25-100 MB of one call; launches over 1 GB run near the streaming rate.
    HOOK_BATCH_BYTES = 1 << 30

    def __init__(self, model: nn.Module, lr: float, *, rank_one_a: bool = False,
                 module_filter: Optional[Callable[[str, nn.Module], bool]] = None,
                 s8_mode: str = "comp_bf16", hook_batch_bytes: Optional[int] = None):
        matrices, modules = select_matrices(model, module_filter)
        if s8_mode not in _native.S8_MODES:
            raise ValueError(f"s8_mode must be one of {sorted(_native.S8_MODES)}")
        limit = self.HOOK_BATCH_BYTES if hook_batch_bytes is None else int(hook_batch_bytes)
        if limit < 0:
            raise ValueError("hook_batch_bytes must be >= 0")
        _native.lib()  # fails loudly without the HIP library

        self.named_matrices = matrices
        self.parameter_names = {id(p): name for name, p in matrices.items()}
        self.rank_one_a = bool(rank_one_a)
        self.statistic_beta = .97
        self.s8_coefficients = S8_COEFFICIENTS
        self.s8_margin = S8_MARGIN
        self.s8_mode = s8_mode
        self._group_constants = {}

        self.a_sources = {id(p): matrices[shared_source(name, matrices)] for name, p in matrices.items()}

        matrix_ids = {id(p) for p in matrices.values()}
        auxiliary = [p for p in model.parameters() if p.requires_grad and id(p) not in matrix_ids]
        matrix_names = {id(p): name for name, p in matrices.items()}
        devices = {p.device for p in list(matrices.values()) + auxiliary}
        if len(devices) > 1:
            raise ValueError("sandmuon_amd runs one optimizer per GPU: every parameter must be on one device "
                             f"(got {sorted(str(d) for d in devices)})")
        for p in list(matrices.values()) + auxiliary:
            if p.device.type != "cuda":
                raise RuntimeError("sandmuon_amd runs on ROCm GPU parameters only; move the model to the GPU "
                                   f"before constructing the optimizer (got {p.device})")
            if p.dtype not in _PARAM_DTYPES:
                raise TypeError(f"sandmuon_amd expects float32, bfloat16 or float16 parameters (got {p.dtype})")
            _check_layout(p, matrix_names.get(id(p), "an auxiliary parameter"), id(p) in matrix_names)
        defaults = dict(lr=float(lr), use_muon=True, momentum=.8, weight_decay=0.,
                        adamw_lr_ratio=.1, adamw_betas=(.9, .999), adamw_eps=1e-8)
        groups = [dict(params=list(matrices.values()), use_muon=True)]
        if auxiliary:
            groups.append(dict(params=auxiliary, use_muon=False, weight_decay=.01))
        super().__init__(groups, defaults)
        # Pending per-chunk partial sums of the hooks, folded into a_sum /
        # b_sum by step() (or before state_dict()).  Not optimizer state.
        self._slots: Dict[Tuple[int, str], Tuple[nn.Parameter, torch.Tensor, Optional[torch.Tensor]]] = {}
        self._queue = _StatsQueue(limit)
        # Leading slot rows any call has added into since the last fold, per
        # slot buffer (data pointer): the fold and finish read only those.
        self._slot_rows: Dict[int, int] = {}
        self._workspace: Optional[torch.Tensor] = None
        # Device tables for the finish and AdamW launches of a step with more
        # descriptors than one by-value launch takes (created on first use).
        self._stage: Optional[_native.DescriptorStage] = None
        self.register_state_dict_pre_hook(DiagonalWeightedPE._flush_slots)
        self.register_load_state_dict_post_hook(DiagonalWeightedPE._drop_slots)
        self.handles = []
        self._matrix_modules = modules
        self._hook_handles = {}
        self._fused = None
        for name, module in modules.items():
            self._hook_handles[name] = self._install_hook(name)
            self.handles.append(self._hook_handles[name])

    def _install_hook(self, name: str):
        parameter = self.named_matrices[name]
        return self._matrix_modules[name].register_forward_hook(
            self._capture(parameter, capture_a=self.a_sources[id(parameter)] is parameter))

    # ------------------------------------------------------------ hooks ---
    def _slot_pair(self, parameter, side: str, n: int, device, first: bool):
        key = (id(parameter), side)
        entry = self._slots.get(key)
        if entry is None or entry[1].shape[1] != n:
            sq = torch.zeros(self.STAT_SLOTS, n, dtype=torch.float32, device=device)
            fs = torch.zeros_like(sq) if first else None
            entry = (parameter, sq, fs)
            self._slots[key] = entry
        return entry[1], entry[2]

    def _a_slots(self, parameter, n: int, device, state: dict):
        """State entries and slot rows the A statistic of `parameter` adds into."""
        if "a_sum" not in state:
            state["a_sum"] = torch.zeros(n, device=device, dtype=torch.float32)
            state["a_count"] = 0
            if self.rank_one_a:
                state["a_first_sum"] = torch.zeros_like(state["a_sum"])
        return self._slot_pair(parameter, "a", n, device, self.rank_one_a)

    def _b_slots(self, parameter, n: int, device, state: dict) -> torch.Tensor:
        if "b_sum" not in state:
            state["b_sum"] = torch.zeros(n, device=device, dtype=torch.float32)
            state["b_count"] = 0
        return self._slot_pair(parameter, "b", n, device, False)[0]

    def _accumulate_a(self, parameter, x: torch.Tensor, state: Optional[dict] = None) -> None:
        """Forward-hook body (sandmuon/optimizer.py:156-168): a_sum += sum x^2,
        a_first_sum += sum x (rank-one), a_count += rows."""
        state = self.state[parameter] if state is None else state
        rows = _rows2d(x)
        sq, fs = self._a_slots(parameter, rows.shape[-1], rows.device, state)
        self._enqueue_stats(rows, sq, fs)
        state["a_count"] += rows.shape[0]

    def _accumulate_b(self, parameter, delta: torch.Tensor, state: Optional[dict] = None) -> None:
        """Cotangent-hook body (sandmuon/optimizer.py:171-177): b_sum += sum delta^2."""
        state = self.state[parameter] if state is None else state
        rows = _rows2d(delta)
        sq = self._b_slots(parameter, rows.shape[-1], rows.device, state)
        self._enqueue_stats(rows, sq, None)
        state["b_count"] += rows.shape[0]

    def _note_slots(self, sq: torch.Tensor, rows: int) -> None:
        """Records the slot rows a statistics call over `rows` rows adds into."""
        n = _native.stats_slot_rows(rows, sq.shape[0])
        key = sq.data_ptr()
        if n > self._slot_rows.get(key, 0):
            self._slot_rows[key] = n

    def _take_slot_rows(self, sq: torch.Tensor) -> int:
        """Slot rows the next fold of `sq` must read (at least one); the count
        restarts, since the fold zeroes them."""
        return max(self._slot_rows.pop(sq.data_ptr(), 0), 1)

    def _enqueue_stats(self, rows: torch.Tensor, sq: torch.Tensor, fs: Optional[torch.Tensor]) -> None:
        """Queues one hook input (or launches at once when batching is off)."""
        q = self._queue
        self._note_slots(sq, rows.shape[0])
        if q.limit == 0:
            _native.stats_accumulate(rows, sq, fs)
            return
        if rows.shape[0] == 0:
            return  # an empty microbatch adds nothing
        stream = _native.stream_of(rows.device)
        if q.entries and (stream != q.stream or rows.device != q.device or sq.data_ptr() in q.slot_ptrs):
            self._flush_stats()
        if not q.entries:
            q.stream, q.device = stream, rows.device
            if q.fresh:
                q.start_phase(_native.stream_busy(rows.device))
        q.entries.append((rows, sq, fs, rows._version))
        q.slot_ptrs.add(sq.data_ptr())
        q.nbytes += rows.numel() * rows.element_size()
        if q.nbytes >= q.threshold:
            self._flush_stats()

    def _stats_barrier(self, sq: torch.Tensor) -> None:
        """Launches the queue if it adds into `sq`, so that an immediate launch
        into the same slot rows comes after it."""
        if sq.data_ptr() in self._queue.slot_ptrs:
            self._flush_stats()

    def _flush_stats(self) -> None:
        """Takes the statistics of every queued hook input in one launch, on
        the stream of the queued hook calls (the current stream waits for it
        when it is another one)."""
        q = self._queue
        if not q.entries:
            return
        entries, stream, device = q.entries, q.stream, q.device
        q.clear()
        q.grow()
        for rows, _, _, version in entries:
            if rows._version != version:
                raise RuntimeError(
                    "a hook input was modified in place before its statistics were taken; construct the "
                    "optimizer with hook_batch_bytes=0 to take them inside the hook")
        _native.stats_accumulate_batch([(rows, sq, fs) for rows, sq, fs, _ in entries], stream)
        current = _native.stream_of(device)
        if current != stream:
            _native.stream_wait(current, stream, device)

    def _capture(self, parameter, *, capture_a):
        def hook(module, inputs, output):
            if (not module.training or not torch.is_grad_enabled() or
                    not isinstance(output, torch.Tensor) or not output.requires_grad):
                return
            state = self.state[parameter]
            if capture_a:
                self._accumulate_a(parameter, inputs[0], state)

            def cotangent_hook(gradient):
                self._accumulate_b(parameter, gradient, state)
                return gradient
            output.register_hook(cotangent_hook)
        return hook

    @staticmethod
    def _flush_slots(self) -> None:
        """Folds pending hook partials into a_sum / b_sum (before state_dict())."""
        self._flush_stats()
        for (pid, side), (parameter, sq, fs) in self._slots.items():
            state = self.state.get(parameter, {})
            total = state.get(f"{side}_sum")
            if total is None:
                continue
            first = state.get("a_first_sum") if side == "a" and fs is not None else None
            name = self.parameter_names.get(pid, "a parameter")
            _require_f32(total, sq.shape[1], sq.device, f"{side}_sum of {name}")
            if first is not None:
                _require_f32(first, sq.shape[1], sq.device, f"a_first_sum of {name}")
            n = self._take_slot_rows(sq)
            _native.stats_fold(total, sq[:n], first, fs[:n] if first is not None else None)

    @staticmethod
    def _drop_slots(self) -> None:
        """Loaded sums are authoritative: pending partials are discarded."""
        self._queue.clear()
        self._slots.clear()
        self._slot_rows.clear()

    def load_state_dict(self, state_dict: dict) -> None:
        """torch's Optimizer.load_state_dict, keeping the FP32 state FP32.

        torch casts every floating state tensor to its parameter's dtype, so
        for a bf16/fp16 parameter the statistics, EMA, momentum and moment
        tensors would come back 16-bit.  The reference creates them FP32
        (sandmuon/optimizer.py:161,164,174,245,270-271) and the kernels read
        and write them as FP32, so they are restored from the saved values
        (not from the rounded copies) as contiguous float32 on the
        parameter's device.
        """
        saved_state = state_dict["state"]
        saved_ids = [i for g in state_dict["param_groups"] for i in g["params"]]
        params = [p for g in self.param_groups for p in g["params"]]
        keep = {}
        for saved_id, parameter in zip(saved_ids, params):
            entry = saved_state.get(saved_id)
            if entry is None:
                continue
            for key in _FP32_STATE:
                value = entry.get(key)
                if isinstance(value, torch.Tensor) and value.is_floating_point():
                    keep[(id(parameter), key)] = value
        super().load_state_dict(state_dict)
        for parameter in params:
            state = self.state.get(parameter)
            if not state:
                continue
            for key in _FP32_STATE:
                value = keep.get((id(parameter), key))
                if value is not None:
                    state[key] = value.to(device=parameter.device, dtype=torch.float32, copy=True).contiguous()

    # ------------------------------------------------------------- step ---
    def _finish_a_check(self, parameter) -> int:
        state = self.state[parameter]
        if state.get("a_count", 0) < 1:
            raise RuntimeError(f"Missing activation statistics: {self.parameter_names[id(parameter)]}")
        return state["a_count"]

    def _finish_b_check(self, parameter, expected_count: int) -> None:
        state = self.state[parameter]
        if state.get("b_count", 0) != expected_count:
            raise RuntimeError(f"Missing or mismatched cotangent statistics: {self.parameter_names[id(parameter)]}; "
                               f"expected {expected_count}, got {state.get('b_count', 0)}")

    def _finish_desc(self, parameter, side: str, count: int, out: Dict[str, torch.Tensor]) -> _native.FinishDesc:
        state = self.state[parameter]
        total = state[f"{side}_sum"]
        n = parameter.shape[1] if side == "a" else parameter.shape[0]
        rank1 = side == "a" and self.rank_one_a
        sq, fs = self._slot_pair(parameter, side, n, total.device, rank1)
        ema_key = f"{side}_ema"
        first = ema_key not in state
        if first:
            state[ema_key] = torch.empty(n, dtype=torch.float32, device=total.device)
            if rank1:
                state["a_mean_ema"] = torch.empty(n, dtype=torch.float32, device=total.device)
        name = self.parameter_names[id(parameter)]
        keys = [f"{side}_sum", ema_key] + (["a_first_sum", "a_mean_ema"] if rank1 else [])
        for key in keys:
            _require_f32(state[key], n, parameter.device, f"{key} of {name}")
        kind = _KIND_B if side == "b" else (_KIND_RANK1_A if rank1 else _KIND_DIAG_A)
        d = _native.FinishDesc(sum_sq=total.data_ptr(), slots_sq=sq.data_ptr(), ema=state[ema_key].data_ptr(),
                               inv=out["inv"].data_ptr(), n=n, count=int(count), n_slots=self._take_slot_rows(sq),
                               kind=kind, first=int(first))
        if rank1:
            d.sum_first, d.slots_first = state["a_first_sum"].data_ptr(), fs.data_ptr()
            d.mean_ema = state["a_mean_ema"].data_ptr()
            d.z, d.kappa = out["z"].data_ptr(), out["kappa"].data_ptr()
        return d

    def _descriptor_stage(self, device) -> "_native.DescriptorStage":
        if self._stage is None or self._stage.device != device:
            self._stage = _native.DescriptorStage(device)
        return self._stage

    def _run_closure(self, closure):
        """sandmuon/optimizer.py:226-230: the closure runs with gradients enabled."""
        if closure is None:
            return None
        with torch.enable_grad():
            return closure()

    def _momentum(self, group) -> float:
        """Matrix momentum of a group (sandmuon/optimizer.py:246-248)."""
        return float(group["momentum"])

    @torch.no_grad()
    def step(self, closure=None):
        loss = self._run_closure(closure)
        self._flush_stats()
        self._queue.restart()
        matrix_items, auxiliary_items = [], []
        a_counts: Dict[int, int] = {}
        device = None
        for group in self.param_groups:
            for parameter in group["params"]:
                if parameter.grad is None:
                    continue
                if parameter.device != device:
                    if device is not None:
                        raise ValueError("sandmuon_amd runs one optimizer per GPU: every parameter must be on one "
                                         f"device (got {device} and {parameter.device})")
                    device = parameter.device
                if group.get("use_muon", True):
                    source = self.a_sources[id(parameter)]
                    if id(source) not in a_counts:
                        a_counts[id(source)] = self._finish_a_check(source)
                    self._finish_b_check(parameter, a_counts[id(source)])
                    matrix_items.append((parameter, source, group))
                else:
                    auxiliary_items.append((parameter, group))
        if matrix_items:
            self._matrix_update(matrix_items, a_counts)
        self._auxiliary_update(auxiliary_items)
        return loss

    def _matrix_update(self, items, a_counts) -> None:
        device = items[0][0].device
        sources = []
        seen = set()
        for parameter, source, _ in items:
            if id(source) not in seen:
                seen.add(id(source))
                sources.append(source)
        # One flat buffer for every factor of this step; each vector starts on
        # a 16-byte boundary (the kernels' vector loads).
        sizes, lengths = [], []
        for s in sources:
            d = self.state[s]["a_sum"].numel()
            lengths += [d, d, 1] if self.rank_one_a else [d]
        for parameter, _, _ in items:
            lengths.append(parameter.shape[0])
        sizes = [-(-n // 4) * 4 for n in lengths]
        flat = torch.empty(sum(sizes), dtype=torch.float32, device=device)
        views = iter(v[:n] for v, n in zip(torch.split(flat, sizes), lengths))
        a_out, b_out, descs = {}, {}, []
        for s in sources:
            out = {"inv": next(views)}
            if self.rank_one_a:
                out["z"], out["kappa"] = next(views), next(views)
            a_out[id(s)] = out
            descs.append(self._finish_desc(s, "a", a_counts[id(s)], out))
        for parameter, source, _ in items:
            out = {"inv": next(views)}
            b_out[id(parameter)] = out
            descs.append(self._finish_desc(parameter, "b", a_counts[id(source)], out))
        _native.stats_finish(descs, self.statistic_beta, device, self._descriptor_stage(device))
        for s in sources:
            self.state[s]["a_count"] = 0
        for parameter, _, _ in items:
            self.state[parameter]["b_count"] = 0

        # Converted or re-laid-out gradients are temporaries: they must stay
        # alive until the launch that reads them is enqueued (the allocator
        # would hand a freed one to the next temporary of this loop).
        mdescs, shapes, keep = [], [], []
        for parameter, source, group in items:
            state = self.state[parameter]
            _check_layout(parameter, self.parameter_names[id(parameter)], True)
            if "momentum_buffer" not in state:
                state["momentum_buffer"] = torch.zeros_like(parameter, dtype=torch.float32)
            elif not state["momentum_buffer"].is_contiguous() or state["momentum_buffer"].dtype != torch.float32:
                state["momentum_buffer"] = state["momentum_buffer"].to(torch.float32).contiguous()
            grad = parameter.grad
            if grad.dtype not in _PARAM_DTYPES:
                grad = grad.float()
            grad = grad.contiguous()
            keep.append(grad)
            a = a_out[id(source)]
            md = _native.MatrixDesc(param=parameter.data_ptr(), grad=grad.data_ptr(),
                                    momentum=state["momentum_buffer"].data_ptr(),
                                    inv_row=b_out[id(parameter)]["inv"].data_ptr(), inv_col=a["inv"].data_ptr(),
                                    rows=parameter.shape[0], cols=parameter.shape[1], lr=float(group["lr"]),
                                    momentum_beta=self._momentum(group),
                                    grad_dtype=_native.dtype_code(grad.dtype),
                                    param_dtype=_native.dtype_code(parameter.dtype))
            if self.rank_one_a:
                md.z, md.kappa = a["z"].data_ptr(), a["kappa"].data_ptr()
            mdescs.append(md)
            shapes.append(tuple(parameter.shape))
        mode = _native.S8_MODES[self.s8_mode]
        need = _native.matrix_step_workspace_bytes(shapes, mode)
        if self._workspace is None or self._workspace.numel() < need or self._workspace.device != device:
            self._workspace = None
            self._workspace = torch.empty(need, dtype=torch.uint8, device=device)
        _native.matrix_step(mdescs, mode, self._workspace)
        del keep

    def _auxiliary_update(self, items) -> None:
        by_group: Dict[int, list] = {}
        for parameter, group in items:
            by_group.setdefault(id(group), []).append((parameter, group))
        for entries in by_group.values():
            group = entries[0][1]
            b1, b2 = group["adamw_betas"]
            descs, offset, keep = [], 0, []
            device = entries[0][0].device
            for parameter, _ in entries:
                state = self.state[parameter]
                # The kernel walks parameter, gradient and state flat, so all
                # of them take the parameter's layout.
                _check_layout(parameter, "an auxiliary parameter", False)
                if "exp_avg" not in state:
                    state["exp_avg"] = torch.zeros_like(parameter, dtype=torch.float32)
                    state["exp_avg_sq"] = torch.zeros_like(parameter, dtype=torch.float32)
                    state["step"] = 0
                for key in ("exp_avg", "exp_avg_sq"):
                    state[key] = _like(state[key], parameter, torch.float32)
                state["step"] = int(state["step"]) + 1
                grad = parameter.grad
                if grad.dtype not in _PARAM_DTYPES:
                    grad = grad.float()
                grad = _like(grad, parameter)
                keep.append(grad)  # alive until the launch below is enqueued
                n = parameter.numel()
                descs.append(_native.AdamwDesc(
                    param=parameter.data_ptr(), grad=grad.data_ptr(), exp_avg=state["exp_avg"].data_ptr(),
                    exp_avg_sq=state["exp_avg_sq"].data_ptr(), n=n, offset=offset,
                    bias1=1 - b1 ** state["step"], bias2=1 - b2 ** state["step"],
                    grad_dtype=_native.dtype_code(grad.dtype), param_dtype=_native.dtype_code(parameter.dtype)))
                offset += n
            lr = group["lr"] * group["adamw_lr_ratio"]
            _native.adamw(descs, offset, lr, b1, b2, group["adamw_eps"], group["weight_decay"], device,
                          self._descriptor_stage(device))
            del keep

    def close(self):
        self._flush_stats()
        if self._fused is not None:
            self._fused.close()
        for handle in self.handles:
            handle.remove()
        self.handles.clear()


class RankOneAWeightedPE(DiagonalWeightedPE):
    """Production SAND variant with exact rank-one activation mean correction
    (sandmuon/optimizer.py:324-328)."""

    def __init__(self, model: nn.Module, lr: float, *,
                 module_filter: Optional[Callable[[str, nn.Module], bool]] = None,
                 s8_mode: str = "comp_bf16", hook_batch_bytes: Optional[int] = None):
        super().__init__(model, lr, rank_one_a=True, module_filter=module_filter, s8_mode=s8_mode,
                         hook_batch_bytes=hook_batch_bytes)
