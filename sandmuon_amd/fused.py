"""Hook statistics fused into the passes a mixed-precision nn.Linear makes
over its input and its output cotangent anyway.

The reference takes the A statistic (sum of x^2, and sum of x for the
rank-one variant) in a forward hook and the B statistic (sum of delta^2) in
a tensor hook on the Linear's output (sandmuon/optimizer.py:151-180).  Each
is one more HBM read of a tensor the layer reads anyway.  Under bf16/f16
autocast the forward first casts an fp32 input to the low precision, and the
backward reduces the output cotangent over its rows for the bias gradient.
``fuse_statistics(optimizer)`` moves the statistics into those two passes:

* forward, fp32 input under autocast: one kernel (``smx_stats_cast``) reads
  x, writes the copy autocast would make and adds the A statistic.  The GEMM
  is torch's ``F.linear`` on the operands autocast would give it, so the
  output is unchanged bit for bit;
  Layers that share the A statistic of another (k and v of a q projection)
  reuse its cast when they are handed the same, unmodified input, where
  autocast would cast it once per layer;
* backward, with a bias: one kernel (``smx_stats_colsum``) reads delta, adds
  the B statistic and writes the bias gradient.  dX = delta W and
  dW = delta^T x are the matrix products torch's own backward of the layer
  runs (``mm_mat1_backward`` / ``mm_mat2_backward``).

* activation, with the model passed to ``fuse_statistics``: an exact
  ``F.gelu`` of a bf16/f16 tensor in the model's forward runs as one kernel
  (``smx_stats_gelu``) that writes the GELU and takes the A statistic of its
  output into per-chunk partials; the Linear that then receives that very
  output adds the partials into its slot rows (``smx_stats_add_partials``)
  instead of reading its input again.  The GELU is torch's formula in FP32
  rounded to the input dtype, so its output equals ``F.gelu``'s bit for bit
  (checked over every bf16 and f16 value); its backward is torch's
  ``gelu_backward``;
* relayout, with the model passed: the copy that hands an attention output
  from [batch, heads, seq, head_dim] back to the projection Linear
  (``y.transpose(1, 2).reshape(b, t, c)``, or ``.contiguous()``, of a
  bf16/f16 view) runs as one kernel (``smx_stats_relayout``) that writes the
  row-major copy and takes the A statistic of it into per-chunk partials,
  which the Linear receiving the copy adds into its slot rows.  The copy is
  torch's bit for bit; its backward reshapes the gradient back.  It applies
  when the sequence length is a multiple of the statistic's row chunk
  (512 rows for up to 64K rows), so that no chunk crosses a sequence.  The
  output of ``F.scaled_dot_product_attention`` on ROCm is seq-major already:
  reshaping it is a view, with no copy to fuse into.

The statistics are the hooks' bit for bit (the same slot rows, the same
summation order).  Two things differ from an unfused nn.Linear: the bias
gradient is the FP32 column sum (FP32 chunk sums folded in FP64) where torch
sums in the low precision and rounds to it, and the layer does not support
double backward.  What the fused passes do not cover keeps its separate
read: the A statistic of a bf16 input that no fused GELU or relayout
produced, and the B statistic of a layer without a bias (its backward has
no elementwise pass over the cotangent, only the two GEMMs).  Modules other
than plain ``nn.Linear`` keep the hooks.
"""
from __future__ import annotations

import math
import types
import weakref
from typing import Dict, Optional

import torch
import torch.nn.functional as F
from torch import nn
from torch.autograd.function import once_differentiable
from torch.overrides import TorchFunctionMode

from . import _native
from .optimizer import _rows2d

__all__ = ["fuse_statistics", "FusedStatistics"]


def _autocast_dtype(device_type: str) -> Optional[torch.dtype]:
    if torch.is_autocast_enabled(device_type):
        return torch.get_autocast_dtype(device_type)
    return None


class _Site:
    """One fused layer: the optimizer, its matrix, whether this layer takes
    the A statistic (the q projection does for k/v), and the layer's
    bias-gradient workspace."""

    def __init__(self, optimizer, name: str, module: nn.Linear):
        self.optimizer = optimizer
        self.name = name
        self.module = module
        self.parameter = optimizer.named_matrices[name]
        self.capture_a = optimizer.a_sources[id(self.parameter)] is self.parameter
        self.workspace: Optional[torch.Tensor] = None
        # The A-source layer's cast of its fp32 input, kept for the layers
        # sharing its statistic (k/v of a q projection), which are handed the
        # same tensor: (weak reference to x, x's version, the cast, uses left).
        self.source: Optional["_Site"] = None
        self.n_sharers = 0
        self.cast_cache = None

    def shared_cast(self, x: torch.Tensor, lp: torch.dtype) -> Optional[torch.Tensor]:
        """The A-source layer's cast of this very input, if it made one."""
        src = self.source
        cache = None if src is None else src.cast_cache
        if cache is None or cache[0]() is not x or cache[1] != x._version or cache[2].dtype != lp:
            return None
        if cache[3] <= 1:
            src.cast_cache = None
        else:
            src.cast_cache = (cache[0], cache[1], cache[2], cache[3] - 1)
        return cache[2]

    def colsum_workspace(self, cols: int, device) -> torch.Tensor:
        need = _native.stats_colsum_workspace_bytes(cols, self.optimizer.STAT_SLOTS)
        ws = self.workspace
        if ws is None or ws.numel() < need or ws.device != device:
            ws = self.workspace = torch.empty(need, dtype=torch.uint8, device=device)
        return ws


class _FusedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, site: _Site):
        opt, p = site.optimizer, site.parameter
        state = opt.state[p]
        lp = _autocast_dtype(x.device.type)
        if lp is not None and x.dtype == torch.float32 and lp in (torch.bfloat16, torch.float16):
            x_lp = None if site.capture_a else site.shared_cast(x, lp)
            if x_lp is None:
                rows = _rows2d(x)
                x_lp = torch.empty(rows.shape, dtype=lp, device=x.device)
                if site.capture_a:
                    sq, fs = opt._a_slots(p, rows.shape[1], rows.device, state)
                    opt._stats_barrier(sq)
                    _native.stats_cast(rows, sq, fs, x_lp)
                    opt._note_slots(sq, rows.shape[0])
                    state["a_count"] += rows.shape[0]
                else:
                    x_lp.copy_(rows)
                x_lp = x_lp.view(x.shape)
                if site.capture_a and site.n_sharers:
                    site.cast_cache = (weakref.ref(x), x._version, x_lp, site.n_sharers)
        else:
            if site.capture_a:
                fused = opt._fused
                entry = fused.take_output(x) if fused is not None else None
                if entry is not None:
                    part_sq, part_first, rows = entry
                    sq, fs = opt._a_slots(p, part_sq.shape[1], x.device, state)
                    opt._stats_barrier(sq)
                    _native.stats_add_partials(sq, part_sq, fs, part_first)
                    opt._note_slots(sq, rows)
                    state["a_count"] += rows
                else:
                    opt._accumulate_a(p, x, state)
            x_lp = x if lp is None or x.dtype == lp else x.to(lp)
        w = weight if lp is None else weight.to(lp)
        b = None if bias is None else (bias if lp is None else bias.to(lp))
        with torch.autocast(device_type=x.device.type, enabled=False):
            y = F.linear(x_lp, w, b)
        ctx.save_for_backward(x_lp, w)
        ctx.site = site
        ctx.x_dtype, ctx.w_dtype = x.dtype, weight.dtype
        ctx.b_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_y):
        x_lp, w = ctx.saved_tensors
        site = ctx.site
        opt, p = site.optimizer, site.parameter
        state = opt.state[p]
        g = _rows2d(grad_y)
        sq = opt._b_slots(p, g.shape[1], g.device, state)
        grad_b = None
        if ctx.b_dtype is not None and ctx.needs_input_grad[2]:
            colsum = torch.empty(g.shape[1], dtype=torch.float32, device=g.device)
            opt._stats_barrier(sq)
            _native.stats_colsum(g, sq, colsum, site.colsum_workspace(g.shape[1], g.device))
            opt._note_slots(sq, g.shape[0])
            grad_b = colsum if ctx.b_dtype == torch.float32 else colsum.to(ctx.b_dtype)
        else:
            opt._enqueue_stats(g, sq, None)
        state["b_count"] += g.shape[0]
        g2 = grad_y.reshape(-1, grad_y.shape[-1])
        grad_x = grad_w = None
        if ctx.needs_input_grad[0]:
            grad_x = g2.mm(w).view(*grad_y.shape[:-1], w.shape[1])
            if grad_x.dtype != ctx.x_dtype:
                grad_x = grad_x.to(ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            grad_w = g2.t().mm(x_lp.reshape(-1, x_lp.shape[-1]))
            if grad_w.dtype != ctx.w_dtype:
                grad_w = grad_w.to(ctx.w_dtype)
        return grad_x, grad_w, grad_b, None


class _FusedGelu(torch.autograd.Function):
    """F.gelu (exact) of a bf16/f16 tensor with the A statistic of its output
    taken in the same pass, into per-chunk partials kept in `holder`."""

    @staticmethod
    def forward(ctx, h, optimizer, holder: list):
        rows = _rows2d(h)
        out = torch.empty(h.shape, dtype=h.dtype, device=h.device)
        n_slots = optimizer.STAT_SLOTS
        chunks = _native.stats_slot_rows(rows.shape[0], n_slots)
        part_sq = torch.empty(chunks, rows.shape[1], dtype=torch.float32, device=h.device)
        part_first = torch.empty_like(part_sq) if optimizer.rank_one_a else None
        _native.stats_gelu(rows, out.view(rows.shape), part_sq, part_first, n_slots)
        holder.extend([part_sq, part_first, rows.shape[0]])
        ctx.save_for_backward(h)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_y):
        (h,) = ctx.saved_tensors
        return torch.ops.aten.gelu_backward(grad_y, h, approximate="none"), None, None


class _FusedRelayout(torch.autograd.Function):
    """The row-major copy of a [batch, seq, heads, head_dim] bf16/f16 view
    (unit last stride) into `shape`, with the A statistic of the copy taken
    in the same pass, into per-chunk partials kept in `holder`."""

    @staticmethod
    def forward(ctx, x, shape, optimizer, holder: list):
        b, t, h, d = x.shape
        out = torch.empty(shape, dtype=x.dtype, device=x.device)
        n_slots = optimizer.STAT_SLOTS
        chunks = _native.stats_slot_rows(b * t, n_slots)
        part_sq = torch.empty(chunks, h * d, dtype=torch.float32, device=x.device)
        part_first = torch.empty_like(part_sq) if optimizer.rank_one_a else None
        _native.stats_relayout(x, out, part_sq, part_first, n_slots)
        holder.extend([part_sq, part_first, b * t])
        ctx.in_shape = x.shape
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_y):
        return grad_y.reshape(ctx.in_shape), None, None, None


_RESHAPES = (torch.Tensor.reshape, torch.reshape)
# The producers whose output statistic a fused forward takes (the model
# given to fuse_statistics): the GELU and the attention output's relayout.
ACTIVATIONS = ("gelu", "relayout")


class _ActivationStatistics(TorchFunctionMode):
    """Active during the forward of the model given to ``fuse_statistics``:
    runs each eligible ``F.gelu`` as ``_FusedGelu`` and each eligible
    relayout copy of an attention output as ``_FusedRelayout`` (other calls,
    and every other function, pass through)."""

    def __init__(self, fused: "FusedStatistics"):
        super().__init__()
        self.fused = fused

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        y = None
        fused = self.fused
        if func is F.gelu and "gelu" in fused.activations:
            y = fused._gelu(args, kwargs)
        elif (func in _RESHAPES or func is torch.Tensor.contiguous) and "relayout" in fused.activations:
            y = fused._relayout(func, args, kwargs)
        if y is not None:
            return y
        return func(*args, **kwargs)


def _fused_forward(site: _Site):
    def forward(module: nn.Linear, x: torch.Tensor) -> torch.Tensor:
        # The reference hook's gate (sandmuon/optimizer.py:153-155): training
        # mode, grad enabled, an output that requires grad.
        if (module.training and torch.is_grad_enabled() and
                (module.weight.requires_grad or x.requires_grad or
                 (module.bias is not None and module.bias.requires_grad))):
            return _FusedLinear.apply(x, module.weight, module.bias, site)
        return F.linear(x, module.weight, module.bias)
    return forward


class FusedStatistics:
    """Handle returned by ``fuse_statistics``; ``close()`` restores the hooks."""

    def __init__(self, optimizer, model: Optional[nn.Module] = None, activations=ACTIVATIONS):
        unknown = set(activations) - set(ACTIVATIONS)
        if unknown:
            raise ValueError(f"fuse_statistics: unknown activations {sorted(unknown)}; expected a subset of "
                             f"{ACTIVATIONS}")
        self.optimizer = optimizer
        self.activations = frozenset(activations)
        self.sites: Dict[str, _Site] = {}
        # Outputs of the running forward's fused GELUs and relayouts, by
        # data pointer: (weak reference, version, kind, partials of sq, of
        # first, rows); taken by the Linear that receives one (or a
        # contiguous view of it), dropped when the forward ends.
        self._outputs: Dict[int, tuple] = {}
        self.gelu_calls = 0       # GELUs run fused
        self.gelu_taken = 0       # of those, outputs whose statistic a Linear took
        self.relayout_calls = 0   # relayout copies run fused
        self.relayout_taken = 0   # of those, copies whose statistic a Linear took
        self._mode: Optional[_ActivationStatistics] = None
        self._depth = 0
        self._model_handles = []
        if model is not None:
            self._model_handles = [model.register_forward_pre_hook(self._enter),
                                   model.register_forward_hook(self._leave, always_call=True)]
        for name, module in optimizer._matrix_modules.items():
            if type(module) is not nn.Linear or "forward" in module.__dict__:
                continue  # keeps its hooks
            site = _Site(optimizer, name, module)
            handle = optimizer._hook_handles.pop(name)
            handle.remove()
            optimizer.handles.remove(handle)
            module.forward = types.MethodType(_fused_forward(site), module)
            self.sites[name] = site
        by_param = {id(site.parameter): site for site in self.sites.values()}
        for site in self.sites.values():
            if not site.capture_a:
                site.source = by_param.get(id(optimizer.a_sources[id(site.parameter)]))
                if site.source is not None:
                    site.source.n_sharers += 1
        optimizer._fused = self

    @property
    def fused_names(self):
        return list(self.sites)

    # ------------------------------------------------------ activations ---
    def _enter(self, module, inputs):
        if self._depth == 0:
            self._mode = _ActivationStatistics(self)
            self._mode.__enter__()
        self._depth += 1

    def _leave(self, module, inputs, output):
        self._depth -= 1
        if self._depth == 0:
            mode, self._mode = self._mode, None
            mode.__exit__(None, None, None)
            self._outputs.clear()

    def _gelu(self, args, kwargs):
        """The fused GELU of an eligible call, else None."""
        h = args[0] if args else kwargs.get("input")
        approximate = args[1] if len(args) > 1 else kwargs.get("approximate", "none")
        if (approximate != "none" or not isinstance(h, torch.Tensor) or h.device.type != "cuda" or
                h.dtype not in (torch.bfloat16, torch.float16) or h.dim() < 2 or h.numel() == 0 or
                h.shape[-1] % 8 != 0 or not torch.is_grad_enabled() or not self.sites):
            return None
        holder: list = []
        y = _FusedGelu.apply(h, self.optimizer, holder)
        self._register(y, "gelu", holder)
        self.gelu_calls += 1
        return y

    def _relayout(self, func, args, kwargs):
        """The fused relayout of an eligible reshape / contiguous call, else None."""
        x = args[0] if args else kwargs.get("input")
        if (not isinstance(x, torch.Tensor) or x.dim() != 4 or x.device.type != "cuda" or
                x.dtype not in (torch.bfloat16, torch.float16) or x.is_contiguous() or x.stride(-1) != 1 or
                not torch.is_grad_enabled() or not self.sites):
            return None
        b, t, h, d = x.shape
        if func is torch.Tensor.contiguous:
            fmt = args[1] if len(args) > 1 else kwargs.get("memory_format", torch.contiguous_format)
            if fmt is not torch.contiguous_format:
                return None
            shape = (b, t, h, d)
        else:
            dims = args[1:] if func is torch.Tensor.reshape else args[1:2]
            if not dims:
                dims = (kwargs.get("shape"),)
            if len(dims) == 1 and isinstance(dims[0], (tuple, list, torch.Size)):
                dims = tuple(dims[0])
            if not dims or not all(isinstance(n, int) for n in dims):
                return None
            shape = tuple(dims)
            if shape.count(-1) == 1:
                known = math.prod(n for n in shape if n != -1)
                if known <= 0 or x.numel() % known:
                    return None
                shape = tuple(x.numel() // known if n == -1 else n for n in shape)
            if shape not in ((b, t, h * d), (b * t, h * d)):
                return None
            # Only where torch's reshape copies: where it returns a view, the
            # result must stay an alias of x (in-place writes reach x).
            merges_hd = x.stride(2) == d
            merges_bt = x.stride(0) == t * x.stride(1)
            if merges_hd and (len(shape) == 3 or merges_bt):
                return None
        rows = b * t
        chunk = max(-(-rows // self.optimizer.STAT_SLOTS), 512)
        if (d % 8 or t % chunk or any(st % 8 for st in x.stride()[:3]) or x.data_ptr() % 16 or
                x.numel() == 0):
            return None
        holder: list = []
        y = _FusedRelayout.apply(x, shape, self.optimizer, holder)
        self._register(y, "relayout", holder)
        self.relayout_calls += 1
        return y

    def _register(self, y: torch.Tensor, kind: str, holder: list) -> None:
        self._outputs[y.data_ptr()] = (weakref.ref(y), y._version, kind, *holder)

    def take_output(self, x: torch.Tensor):
        """(partials of sq, of first, rows) if x is an unmodified fused GELU or
        relayout output of the running forward, or a contiguous view of all
        of one (removed from the registry), else None."""
        entry = self._outputs.get(x.data_ptr())
        if entry is None:
            return None
        y = entry[0]()
        if (y is None or entry[1] != x._version or x.dtype != y.dtype or x.numel() != y.numel() or
                not x.is_contiguous() or x.shape[-1] != entry[3].shape[1]):
            return None
        del self._outputs[x.data_ptr()]
        if entry[2] == "gelu":
            self.gelu_taken += 1
        else:
            self.relayout_taken += 1
        return entry[3], entry[4], entry[5]

    def close(self) -> None:
        for h in self._model_handles:
            h.remove()
        self._model_handles = []
        if self._mode is not None:
            self._mode.__exit__(None, None, None)
            self._mode, self._depth = None, 0
        self._outputs.clear()
        opt = self.optimizer
        for name, site in self.sites.items():
            site.cast_cache = None
            site.module.__dict__.pop("forward", None)
            handle = opt._install_hook(name)
            opt._hook_handles[name] = handle
            opt.handles.append(handle)
        self.sites.clear()
        if opt._fused is self:
            opt._fused = None


def fuse_statistics(optimizer, model: Optional[nn.Module] = None, activations=ACTIVATIONS) -> FusedStatistics:
    """Fuse the hook statistics of every selected plain ``nn.Linear`` into
    the layer's own input cast and bias-gradient passes, and, when the model
    is given, the A statistic of a GELU's output into the GELU and that of
    an attention output into its relayout copy (during ``model``'s forward;
    ``activations`` names which of the two).  Returns the handle (the
    existing one if the optimizer is already fused)."""
    if optimizer._fused is not None:
        return optimizer._fused
    if not optimizer.handles and optimizer._hook_handles == {}:
        raise RuntimeError("fuse_statistics: the optimizer is closed")
    return FusedStatistics(optimizer, model, activations)
