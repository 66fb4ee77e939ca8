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

The statistics are the hooks' bit for bit (the same slot rows, the same
summation order).  Two things differ from an unfused nn.Linear: the bias
gradient is the FP32 column sum (FP32 chunk sums folded in FP64) where torch
sums in the low precision and rounds to it, and the layer does not support
double backward.  What the fused passes do not cover keeps its separate
read: the A statistic of a bf16 input (there is no cast to fuse into) and
the B statistic of a layer without a bias.  Modules other than plain
``nn.Linear`` keep the hooks.
"""
from __future__ import annotations

import types
import weakref
from typing import Dict, Optional

import torch
import torch.nn.functional as F
from torch import nn
from torch.autograd.function import once_differentiable

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

    def __init__(self, optimizer):
        self.optimizer = optimizer
        self.sites: Dict[str, _Site] = {}
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

    def close(self) -> None:
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


def fuse_statistics(optimizer) -> FusedStatistics:
    """Fuse the hook statistics of every selected plain ``nn.Linear`` into
    the layer's own input cast and bias-gradient passes.  Returns the handle
    (the existing one if the optimizer is already fused)."""
    if optimizer._fused is not None:
        return optimizer._fused
    if not optimizer.handles and optimizer._hook_handles == {}:
        raise RuntimeError("fuse_statistics: the optimizer is closed")
    return FusedStatistics(optimizer)
