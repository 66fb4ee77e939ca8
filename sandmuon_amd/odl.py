"""The historical ODL trainer's optimizer plugin boundary, on the same HIP
kernels as the portable classes.

Mirrors reproduction/odl/optim/registry.py:21-75 (the registry and
``create_optimizer``) and the factories and classes of
reproduction/odl/optim/diagonal_weighted_pe.py:165-564:

* ``create_optimizer(model, lr, betas, weight_decay, optimizer_type,
  device_type)`` looks the name up case-insensitively and raises
  ``ValueError`` listing the registered names otherwise (registry.py:57-75);
* ``sand_muon`` and ``muon_raw_diagonal_weighted_pe`` build
  ``DiagonalWeightedPE(model, lr=lr)``; ``sand_muon_rank1`` builds
  ``RankOneAWeightedPE(model, lr=lr, split_sides=False)``
  (diagonal_weighted_pe.py:551-561).  The factories ignore betas,
  weight_decay and device_type, as the historical ones do.

The historical classes differ from the portable ones (sandmuon/optimizer.py)
in these respects, all reproduced here:

* matrices are the ``nn.Linear`` modules whose name matches
  ``^transformer\\.h\\.\\d+\\.`` (diagonal_weighted_pe.py:178-186), with
  ``ValueError("No transformer.h.* linear weights found")`` if none;
* a selected k/v projection whose block has no selected q projection raises
  ``RuntimeError("Split attention projection is missing q_proj")``
  (:212-220) instead of keeping its own statistic;
* matrix momentum is fixed at .8 (:335-338), whatever the group says;
* the closure runs under ``no_grad`` (:292-294);
* the AdamW ``step`` of a checkpoint is a float32 tensor on the parameter's
  device (:316-321); internally the count stays a host integer, so no step
  reads a device value, and ``state_dict()`` emits the tensor form;
* ``RankOneAWeightedPE`` takes ``split_sides`` (:424-427).  It only orders
  the historical batches so that one-sided maps are contiguous
  (:500-543); every matrix here carries its own one-sided rank-one factor
  through the kernels, so the flag is kept as an attribute and does not
  change the arithmetic.

Two historical behaviours are deliberately not reproduced: the S8 products
use this build's compensated BF16 in all five stages (the historical recipe
compensates stage 1 only and runs stages 2-5 in plain BF16, about 100x less
accurate on ill-conditioned inputs), and the diagonal inverse square root
keeps the portable path's final clamp at 1e-6 (the two agree unless a whole
statistic vector is zero, where the historical path returns inf).
"""
from __future__ import annotations

import re
from typing import Any, Callable, Dict

import torch
from torch import nn

from . import optimizer as _portable
from .optimizer import select_matrices

__all__ = ["register_optimizer", "create_optimizer", "available_optimizers", "historical_filter",
           "DiagonalWeightedPE", "RankOneAWeightedPE"]

_REGISTRY: Dict[str, Callable[..., Any]] = {}


def register_optimizer(name: str):
    """Decorator registering a factory ``fn(model, *, lr, betas, weight_decay,
    device_type)`` under ``name`` (registry.py:31-37)."""
    def deco(fn: Callable[..., Any]) -> Callable[..., Any]:
        _REGISTRY[name] = fn
        return fn
    return deco


def available_optimizers():
    return sorted(_REGISTRY)


def create_optimizer(model, lr: float = 3e-4, betas=(0.9, 0.95), weight_decay: float = 0.1,
                     optimizer_type: str = "dense", device_type: str = "cuda"):
    """Build an optimizer by registered name (registry.py:57-75)."""
    fn = _REGISTRY.get(optimizer_type.lower())
    if fn is None:
        available = ", ".join(available_optimizers()) or "(none)"
        raise ValueError(f"Unknown optimizer_type '{optimizer_type}'. Available: {available}")
    return fn(model, lr=lr, betas=betas, weight_decay=weight_decay, device_type=device_type)


_TRANSFORMER_BLOCK = re.compile(r"^transformer\.h\.\d+\.")
_KV_PROJ = re.compile(r"^(transformer\.h\.\d+\.attn\.)[kv]_proj\.weight$")


def historical_filter(name: str, module: nn.Module) -> bool:
    """The historical matrix selection (diagonal_weighted_pe.py:178-186)."""
    return bool(_TRANSFORMER_BLOCK.match(name)) and isinstance(module, nn.Linear)


def _check_selection(model: nn.Module) -> None:
    try:
        matrices, _ = select_matrices(model, historical_filter)
    except ValueError:
        raise ValueError("No transformer.h.* linear weights found") from None
    for name in matrices:
        match = _KV_PROJ.match(name)
        if match and (match.group(1) + "q_proj.weight") not in matrices:
            raise RuntimeError("Split attention projection is missing q_proj")


class _Historical:
    """Behaviour shared by the two historical classes (mixed in first)."""

    HISTORICAL_MOMENTUM = .8

    def _run_closure(self, closure):
        # diagonal_weighted_pe.py:292-294: step() is no_grad throughout.
        return closure() if closure is not None else None

    def _momentum(self, group) -> float:
        return self.HISTORICAL_MOMENTUM

    def _finish_b_check(self, parameter, expected_count: int) -> None:
        # diagonal_weighted_pe.py:279-283 (the message names the matrix only)
        if self.state[parameter].get("b_count", 0) != expected_count:
            raise RuntimeError("Missing or mismatched cotangent statistics: " + self.parameter_names[id(parameter)])

    def state_dict(self):
        sd = super().state_dict()
        flat = [p for group in self.param_groups for p in group["params"]]
        for index, entry in list(sd["state"].items()):
            step = entry.get("step")
            if step is not None and not torch.is_tensor(step):
                # The packed entries are this optimizer's own state dicts:
                # replace, do not mutate.
                sd["state"][index] = dict(entry, step=torch.tensor(float(step), dtype=torch.float32,
                                                                   device=flat[index].device))
        return sd


class DiagonalWeightedPE(_Historical, _portable.DiagonalWeightedPE):
    """Historical diagonal SAND (diagonal_weighted_pe.py:165-419)."""

    def __init__(self, model: nn.Module, lr: float, *, rank_one_a: bool = False, s8_mode: str = "comp_bf16"):
        _check_selection(model)
        super().__init__(model, lr, rank_one_a=rank_one_a, module_filter=historical_filter, s8_mode=s8_mode)


class RankOneAWeightedPE(_Historical, _portable.RankOneAWeightedPE):
    """Historical production SAND with rank-one activation geometry
    (diagonal_weighted_pe.py:422-548)."""

    def __init__(self, model: nn.Module, lr: float, *, split_sides: bool = False, s8_mode: str = "comp_bf16"):
        _check_selection(model)
        super().__init__(model, lr, module_filter=historical_filter, s8_mode=s8_mode)
        self.split_sides = bool(split_sides)


@register_optimizer("sand_muon")
@register_optimizer("muon_raw_diagonal_weighted_pe")
def _create(model, *, lr, betas, weight_decay, device_type):
    del betas, weight_decay, device_type
    return DiagonalWeightedPE(model, lr=lr)


@register_optimizer("sand_muon_rank1")
def _create_rank1(model, *, lr, betas, weight_decay, device_type):
    del betas, weight_decay, device_type
    return RankOneAWeightedPE(model, lr=lr, split_sides=False)
