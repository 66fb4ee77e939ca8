"""SandMuon optimizer step for AMD Instinct MI355X (gfx950 HIP kernels).

Same public names as the reference package (sandmuon/__init__.py:3-6).
"""

from .optimizer import DiagonalWeightedPE, RankOneAWeightedPE
from .coefficients import S8_COEFFICIENTS, S8_MARGIN, S8_MULTIPLIER

__all__ = ["DiagonalWeightedPE", "RankOneAWeightedPE", "S8_COEFFICIENTS", "S8_MARGIN", "S8_MULTIPLIER"]
