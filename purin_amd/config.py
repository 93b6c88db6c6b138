"""Validated, immutable configurations (names and defaults of the reference).

Reference: src/purin/solvers/chambolle_pock/config.py:10-61 and
src/purin/solvers/config.py:9-43.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field


def validate_metric_diagonal(diagonal):
    """Positive finite tuple or None (reference src/purin/_utils/validation.py:56-70)."""
    if diagonal is None:
        return None
    values = tuple(float(v) for v in diagonal)
    if not values or any(not math.isfinite(v) or v <= 0.0 for v in values):
        raise ValueError("metric_diagonal must contain positive finite values")
    return values


@dataclass(frozen=True)
class LinearSolverConfig:
    """Linear-system solver choices and tolerances for the adjoint GMRES."""

    tolerance: float = 1e-9
    atol: float = 0.0
    restart: int = 30
    max_iterations: int = 100
    use_preconditioner: bool = True
    mode: str = "auto"

    def __post_init__(self):
        if self.tolerance <= 0.0 or self.atol < 0.0:
            raise ValueError("linear tolerances are invalid")
        if self.restart < 1 or self.max_iterations < 1:
            raise ValueError("linear iteration limits must be positive")


@dataclass(frozen=True)
class ImplicitGradientConfig:
    """Adjoint solve settings for implicit differentiation through a projection."""

    policy: str = "residual_checked"
    inexact_tolerance: float = 1e-6
    adjoint_tolerance: float = 1e-8
    invalid_batch_policy: str = "skip"
    differentiate_problem_parameters: bool = False

    def __post_init__(self):
        if self.policy not in {"strict", "residual_checked", "always"}:
            raise ValueError("invalid gradient policy")
        if self.invalid_batch_policy not in {"skip", "use_valid"}:
            raise ValueError("invalid batch policy")
        if self.inexact_tolerance < 0.0 or self.adjoint_tolerance < 0.0:
            raise ValueError("gradient tolerances must be nonnegative")


@dataclass(frozen=True)
class ChambollePockConfig:
    """Affine distance projection with Chambolle--Pock iterations.

    ``early_stop`` is this build's addition: ``False`` runs exactly
    ``max_iterations`` iterations for every sample (the reference reaches that
    with a tolerance too small to be met); the final diagnostics still use
    ``tolerance``.
    """

    tolerance: float = 1e-9
    max_iterations: int = 10000
    accelerated: bool = False
    safety: float = 0.95
    norm_iterations: int = 20
    norm_seed: int = 42
    row_scaling: bool = True
    norm_bound: bool = True
    linear_solver: LinearSolverConfig = field(default_factory=LinearSolverConfig)
    implicit_gradient: ImplicitGradientConfig = field(default_factory=ImplicitGradientConfig)
    diagonal_preconditioning: bool = False
    metric_diagonal: tuple | None = None
    early_stop: bool = True

    def __post_init__(self):
        object.__setattr__(self, "metric_diagonal", validate_metric_diagonal(self.metric_diagonal))
        if not math.isfinite(self.tolerance) or self.tolerance <= 0:
            raise ValueError("tolerance must be positive and finite")
        if not isinstance(self.max_iterations, int) or self.max_iterations < 1:
            raise ValueError("max_iterations must be a positive integer")
        if not 0 < self.safety < 1:
            raise ValueError("safety must be between zero and one")
        if not isinstance(self.norm_iterations, int) or self.norm_iterations < 1:
            raise ValueError("norm_iterations must be a positive integer")
