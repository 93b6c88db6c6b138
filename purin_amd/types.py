"""Statuses and result tuples (reference src/purin/solvers/types.py:36-86)."""

from __future__ import annotations

from enum import Enum, IntEnum
from typing import Any, NamedTuple


class ProjectionMethod(str, Enum):
    """Projection backends; this build implements Chambolle--Pock only."""

    CHAMBOLLE_POCK = "chambolle-pock"

    @classmethod
    def normalize(cls, value):
        if isinstance(value, cls):
            return value
        try:
            return cls(str(value).strip().lower())
        except ValueError as error:
            supported = ", ".join(item.value for item in cls)
            raise ValueError(
                f"Unknown projection method {value!r}. Supported methods: {supported}."
            ) from error


class SolveStatus(IntEnum):
    """Backend-neutral solver termination status."""

    CONVERGED = 0
    MAX_ITERATIONS = 1
    LINEAR_SOLVE_FAILURE = 2
    NONFINITE = 3
    LINE_SEARCH_FAILURE = 4


class ProjectionResult(NamedTuple):
    """Complete fixed-shape projection result."""

    y: Any
    multipliers_eq: Any
    multipliers_ineq: Any
    slacks: Any
    status: Any
    iterations: Any
    residual_inf_norm: Any
    finite: Any
    gradient_eligible: Any


class ProjectionInfo(NamedTuple):
    """Lightweight diagnostics returned by ``with_info``."""

    forward_status_codes: Any
    forward_iterations: Any
    forward_residual_inf_norm: Any
    forward_state_finite: Any
    gradient_eligible: Any

    @property
    def forward_converged(self):
        return self.forward_status_codes == int(SolveStatus.CONVERGED)


class ProjectionTrainingOutput(NamedTuple):
    """Projected primal/latent-dual state used by the training frontend."""

    y_tilde: Any
    multipliers_eq: Any
    multipliers_ineq: Any
    slacks: Any
    forward_status_codes: Any
    forward_iterations: Any
    forward_residual_inf_norm: Any
    forward_state_finite: Any
    forward_gradient_eligible: Any
