"""Statuses and result tuples (reference src/purin/solvers/types.py:36-86)."""

from __future__ import annotations

from enum import Enum, IntEnum
from typing import Any, NamedTuple


class ProjectionMethod(str, Enum):
    """Which projection solver to run; only Chambolle--Pock exists in this build."""

    CHAMBOLLE_POCK = "chambolle-pock"

    @classmethod
    def normalize(cls, value):
        """Accept a member or its name in any case/padding; raise ValueError otherwise
        (the reference raises for unknown names too, types.py:22-33)."""
        if isinstance(value, cls):
            return value
        key = str(value).strip().lower()
        for member in cls:
            if member.value == key:
                return member
        names = ", ".join(m.value for m in cls)
        raise ValueError(f"Unknown projection method {value!r}; this build supports: {names}.")


class SolveStatus(IntEnum):
    """Why a solve stopped; the integer codes are part of the result interface."""

    CONVERGED = 0
    MAX_ITERATIONS = 1
    LINEAR_SOLVE_FAILURE = 2
    NONFINITE = 3
    LINE_SEARCH_FAILURE = 4


class ProjectionResult(NamedTuple):
    """Every output of one batched projection, each with a fixed shape."""

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
    """Per-sample forward diagnostics that ``with_info`` returns beside y."""

    forward_status_codes: Any
    forward_iterations: Any
    forward_residual_inf_norm: Any
    forward_state_finite: Any
    gradient_eligible: Any

    @property
    def forward_converged(self):
        return self.forward_status_codes == int(SolveStatus.CONVERGED)


class ProjectionTrainingOutput(NamedTuple):
    """The training front end's output: the projected point, its multipliers and forward diagnostics."""

    y_tilde: Any
    multipliers_eq: Any
    multipliers_ineq: Any
    slacks: Any
    forward_status_codes: Any
    forward_iterations: Any
    forward_residual_inf_norm: Any
    forward_state_finite: Any
    forward_gradient_eligible: Any
