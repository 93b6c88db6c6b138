"""General positive diagonal QP layer on the HIP CP kernels.

Mirrors ``src/purin/solvers/diagonal_qp.py``: ``QPData`` (26-34),
``QPStructure`` (37-67), ``PreparedDiagonalQP`` (70-319) and ``dense_qp_data``
(322-349).  Every input (q, c, the constraint coefficients, rhs, bounds) is
differentiable with torch autograd; the backward is ``purin_cp_qp_adjoint``
(the reference's custom_vjp ``bwd``, 131-219), including the multipliers'
cotangent.  Values use the reference's ELL layout ``(B, m, width)`` on the
structure's row supports; the plan takes their stored slots in row order.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import numpy as np
import torch

from purin_amd.config import ChambollePockConfig
from purin_amd.plan import Plan
from purin_amd.projection import resolve_device, resolve_dtype
from purin_amd.types import ProjectionResult


class QPData(NamedTuple):
    """Batched diagonal objective, constraint coefficients and variable bounds."""

    q: object
    c: object
    values: object
    rhs: object
    lower: object
    upper: object


def layout(rows, n):
    """ELL support and mask of row supports (reference kernels.py:26-40)."""
    width = max((len(r) for r in rows), default=0)
    width = max(width, 1)
    support = np.zeros((len(rows), width), np.int32)
    mask = np.zeros((len(rows), width), bool)
    for i, r in enumerate(rows):
        support[i, : len(r)] = r
        mask[i, : len(r)] = True
    return support, mask


@dataclass(frozen=True)
class QPStructure:
    """Variable dimension and fixed row supports for a family of diagonal QPs."""

    variable_size: int
    equality_rows: tuple = ()
    inequality_rows: tuple = ()

    def __post_init__(self):
        if self.variable_size < 1:
            raise ValueError("variable_size must be positive")
        for key in ("equality_rows", "inequality_rows"):
            rows = tuple(tuple(int(i) for i in row) for row in getattr(self, key))
            if any(len(set(row)) != len(row) or any(i < 0 or i >= self.variable_size for i in row)
                   for row in rows):
                raise ValueError("constraint supports must contain unique valid indices")
            object.__setattr__(self, key, rows)

    @property
    def rows(self):
        """Equality rows followed by inequality rows in solver order."""
        return self.equality_rows + self.inequality_rows

    def prepare(self, *, batch_size, config=None, dtype=torch.float64, backend="gpu"):
        """Prepare a solver for this fixed sparse structure and batch shape."""
        return PreparedDiagonalQP(self, int(batch_size), config or ChambollePockConfig(), dtype,
                                  backend)


class _QPFn(torch.autograd.Function):
    """(y, multipliers) = QP(q, c, values, rhs, lower, upper) with the implicit VJP."""

    @staticmethod
    def forward(ctx, q, c, values, rhs, lower, upper, layer, y0, dual0):
        cfg = layer.config
        out = layer.plan.qp_solve(q, c, rhs, lower, upper, values=values, y0=y0, dual0=dual0,
                                  tolerance=cfg.tolerance, max_iterations=cfg.max_iterations,
                                  early_stop=cfg.early_stop, save=True)
        ctx.layer = layer
        ctx.saved_state = out.saved
        ctx.save_for_backward(q.detach(), c.detach(), values.detach())
        ctx.mark_non_differentiable(out.slacks, out.status, out.iterations, out.residual,
                                    out.finite, out.converged)
        return (out.y, out.multipliers, out.slacks, out.status, out.iterations, out.residual,
                out.finite, out.converged)

    @staticmethod
    def backward(ctx, cot_y, cot_mult, *unused):
        layer = ctx.layer
        q, c, values = ctx.saved_tensors
        if cot_y is None:
            cot_y = torch.zeros_like(q)
        if not layer.differentiate_duals:
            cot_mult = None
        lin = layer.config.linear_solver
        adj = layer.plan.qp_adjoint(
            ctx.saved_state, q, c, cot_y.contiguous(), values=values,
            cot_dual=None if cot_mult is None else cot_mult.contiguous(),
            tolerance=lin.tolerance, atol=lin.atol, restart=lin.restart,
            max_iterations=lin.max_iterations,
            adjoint_tolerance=layer.config.implicit_gradient.adjoint_tolerance)
        return (adj.g_q, adj.g_c, adj.g_values, adj.g_rhs, adj.g_lower, adj.g_upper, None, None,
                None)


@dataclass(eq=False)
class PreparedDiagonalQP:
    """Prepared diagonal-QP solve on the shared sparse CP kernels."""

    structure: QPStructure
    batch_size: int
    config: ChambollePockConfig
    dtype: object = torch.float64
    backend: str = "gpu"
    differentiate_duals: bool = True

    def __post_init__(self):
        if self.batch_size < 1:
            raise ValueError("batch_size must be positive")
        if self.config.metric_diagonal is not None:
            raise ValueError("QPData.q already defines the quadratic metric")
        n = self.structure.variable_size
        rows = self.structure.rows
        self.support, self.mask = layout(rows, n)
        self.device = resolve_device(self.backend)
        self.torch_dtype = resolve_dtype(self.dtype)
        cfg = self.config
        indptr = np.zeros(len(rows) + 1, np.int64)
        indptr[1:] = np.cumsum([len(r) for r in rows])
        indices = np.asarray([i for r in rows for i in r], np.int32)
        # coefficients arrive per call; the plan keeps the sparsity and options
        self.plan = Plan(n, len(self.structure.equality_rows), len(self.structure.inequality_rows),
                         indptr, indices, np.ones(indptr[-1]), dtype=self.torch_dtype,
                         accelerated=cfg.accelerated, row_scaling=cfg.row_scaling,
                         norm_bound=cfg.norm_bound, norm_iterations=cfg.norm_iterations,
                         norm_seed=cfg.norm_seed, safety=cfg.safety,
                         diagonal_preconditioning=cfg.diagonal_preconditioning,
                         device=self.device, bound_presolve=False)
        self._mask_t = torch.as_tensor(self.mask, device=self.device)

    def _as(self, x):
        return torch.as_tensor(x).to(device=self.device, dtype=self.torch_dtype)

    def solve(self, data, *, initial_y=None, initial_dual=None):
        """Solve the batched diagonal QP (diagonal_qp.py:222-319)."""
        data = QPData(*(self._as(x) for x in data))
        b, n = self.batch_size, self.structure.variable_size
        m, width = self.mask.shape
        expected = ((b, n), (b, n), (b, m, width), (b, m), (b, n), (b, n))
        for key, value, shape in zip(QPData._fields, data, expected):
            if tuple(value.shape) != shape:
                raise ValueError(f"{key} must have shape {shape}; got {tuple(value.shape)}")
        y0 = None if initial_y is None else self._as(initial_y)
        dual0 = None if initial_dual is None else self._as(initial_dual)
        if (y0 is not None and tuple(y0.shape) != (b, n)) or (
                dual0 is not None and tuple(dual0.shape) != (b, m)):
            raise ValueError("initial primal/dual shapes do not match the prepared QP")
        y0 = None if y0 is None else y0.detach()
        dual0 = None if dual0 is None else dual0.detach()
        # stored slots of the ELL values, in row order (the plan's CSR entry order)
        values = data.values[:, self._mask_t]
        y, mult, slacks, status, iters, res, fin, conv = _QPFn.apply(
            data.q, data.c, values, data.rhs, data.lower, data.upper, self, y0, dual0)
        me = len(self.structure.equality_rows)
        return ProjectionResult(y, mult[:, :me], mult[:, me:], slacks, status, iters, res, fin,
                                conv)


def dense_qp_data(q, c, A, b, C, d, lower, upper):
    """Dense rows over all n variables, broadcast to the batch (diagonal_qp.py:322-349)."""
    q, c = torch.as_tensor(q), torch.as_tensor(c)
    if q.ndim != 2 or q.shape != c.shape:
        raise ValueError("q and c must be matching batched matrices")
    batch, n = q.shape
    A = torch.broadcast_to(torch.as_tensor(A, dtype=q.dtype), (batch,) + tuple(np.shape(A)[-2:]))
    C = torch.broadcast_to(torch.as_tensor(C, dtype=q.dtype), (batch,) + tuple(np.shape(C)[-2:]))
    rows = tuple(tuple(range(n)) for _ in range(A.shape[1]))
    iq = tuple(tuple(range(n)) for _ in range(C.shape[1]))
    structure = QPStructure(n, rows, iq)
    values = torch.cat((A, C), dim=1)  # every row has the full support: ELL == dense
    rhs = torch.cat((torch.broadcast_to(torch.as_tensor(b, dtype=q.dtype), (batch, A.shape[1])),
                     torch.broadcast_to(torch.as_tensor(d, dtype=q.dtype), (batch, C.shape[1]))),
                    dim=1)
    return structure, QPData(q, c, values, rhs,
                             torch.broadcast_to(torch.as_tensor(lower, dtype=q.dtype), q.shape),
                             torch.broadcast_to(torch.as_tensor(upper, dtype=q.dtype), q.shape))
