"""Dense and packed CP adapters with Ruiz equilibration (the NLPOPTNet path).

Mirrors ``src/purin/solvers/chambolle_pock/dense_layer.py:13-134``
(``solve_dense_implicit``), ``dense.py:26-105`` (``solve_dense``),
``sparse_layer.py:44-122`` (a packed ``inequality_support``) and
``src/purin/linalg/equilibration.py:21-57`` (``ruiz_equilibrate``).

The iteration runs in the HIP library (``purin_cp_dense_solve``: factored
prox, no freezing, no stationarity test, power-iteration steps) and the
backward is ``purin_cp_dense_adjoint`` (BiCGSTAB over the batch with the
frozen prox, as ``dense_implicit.py`` + ``autodiff/fixed_point.py``).  The
equilibration is batched elementwise torch work on the GPU around the call;
torch autograd differentiates through it (``amax`` splits ties evenly, as
JAX's max does), as JAX does through the reference's.
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np
import torch

from purin_amd.plan import Plan


def ruiz_equilibrate(q, c, A, b, C, d, lower, upper, *, iterations=4, eps=1e-6):
    """Batched Ruiz scaling of a diagonal QP (equilibration.py:21-57).

    Returns ``(q, c, A, b, C, d, lower, upper, columns, equalities, inequalities)``.
    """
    columns = torch.ones_like(q)
    eqs, iqs = torch.ones_like(b), torch.ones_like(d)
    epsilon = torch.as_tensor(eps, dtype=q.dtype, device=q.device)
    for _ in range(iterations):
        colA = A.abs().amax(dim=1) if A.shape[1] else torch.zeros_like(q)
        colC = C.abs().amax(dim=1) if C.shape[1] else torch.zeros_like(q)
        metric = torch.maximum(torch.maximum(colA, colC), q.abs())
        update = 1.0 / torch.sqrt(torch.maximum(metric, epsilon))
        A, C = A * update[:, None, :], C * update[:, None, :]
        q, c = q * update ** 2, c * update
        lower, upper, columns = lower / update, upper / update, columns * update
        if A.shape[1]:
            update = 1.0 / torch.sqrt(torch.maximum(A.abs().amax(dim=2), epsilon))
            A, b, eqs = A * update[:, :, None], b * update, eqs * update
        if C.shape[1]:
            update = 1.0 / torch.sqrt(torch.maximum(C.abs().amax(dim=2), epsilon))
            C, d, iqs = C * update[:, :, None], d * update, iqs * update
    return q, c, A, b, C, d, lower, upper, columns, eqs, iqs


@lru_cache(maxsize=64)
def _plan(n, me, mi, support, accelerated, safety, norm_iterations, norm_seed, dtype, device):
    """One plan per (shape, support, options): equality rows dense, inequality
    rows dense or on the packed support."""
    rows = [tuple(range(n))] * me + (list(support) if support is not None
                                     else [tuple(range(n))] * mi)
    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([c for r in rows for c in r], np.int32)
    return Plan(n, me, mi, indptr, indices, np.ones(indptr[-1]), dtype=dtype,
                accelerated=accelerated, row_scaling=False, norm_bound=False,
                norm_iterations=norm_iterations, norm_seed=norm_seed, safety=safety,
                device=device, bound_presolve=False)


class _DenseFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, c, values, rhs, lower, upper, plan, y0, dual0, opts):
        y, mult, it, saved = plan.dense_solve(q, c, rhs, lower, upper, values=values, y0=y0,
                                              dual0=dual0, tolerance=opts["tolerance"],
                                              max_iterations=opts["max_iterations"], save=True)
        ctx.plan, ctx.saved_state, ctx.opts = plan, saved, opts
        ctx.save_for_backward(q.detach(), c.detach(), values.detach())
        ctx.mark_non_differentiable(it)
        return y, mult, it

    @staticmethod
    def backward(ctx, cot_y, cot_mult, _):
        q, c, values = ctx.saved_tensors
        if cot_y is None:
            cot_y = torch.zeros_like(q)
        adj = ctx.plan.dense_adjoint(ctx.saved_state, q, c, cot_y.contiguous(), values=values,
                                     cot_dual=None if cot_mult is None else cot_mult.contiguous(),
                                     tolerance=1e-6, max_iterations=ctx.opts["adjoint_iterations"])
        return (adj.g_q, adj.g_c, adj.g_values, adj.g_rhs, adj.g_lower, adj.g_upper, None, None,
                None, None)


def solve_dense_implicit(q, c, a, b, matrix, d, lower, upper, *, accelerated=False,
                         safety=0.95, norm_iterations=20, norm_seed=42, max_iterations=5000,
                         tolerance=1e-9, adjoint_iterations=50, equilibrate=False,
                         equilibration_iterations=10, y0=None, lambda0=None, mu0=None,
                         inequality_support=None, return_iterations=False):
    """Batched diagonal QPs ``min 0.5 sum(q y^2) + sum(c y)`` s.t. ``a y = b``,
    ``matrix y <= d``, ``lower <= y <= upper`` (dense_layer.py:13-134).

    Returns ``(y, equality_multipliers, inequality_multipliers)`` in the
    original coordinates, and the per-sample iteration counts with
    ``return_iterations``.  Differentiable in every input with torch autograd.
    """
    q = torch.as_tensor(q)
    if not torch.is_floating_point(q):
        q = q.to(torch.float64)
    device = q.device if q.is_cuda else torch.device("cuda", torch.cuda.current_device())
    dtype = q.dtype
    as_t = lambda x: torch.as_tensor(x, dtype=dtype, device=device)
    q, c, a, b, matrix, d, lower, upper = (as_t(x) for x in (q, c, a, b, matrix, d, lower, upper))
    batch, n = q.shape
    if a.ndim == 2:
        a = a[None].expand(batch, *a.shape)
    if matrix.ndim == 2:
        matrix = matrix[None].expand(batch, *matrix.shape)
    me, mi = a.shape[1], matrix.shape[1]
    b, d = torch.broadcast_to(b, (batch, me)), torch.broadcast_to(d, (batch, mi))
    lower, upper = torch.broadcast_to(lower, (batch, n)), torch.broadcast_to(upper, (batch, n))
    y0 = torch.zeros((batch, n), dtype=dtype, device=device) if y0 is None else as_t(y0)
    lambda0 = (torch.zeros((batch, me), dtype=dtype, device=device) if lambda0 is None
               else as_t(lambda0))
    mu0 = torch.zeros((batch, mi), dtype=dtype, device=device) if mu0 is None else as_t(mu0)
    if equilibrate:
        q, c, a, b, matrix, d, lower, upper, columns, eq_scale, iq_scale = ruiz_equilibrate(
            q, c, a, b, matrix, d, lower, upper, iterations=equilibration_iterations)
        y0 = y0 / columns
        lambda0 = lambda0 / torch.where(eq_scale == 0.0, torch.ones_like(eq_scale), eq_scale)
        mu0 = mu0 / torch.where(iq_scale == 0.0, torch.ones_like(iq_scale), iq_scale)
    support = None
    if inequality_support is not None:
        support = tuple(tuple(int(i) for i in row) for row in inequality_support)
        if len(support) != mi:
            raise ValueError("inequality_support must have one row per inequality.")
        for row in support:
            if any(i < 0 or i >= n for i in row) or len(set(row)) != len(row):
                raise ValueError("Sparse support indices must be unique integers in [0, n).")
        support = tuple(tuple(sorted(row)) for row in support)
    plan = _plan(n, me, mi, support, bool(accelerated), float(safety), int(norm_iterations),
                 int(norm_seed), dtype, device)
    if support is None:
        ineq_values = matrix.reshape(batch, mi * n)
    else:  # packed: only the listed entries are coefficients (sparse_layer.py:88-90)
        cols = torch.as_tensor([j for row in support for j in row], device=device)
        rows = torch.as_tensor([i for i, row in enumerate(support) for _ in row], device=device)
        ineq_values = matrix[:, rows, cols]
    values = torch.cat((a.reshape(batch, me * n), ineq_values), dim=1)
    rhs = torch.cat((b, d), dim=1)
    opts = dict(tolerance=float(tolerance), max_iterations=int(max_iterations),
                adjoint_iterations=int(adjoint_iterations))
    y, mult, it = _DenseFn.apply(q, c, values, rhs, lower, upper, plan, y0.detach(),
                                 torch.cat((lambda0, mu0), dim=1).detach(), opts)
    equality, inequality = mult[:, :me], mult[:, me:]
    if equilibrate:
        y, equality, inequality = columns * y, eq_scale * equality, iq_scale * inequality
    return (y, equality, inequality, it) if return_iterations else (y, equality, inequality)


def solve_dense(q, c, A, b, C, d, lower, upper, *, accelerated=False, safety=0.95,
                norm_iterations=20, norm_seed=42, max_iterations=5000, tolerance=1e-9, y0=None,
                lambda0=None, mu0=None, equilibrate=None, return_iterations=False):
    """dense.py:26-105: the forward on dense blocks, with an optional
    ``equilibrate`` callable (e.g. ``ruiz_equilibrate``)."""
    q = torch.as_tensor(q)
    dtype, device = q.dtype, (q.device if q.is_cuda else torch.device("cuda"))
    as_t = lambda x: torch.as_tensor(x, dtype=dtype, device=device)
    args = [as_t(x) for x in (q, c, A, b, C, d, lower, upper)]
    if equilibrate is not None:
        q_, c_, A_, b_, C_, d_, lo_, hi_, columns, eqs, iqs = equilibrate(*args)
        y0_ = None if y0 is None else as_t(y0) / columns
        l0 = None if lambda0 is None else as_t(lambda0) / torch.where(eqs == 0, 1.0, eqs)
        m0 = None if mu0 is None else as_t(mu0) / torch.where(iqs == 0, 1.0, iqs)
        y, lam, mu, it = solve_dense_implicit(q_, c_, A_, b_, C_, d_, lo_, hi_,
                                              accelerated=accelerated, safety=safety,
                                              norm_iterations=norm_iterations,
                                              norm_seed=norm_seed, max_iterations=max_iterations,
                                              tolerance=tolerance, y0=y0_, lambda0=l0, mu0=m0,
                                              return_iterations=True)
        out = (columns * y, eqs * lam, iqs * mu)
    else:
        y, lam, mu, it = solve_dense_implicit(*args, accelerated=accelerated, safety=safety,
                                              norm_iterations=norm_iterations,
                                              norm_seed=norm_seed, max_iterations=max_iterations,
                                              tolerance=tolerance, y0=y0, lambda0=lambda0,
                                              mu0=mu0, return_iterations=True)
        out = (y, lam, mu)
    return (*out, it) if return_iterations else out
