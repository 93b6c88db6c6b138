"""Prepared Chambolle--Pock projections (the reference's public entry points).

``Distance(problem, "chambolle-pock", config).prepare(batch_size=, dtype=, backend=)``,
``WeightedDistance(problem, diagonal, ...).prepare(...)`` and
``prepare_projection(problem, method=, config=, batch_size=, dtype=, backend=)``
return a ``PreparedChambollePockProjection`` with the reference's methods
``__call__``, ``solve``, ``with_info`` and ``project_training``
(src/purin/solvers/chambolle_pock/solver.py:368-402, bounds.py:170-317,
src/purin/projections/distance.py:8-61, src/purin/solvers/metric.py:87-182).

Arrays are torch tensors on the GPU (inputs may be numpy or CPU tensors; they
are moved to the device like ``jax.device_put``).  ``__call__`` and
``project_training(...).y_tilde`` are differentiable with torch autograd: the
backward is the implicit VJP of ``purin_cp_adjoint`` w.r.t. ``y_hat`` and, when
``ImplicitGradientConfig.differentiate_problem_parameters`` is set, w.r.t. the
parameters through ``rhs(theta)`` and, for parameter-dependent coefficients,
through the per-sample values ``values(theta)`` (``purin_cp_project_values`` /
``purin_cp_adjoint_values``).  Every computation runs in the HIP library;
``backend="cpu"`` is rejected because this build has no CPU execution path.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

from purin_amd.config import ChambollePockConfig
from purin_amd.plan import Plan
from purin_amd.problems import CanonicalRows
from purin_amd.types import (ProjectionInfo, ProjectionMethod, ProjectionResult,
                             ProjectionTrainingOutput)

_GPU_BACKENDS = {"gpu", "cuda", "rocm", "hip", "amd", "mi355x"}


def resolve_device(backend):
    """Map a backend string to a torch device (reference execution/runtime.py:33-78)."""
    if isinstance(backend, torch.device):
        if backend.type != "cuda":
            raise ValueError("this build executes on the GPU; use backend='gpu'")
        return backend
    text = str(backend).strip().lower()
    head, _, index = text.partition(":")
    if head == "cpu":
        raise ValueError("backend='cpu' is not provided: the projection runs in HIP kernels on "
                         "the GPU; use backend='gpu' (or 'rocm')")
    if head not in _GPU_BACKENDS:
        raise ValueError(f"unknown backend {backend!r}; use 'gpu', 'rocm' or 'cuda:N'")
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU is visible to torch; the HIP projection needs one")
    return torch.device("cuda", int(index) if index else torch.cuda.current_device())


def resolve_dtype(dtype):
    if dtype in (np.float64, torch.float64, "float64", "f64", "double"):
        return torch.float64
    if dtype in (np.float32, torch.float32, "float32", "f32", "float"):
        return torch.float32
    if hasattr(dtype, "name") and str(dtype.name) in ("float64", "float32"):
        return torch.float64 if dtype.name == "float64" else torch.float32
    raise ValueError(f"dtype must be float32 or float64; got {dtype!r}")


def constant_rows(c):
    """Rows whose right-hand side does not depend on the parameters (a zero row
    of ``rhs_map``)."""
    rhs_map = np.asarray(c.rhs_map, np.float64)
    if rhs_map.size == 0:  # no rows, or no parameters
        return np.ones(len(c.rhs0), bool)
    return ~np.any(rhs_map.reshape(len(c.rhs0), -1) != 0.0, axis=1)


def bounds_are_shared(c):
    """True when every sample gets the same variable bounds: the bound rows
    (inequality rows with one stored entry, presolved into bounds,
    bounds.py:320-326) all have constant right-hand sides and the coefficients
    are shared, so lower = max rhs/coef and upper = min rhs/coef
    (bounds.py:193-209) are the same for the whole batch.  The plan then reads
    one copy of the bounds (``shared_bounds``), which selects the on-chip
    kernels' broadcast-bounds variant; the results are identical either way."""
    if c.parametric_coefficients:
        return False
    lengths = np.diff(np.asarray(c.indptr, np.int64))
    bound_rows = np.zeros(len(lengths), bool)
    bound_rows[c.me:] = lengths[c.me:] == 1
    return bool(np.all(constant_rows(c)[bound_rows]))


class _ProjectFn(torch.autograd.Function):
    """y = P(y_hat; rhs, values) with the implicit VJP of the HIP adjoint.

    ``values`` (B, nnz) are per-sample coefficients (parameter-dependent rows)
    or None for the plan's shared ones.
    """

    @staticmethod
    def forward(ctx, y_hat, rhs, values, layer, multipliers0, save):
        vals = None if values is None else values.detach().contiguous()
        out = layer.plan.project(y_hat, rhs, multipliers0=multipliers0, save=save, values=vals,
                                 **layer._solve_kwargs())
        ctx.layer = layer
        ctx.saved_state = out.saved
        ctx.values = vals
        ctx.shapes = (y_hat.shape, rhs.shape)
        ctx.mark_non_differentiable(out.multipliers, out.slacks, out.status, out.iterations,
                                    out.residual, out.finite, out.eligible)
        return (out.y, out.multipliers, out.slacks, out.status, out.iterations, out.residual,
                out.finite, out.eligible)

    @staticmethod
    def backward(ctx, cot_y, *unused):
        layer = ctx.layer
        if cot_y is None:
            return None, None, None, None, None, None
        lin = layer.config.linear_solver
        adj = layer.plan.adjoint(ctx.saved_state, None, None, cot_y.contiguous(),
                                 tolerance=lin.tolerance, atol=lin.atol, restart=lin.restart,
                                 max_iterations=lin.max_iterations,
                                 adjoint_tolerance=layer.config.implicit_gradient.adjoint_tolerance,
                                 rhs_rows=layer.plan.me + layer.plan.mi, values=ctx.values)
        g_rhs = adj.g_rhs if ctx.needs_input_grad[1] else None
        g_values = adj.g_values if ctx.needs_input_grad[2] else None
        return adj.g_target, g_rhs, g_values, None, None, None


@dataclass(eq=False)
class PreparedChambollePockProjection:
    """A prepared CP projection for fixed (batch, dtype, backend)."""

    canonical: CanonicalRows
    config: ChambollePockConfig
    batch_size: int
    dtype: object
    backend: str

    def __post_init__(self):
        c = self.canonical
        if not c.affine:
            raise ValueError("chambolle-pock requires verified affine equalities and "
                             "inequalities; nonlinear or unverified constraints are unsupported")
        if not c.parameter_affine:
            raise NotImplementedError(
                "constraint coefficients and right-hand sides must be affine in the parameters "
                "(products of parameters are not supported by the symbolic layer)")
        if self.batch_size < 1 or c.n < 1:
            raise ValueError("batch_size and variable_size must be positive")
        self.device = resolve_device(self.backend)
        self.torch_dtype = resolve_dtype(self.dtype)
        cfg = self.config
        values = c.values
        self.metric = None
        if cfg.metric_diagonal is not None and not all(v == 1.0 for v in cfg.metric_diagonal):
            diag = np.asarray(cfg.metric_diagonal, np.float64)
            if diag.size != c.n:
                raise ValueError(f"metric_diagonal must have {c.n} entries; got {diag.size}")
            inverse = 1 / np.sqrt(diag)
            values = values * inverse[c.indices]        # metric.py:59-68
            self.metric = diag
        self.plan = Plan(c.n, c.me, c.mi, c.indptr, c.indices, values, dtype=self.torch_dtype,
                         accelerated=cfg.accelerated, row_scaling=cfg.row_scaling,
                         norm_bound=cfg.norm_bound, norm_iterations=cfg.norm_iterations,
                         norm_seed=cfg.norm_seed, safety=cfg.safety,
                         diagonal_preconditioning=cfg.diagonal_preconditioning,
                         device=self.device)
        if self.metric is not None:
            root = np.sqrt(self.metric.astype(np.float64 if self.torch_dtype == torch.float64
                                              else np.float32)).astype(np.float64)
            self.plan.set_metric(root)
        self._rhs0 = torch.as_tensor(c.rhs0, dtype=self.torch_dtype, device=self.device)
        self._rhs_map = torch.as_tensor(c.rhs_map, dtype=self.torch_dtype, device=self.device)
        # rows whose right-hand side does not involve the parameters keep their
        # constant value for every sample (the reference evaluates them as
        # constants, so a non-finite theta does not reach them)
        self._const_rows = torch.as_tensor(constant_rows(c), device=self.device)
        self.shared_bounds = bounds_are_shared(c)
        # parameter-dependent coefficients: values(theta) = values0 + theta @ value_map.T
        # per sample (the reference's vmap(_numeric_one), bounds.py:192), scaled by the
        # metric like the shared values
        self._values0 = self._value_map = None
        if c.parametric_coefficients:
            vmap = np.asarray(c.value_map, np.float64)
            if self.metric is not None:
                vmap = vmap * (1 / np.sqrt(self.metric))[c.indices][:, None]
            self._values0 = torch.as_tensor(values, dtype=self.torch_dtype, device=self.device)
            self._value_map = torch.as_tensor(vmap, dtype=self.torch_dtype, device=self.device)

    # -- sizes (solver.py:67-85) ---------------------------------------------------
    @property
    def parameter_size(self):
        return int(self.canonical.parameter_size)

    @property
    def output_size(self):
        return int(self.canonical.n)

    @property
    def equality_size(self):
        return int(self.canonical.me)

    @property
    def inequality_size(self):
        return int(self.canonical.mi)

    # -- helpers -------------------------------------------------------------------
    def _solve_kwargs(self):
        return dict(tolerance=self.config.tolerance, max_iterations=self.config.max_iterations,
                    early_stop=self.config.early_stop, shared_bounds=self.shared_bounds)

    def _target(self, y_hat):
        t = torch.as_tensor(y_hat).to(device=self.device, dtype=self.torch_dtype)
        if t.ndim == 1:
            t = t[None, :]
        if tuple(t.shape) != (self.batch_size, self.output_size):
            raise ValueError(f"y_hat must have shape {(self.batch_size, self.output_size)}; "
                             f"got {tuple(t.shape)}")
        return t

    def _theta(self, parameters):
        p = self.parameter_size
        if parameters is None:
            if p:
                raise ValueError("parameters are required for this problem")
            theta = torch.zeros((self.batch_size, 0), dtype=self.torch_dtype, device=self.device)
        else:
            theta = torch.as_tensor(parameters).to(device=self.device, dtype=self.torch_dtype)
            if tuple(theta.shape) != (self.batch_size, p):
                raise ValueError(f"parameters must have shape {(self.batch_size, p)}; "
                                 f"got {tuple(theta.shape)}")
        if not self.config.implicit_gradient.differentiate_problem_parameters:
            theta = theta.detach()
        return theta

    def _rhs(self, theta):
        return torch.where(self._const_rows, self._rhs0, self._rhs0[None, :] + theta @ self._rhs_map.T)

    def _values(self, theta):
        if self._value_map is None:
            return None
        return self._values0[None, :] + theta @ self._value_map.T

    def _multipliers0(self, eq, iq):
        if eq is None and iq is None:
            return None
        B = self.batch_size
        eq = (torch.zeros((B, self.equality_size), dtype=self.torch_dtype, device=self.device)
              if eq is None else torch.as_tensor(eq).to(self.device, self.torch_dtype))
        iq = (torch.zeros((B, self.inequality_size), dtype=self.torch_dtype, device=self.device)
              if iq is None else torch.as_tensor(iq).to(self.device, self.torch_dtype))
        if tuple(eq.shape) != (B, self.equality_size) or tuple(iq.shape) != (B, self.inequality_size):
            raise ValueError("warm-start multiplier shapes do not match constraints")
        return torch.cat((eq, iq), dim=1).detach()

    def _run(self, y_hat, parameters, multipliers_eq=None, multipliers_ineq=None):
        target = self._target(y_hat)
        theta = self._theta(parameters)
        rhs = self._rhs(theta)
        values = self._values(theta)
        mult0 = self._multipliers0(multipliers_eq, multipliers_ineq)
        # the state the backward pass reads is saved only when a backward pass can run
        save = torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (target, rhs, values))
        y, mult, slacks, status, iters, res, fin, elig = _ProjectFn.apply(target, rhs, values,
                                                                          self, mult0, save)
        me = self.equality_size
        return ProjectionResult(y, mult[:, :me], mult[:, me:], slacks, status, iters, res, fin,
                                elig)

    # -- public API (solver.py:368-402) --------------------------------------------
    def solve(self, y_hat, parameters=None, initial_state=None):
        if initial_state is not None:
            raise ValueError("Use project_training multiplier arguments for CP warm starts")
        return self._run(y_hat, parameters)

    def __call__(self, y_hat, parameters=None):
        r = self.solve(y_hat, parameters)
        return r.y[0] if torch.as_tensor(y_hat).ndim == 1 else r.y

    def with_info(self, y_hat, parameters=None):
        r = self.solve(y_hat, parameters)
        y = r.y[0] if torch.as_tensor(y_hat).ndim == 1 else r.y
        return y, ProjectionInfo(r.status, r.iterations, r.residual_inf_norm, r.finite,
                                 r.gradient_eligible)

    def project_training(self, y_hat, parameters=None, *, multipliers_eq=None,
                         multipliers_ineq=None):
        r = self._run(y_hat, parameters, multipliers_eq, multipliers_ineq)
        return ProjectionTrainingOutput(r.y, r.multipliers_eq, r.multipliers_ineq, r.slacks,
                                        r.status, r.iterations, r.residual_inf_norm, r.finite,
                                        r.gradient_eligible)


def _canonical(problem):
    if isinstance(problem, CanonicalRows):
        return problem
    if hasattr(problem, "canonicalize"):
        return problem.canonicalize()
    raise TypeError("problem must be a Projection, ParametricQP/MatrixProblem or CanonicalRows")


@dataclass(frozen=True)
class ChambollePockProjection:
    """Definition object (reference solver.py:405-432)."""

    problem: object
    config: ChambollePockConfig = ChambollePockConfig()

    def prepare(self, *, batch_size, dtype=torch.float64, backend="gpu"):
        return PreparedChambollePockProjection(_canonical(self.problem), self.config,
                                               int(batch_size), dtype, str(backend))


def registered_methods():
    return tuple(m.value for m in ProjectionMethod)


def prepare_projection(problem, *, method="chambolle-pock", config=None, batch_size,
                       dtype=torch.float64, backend="gpu"):
    """One fixed-shape projection backend (reference src/purin/solvers/api.py:106-141)."""
    ProjectionMethod.normalize(method)
    cfg = ChambollePockConfig() if config is None else config
    if not isinstance(cfg, ChambollePockConfig):
        raise TypeError("chambolle-pock expects a ChambollePockConfig")
    return ChambollePockProjection(problem, cfg).prepare(batch_size=batch_size, dtype=dtype,
                                                         backend=backend)


@dataclass(frozen=True)
class Distance:
    """Euclidean nearest-feasible-point projection (reference projections/distance.py:8-34)."""

    problem: object
    method: str = "chambolle-pock"
    config: object = None

    def prepare(self, *, batch_size, dtype=torch.float64, backend="gpu"):
        return prepare_projection(self.problem, method=self.method, config=self.config,
                                  batch_size=batch_size, dtype=dtype, backend=backend)


@dataclass(frozen=True)
class WeightedDistance:
    """Nearest point in a positive diagonal metric (reference projections/distance.py:37-61)."""

    problem: object
    diagonal: object
    method: str = "chambolle-pock"
    config: object = None

    def prepare(self, *, batch_size, dtype=torch.float64, backend="gpu"):
        if ProjectionMethod.normalize(self.method) is not ProjectionMethod.CHAMBOLLE_POCK:
            raise ValueError("weighted projection supports chambolle-pock in this build")
        cfg = replace(self.config or ChambollePockConfig(),
                      metric_diagonal=tuple(float(v) for v in self.diagonal))
        return Distance(self.problem, self.method, cfg).prepare(batch_size=batch_size,
                                                                dtype=dtype, backend=backend)
