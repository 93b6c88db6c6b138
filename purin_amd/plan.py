"""Host-side wrapper of a prepared ``purin_cp_plan`` operating on torch device tensors.

torch supplies device memory and the current HIP stream; every computation
runs in the HIP kernels of ``libpurin_cp.so``.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from purin_amd import _lib


def _dtype_code(dtype):
    dtype = torch.float64 if dtype in (np.float64, torch.float64, "float64") else dtype
    dtype = torch.float32 if dtype in (np.float32, torch.float32, "float32") else dtype
    if dtype == torch.float64:
        return _lib.F64, torch.float64
    if dtype == torch.float32:
        return _lib.F32, torch.float32
    raise ValueError(f"dtype must be float32 or float64; got {dtype}")


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _u8(t):
    return None if t is None else C.cast(C.c_void_p(t.data_ptr()), C.POINTER(C.c_uint8))


def _i32(t):
    return None if t is None else C.cast(C.c_void_p(t.data_ptr()), C.POINTER(C.c_int32))


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _set_workspace(o, workspace):
    """Point an options struct at a caller workspace (a device tensor) or leave
    the plan's own (None)."""
    if workspace is None:
        return
    if not isinstance(workspace, torch.Tensor) or not workspace.is_cuda:
        raise ValueError("workspace must be a device tensor")
    o.workspace = C.c_void_p(workspace.data_ptr())
    o.workspace_bytes = workspace.numel() * workspace.element_size()


def _flags(t):
    """A 0/1 uint8 flag array returned by the library, seen as bool without a copy
    (every flag the kernels write is exactly 0 or 1), so a call launches no
    conversion kernel after the library's own work."""
    return t.view(torch.bool)


@dataclass
class CPOutput:
    """Inner solve result (reference src/purin/solvers/chambolle_pock/kernels.py:15-23)."""

    y: torch.Tensor
    dual: torch.Tensor
    iterations: torch.Tensor
    residual: torch.Tensor
    gap: torch.Tensor
    converged: torch.Tensor


@dataclass
class ProjectOutput:
    y: torch.Tensor
    multipliers: torch.Tensor
    slacks: torch.Tensor
    status: torch.Tensor
    iterations: torch.Tensor
    residual: torch.Tensor
    finite: torch.Tensor
    eligible: torch.Tensor
    saved: torch.Tensor | None


@dataclass
class AdjointOutput:
    g_target: torch.Tensor
    g_rhs: torch.Tensor
    g_lower: torch.Tensor | None
    g_upper: torch.Tensor | None
    valid: torch.Tensor
    info: torch.Tensor
    residual: torch.Tensor
    g_values: torch.Tensor | None = None
    steps: torch.Tensor | None = None  # per-sample Arnoldi steps (arnoldi_iterations)


@dataclass
class QPOutput:
    y: torch.Tensor
    multipliers: torch.Tensor
    slacks: torch.Tensor
    status: torch.Tensor
    iterations: torch.Tensor
    residual: torch.Tensor
    finite: torch.Tensor
    converged: torch.Tensor
    saved: torch.Tensor | None


@dataclass
class QPAdjointOutput:
    g_q: torch.Tensor
    g_c: torch.Tensor
    g_values: torch.Tensor
    g_rhs: torch.Tensor
    g_lower: torch.Tensor
    g_upper: torch.Tensor
    valid: torch.Tensor
    info: torch.Tensor
    residual: torch.Tensor


class Plan:
    """A prepared shared-matrix CP plan (``purin_cp_plan_create``)."""

    def __init__(self, n, me, mi, indptr, indices, values, *, dtype=torch.float64,
                 accelerated=False, row_scaling=True, norm_bound=True, norm_iterations=20,
                 norm_seed=42, safety=0.95, diagonal_preconditioning=False, device="cuda",
                 bound_presolve=True):
        self.lib = _lib.load()
        self.code, self.dtype = _dtype_code(dtype)
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("the HIP projection runs on a GPU device ('cuda'/'cuda:N')")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        indptr = np.ascontiguousarray(indptr, dtype=np.int64)
        indices = np.ascontiguousarray(indices, dtype=np.int32)
        values = np.ascontiguousarray(values, dtype=np.float64)
        if indptr.size != me + mi + 1:
            raise ValueError("indptr must have me + mi + 1 entries")
        opts = _lib.default_options()
        opts.accelerated = int(bool(accelerated))
        opts.row_scaling = int(bool(row_scaling))
        opts.norm_bound = int(bool(norm_bound))
        opts.norm_iterations = int(norm_iterations)
        opts.norm_seed = int(norm_seed)
        opts.safety = float(safety)
        opts.diagonal_preconditioning = int(bool(diagonal_preconditioning))
        opts.bound_presolve = int(bool(bound_presolve))
        handle = C.c_void_p()
        torch.cuda.set_device(self.device)
        _lib.check(self.lib.purin_cp_plan_create(
            C.byref(handle), self.code, int(n), int(me), int(mi),
            indptr.ctypes.data_as(C.POINTER(C.c_int64)),
            indices.ctypes.data_as(C.POINTER(C.c_int32)),
            values.ctypes.data_as(C.POINTER(C.c_double)), C.byref(opts)))
        self.handle = handle
        self.n, self.me, self.mi = int(n), int(me), int(mi)
        self.nnz = int(indptr[-1])  # entries of the caller's CSR (per-sample values width)
        info = _lib.PlanInfo()
        _lib.check(self.lib.purin_cp_plan_get_info(self.handle, C.byref(info)))
        self.info = info
        self.m = int(info.kept_rows)
        rows = np.zeros(self.m, np.int64)
        scale = np.zeros(self.m, np.float64)
        _lib.check(self.lib.purin_cp_plan_kept_rows(
            self.handle, rows.ctypes.data_as(C.POINTER(C.c_int64)),
            scale.ctypes.data_as(C.POINTER(C.c_double))))
        self.kept_rows = rows
        self.row_scale = scale
        self.metric_sqrt = None

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                self.lib.purin_cp_plan_destroy(h)
            except Exception:
                pass
            self.handle = None

    # ------------------------------------------------------------------
    def set_metric(self, sqrt_diagonal):
        if sqrt_diagonal is None:
            _lib.check(self.lib.purin_cp_plan_set_metric(self.handle, None))
            self.metric_sqrt = None
            return
        arr = np.ascontiguousarray(sqrt_diagonal, dtype=np.float64)
        if arr.shape != (self.n,):
            raise ValueError(f"metric_diagonal must have {self.n} entries; got {arr.size}")
        _lib.check(self.lib.purin_cp_plan_set_metric(self.handle,
                                                     arr.ctypes.data_as(C.POINTER(C.c_double))))
        self.metric_sqrt = arr

    def _tensor(self, x, shape, name):
        if not isinstance(x, torch.Tensor):
            x = torch.as_tensor(x)
        x = x.to(device=self.device, dtype=self.dtype)
        if tuple(x.shape) != tuple(shape):
            raise ValueError(f"{name} must have shape {tuple(shape)}; got {tuple(x.shape)}")
        return x.contiguous()

    def _empty(self, *shape, dtype=None):
        return torch.empty(shape, device=self.device, dtype=dtype or self.dtype)

    def saved_bytes(self, batch):
        return int(self.lib.purin_cp_saved_bytes(self.handle, int(batch)))

    def workspace_bytes(self, entry, batch, *, restart=30, max_iterations=100):
        """Caller-workspace bytes of an entry point (``purin_cp_workspace_bytes``);
        ``entry`` is a name of ``_lib.ENTRY``; restart / max_iterations are the
        adjoints' GMRES settings."""
        o = _lib.default_adjoint_options()
        o.restart = int(restart)
        o.max_iterations = int(max_iterations)
        n = int(self.lib.purin_cp_workspace_bytes(self.handle, _lib.ENTRY[entry], int(batch),
                                                   C.byref(o)))
        if n < 0:
            _lib.check(_lib.ERR_ARG)
        return n

    def new_workspace(self, entry, batch, **kw):
        """A device buffer of ``workspace_bytes(entry, batch, **kw)`` bytes."""
        return torch.empty(self.workspace_bytes(entry, batch, **kw), dtype=torch.uint8,
                           device=self.device)

    def current_info(self):
        """The plan's info now (its own workspaces' sizes change as calls grow them)."""
        info = _lib.PlanInfo()
        _lib.check(self.lib.purin_cp_plan_get_info(self.handle, C.byref(info)))
        return info

    # ------------------------------------------------------------------
    def spmm(self, x, *, transpose=False, scaled=True):
        """``K x`` (``(B, n) -> (B, m)``) or ``K^T x`` over the kept rows."""
        batch = x.shape[0]
        x = self._tensor(x, (batch, self.m if transpose else self.n), "x")
        out = self._empty(batch, self.n if transpose else self.m)
        _lib.check(self.lib.purin_cp_spmm(self.handle, _stream(), batch, int(transpose),
                                          int(scaled), _ptr(x), _ptr(out)))
        return out

    def solve(self, rhs, target, lower, upper, *, dual0=None, tol=None, feasible=None,
              tolerance=1e-9, max_iterations=10000, early_stop=True, check_every=32,
              shared_bounds=False, save=False, streaming=False, timing=False, workspace=None):
        """Inner CP solve on the kept rows (``purin_cp_solve``), scaled units."""
        batch = target.shape[0]
        target = self._tensor(target, (batch, self.n), "target")
        rhs = self._tensor(rhs, (batch, self.m), "rhs")
        bshape = (self.n,) if shared_bounds else (batch, self.n)
        lower = self._tensor(lower, bshape, "lower")
        upper = self._tensor(upper, bshape, "upper")
        dual0 = None if dual0 is None else self._tensor(dual0, (batch, self.m), "dual0")
        tol = None if tol is None else self._tensor(tol, (batch,), "tol")
        if feasible is not None:
            feasible = torch.as_tensor(feasible, device=self.device).to(torch.uint8).contiguous()
        o = _lib.default_solve_options()
        o.tolerance = float(tolerance)
        o.max_iterations = int(max_iterations)
        o.early_stop = int(bool(early_stop))
        o.check_every = int(check_every)
        o.shared_bounds = int(bool(shared_bounds))
        o.streaming = int(bool(streaming))
        o.timing = int(bool(timing))
        _set_workspace(o, workspace)
        y = self._empty(batch, self.n)
        dual = self._empty(batch, self.m)
        it = self._empty(batch, dtype=torch.int32)
        res = self._empty(batch)
        gap = self._empty(batch)
        conv = self._empty(batch, dtype=torch.uint8)
        saved = self._empty(self.saved_bytes(batch), dtype=torch.uint8) if save else None
        _lib.check(self.lib.purin_cp_solve(
            self.handle, _stream(), batch, _ptr(rhs), _ptr(target), _ptr(dual0), _ptr(lower),
            _ptr(upper), _ptr(tol), _u8(feasible), C.byref(o), _ptr(y), _ptr(dual), _i32(it),
            _ptr(res), _ptr(gap), _u8(conv), _ptr(saved)))
        out = CPOutput(y, dual, it, res, gap, _flags(conv))
        return (out, saved) if save else out

    def last_timing(self):
        """Kernel times of the last call made with ``timing=True`` (HIP events)."""
        t = _lib.Timing()
        _lib.check(self.lib.purin_cp_last_timing(self.handle, C.byref(t)))
        return {k: getattr(t, k) for k, _ in _lib.Timing._fields_}

    def last_adjoint_stats(self):
        """Arnoldi steps and restart cycles of the last ``adjoint`` call."""
        s = _lib.AdjointStats()
        _lib.check(self.lib.purin_cp_last_adjoint_stats(self.handle, C.byref(s)))
        return {"arnoldi_steps": int(s.arnoldi_steps), "cycles": int(s.cycles)}

    def last_adjoint_iterations(self, batch):
        """Per-sample Arnoldi steps of the last GMRES ``adjoint`` call (int32 (B,))."""
        out = self._empty(int(batch), dtype=torch.int32)
        _lib.check(self.lib.purin_cp_last_adjoint_iterations(self.handle, _stream(), int(batch),
                                                             _i32(out)))
        return out

    def project(self, target, rhs, *, multipliers0=None, tolerance=1e-9, max_iterations=10000,
                early_stop=True, check_every=32, shared_bounds=False, save=False, timing=False,
                streaming=False, values=None, noalloc=False, workspace=None, saved=None):
        """Full projection (``purin_cp_project``): BoundProjection.solve semantics.

        ``values`` (B, nnz): per-sample coefficients in the plan's CSR entry order
        (``purin_cp_project_values``); the plan's own coefficients are then unused.
        ``noalloc``: run ``purin_cp_project_noalloc`` (the library allocates no
        device memory during the call; its buffers sit in a static per-GPU
        scratch array of ``_lib.NOALLOC_SCRATCH_BYTES``).
        ``workspace``: a device buffer of at least ``workspace_bytes("project"
        or "project_values", B)`` bytes for the call's scratch (calls with
        their own workspaces may overlap on one plan); ``saved``: a buffer of
        ``saved_bytes(B)`` to fill (``save=True`` allocates one).
        """
        batch = target.shape[0]
        M = self.me + self.mi
        target = self._tensor(target, (batch, self.n), "y_hat")
        rhs = self._tensor(rhs, (batch, M), "rhs")
        if values is not None:
            values = self._tensor(values, (batch, self.nnz), "values")
        mult0 = None if multipliers0 is None else self._tensor(multipliers0, (batch, M),
                                                               "multipliers")
        o = _lib.default_solve_options()
        o.tolerance = float(tolerance)
        o.max_iterations = int(max_iterations)
        o.early_stop = int(bool(early_stop))
        o.check_every = int(check_every)
        o.shared_bounds = int(bool(shared_bounds))
        o.timing = int(bool(timing))
        o.streaming = int(bool(streaming))
        _set_workspace(o, workspace)
        y = self._empty(batch, self.n)
        mult = self._empty(batch, M)
        slacks = self._empty(batch, self.mi)
        status = self._empty(batch, dtype=torch.int32)
        it = self._empty(batch, dtype=torch.int32)
        res = self._empty(batch)
        fin = self._empty(batch, dtype=torch.uint8)
        elig = self._empty(batch, dtype=torch.uint8)
        if saved is None and save:
            saved = self._empty(self.saved_bytes(batch), dtype=torch.uint8)
        if values is not None:
            if noalloc:
                raise ValueError("the no-allocation entry takes the plan's own coefficients")
            _lib.check(self.lib.purin_cp_project_values(
                self.handle, _stream(), batch, _ptr(values), _ptr(target), _ptr(rhs),
                _ptr(mult0), C.byref(o), _ptr(y), _ptr(mult), _ptr(slacks), _i32(status),
                _i32(it), _ptr(res), _u8(fin), _u8(elig), _ptr(saved)))
            return ProjectOutput(y, mult, slacks, status, it, res, _flags(fin), _flags(elig),
                                 saved)
        entry = self.lib.purin_cp_project_noalloc if noalloc else self.lib.purin_cp_project
        _lib.check(entry(
            self.handle, _stream(), batch, _ptr(target), _ptr(rhs), _ptr(mult0), C.byref(o),
            _ptr(y), _ptr(mult), _ptr(slacks), _i32(status), _i32(it), _ptr(res), _u8(fin),
            _u8(elig), _ptr(saved)))
        return ProjectOutput(y, mult, slacks, status, it, res, _flags(fin), _flags(elig), saved)

    def qp_solve(self, q, c, rhs, lower, upper, *, values=None, y0=None, dual0=None,
                 tolerance=1e-9, max_iterations=10000, early_stop=True, check_every=32,
                 save=False, timing=False, workspace=None, streaming=False):
        """General diagonal QP (``purin_cp_qp_solve``): PreparedDiagonalQP.solve
        semantics on a plan created with ``bound_presolve=False``.  Fixed
        iterations with the plan's own coefficients run on the resident kernel
        where it applies; ``streaming`` forces the streaming passes."""
        batch = q.shape[0]
        M = self.me + self.mi
        q = self._tensor(q, (batch, self.n), "q")
        c = self._tensor(c, (batch, self.n), "c")
        rhs = self._tensor(rhs, (batch, M), "rhs")
        lower = self._tensor(lower, (batch, self.n), "lower")
        upper = self._tensor(upper, (batch, self.n), "upper")
        values = None if values is None else self._tensor(values, (batch, self.nnz), "values")
        y0 = None if y0 is None else self._tensor(y0, (batch, self.n), "initial_y")
        dual0 = None if dual0 is None else self._tensor(dual0, (batch, M), "initial_dual")
        o = _lib.default_solve_options()
        o.tolerance = float(tolerance)
        o.max_iterations = int(max_iterations)
        o.early_stop = int(bool(early_stop))
        o.check_every = int(check_every)
        o.timing = int(bool(timing))
        o.streaming = int(bool(streaming))
        _set_workspace(o, workspace)
        y = self._empty(batch, self.n)
        mult = self._empty(batch, M)
        slacks = self._empty(batch, self.mi)
        status = self._empty(batch, dtype=torch.int32)
        it = self._empty(batch, dtype=torch.int32)
        res = self._empty(batch)
        fin = self._empty(batch, dtype=torch.uint8)
        conv = self._empty(batch, dtype=torch.uint8)
        saved = self._empty(self.saved_bytes(batch), dtype=torch.uint8) if save else None
        _lib.check(self.lib.purin_cp_qp_solve(
            self.handle, _stream(), batch, _ptr(q), _ptr(c), _ptr(values), _ptr(rhs),
            _ptr(lower), _ptr(upper), _ptr(y0), _ptr(dual0), C.byref(o), _ptr(y), _ptr(mult),
            _ptr(slacks), _i32(status), _i32(it), _ptr(res), _u8(fin), _u8(conv), _ptr(saved)))
        return QPOutput(y, mult, slacks, status, it, res, _flags(fin), _flags(conv), saved)

    def dense_solve(self, q, c, rhs, lower, upper, *, values=None, y0=None, dual0=None,
                    tolerance=1e-9, max_iterations=5000, early_stop=True, check_every=32,
                    save=False, timing=False, workspace=None):
        """The dense adapter's forward (``purin_cp_dense_solve``, solve_dense
        semantics) on a plan with bound_presolve, row_scaling, norm_bound and
        diagonal_preconditioning off.  Returns (y, multipliers, iterations, saved)."""
        batch = q.shape[0]
        M = self.me + self.mi
        q = self._tensor(q, (batch, self.n), "q")
        c = self._tensor(c, (batch, self.n), "c")
        rhs = self._tensor(rhs, (batch, M), "rhs")
        lower = self._tensor(lower, (batch, self.n), "lower")
        upper = self._tensor(upper, (batch, self.n), "upper")
        values = None if values is None else self._tensor(values, (batch, self.nnz), "values")
        y0 = None if y0 is None else self._tensor(y0, (batch, self.n), "y0")
        dual0 = None if dual0 is None else self._tensor(dual0, (batch, M), "dual0")
        o = _lib.default_solve_options()
        o.tolerance = float(tolerance)
        o.max_iterations = int(max_iterations)
        o.early_stop = int(bool(early_stop))
        o.check_every = int(check_every)
        o.timing = int(bool(timing))
        _set_workspace(o, workspace)
        y = self._empty(batch, self.n)
        mult = self._empty(batch, M)
        it = self._empty(batch, dtype=torch.int32)
        saved = self._empty(self.saved_bytes(batch), dtype=torch.uint8) if save else None
        _lib.check(self.lib.purin_cp_dense_solve(
            self.handle, _stream(), batch, _ptr(q), _ptr(c), _ptr(values), _ptr(rhs),
            _ptr(lower), _ptr(upper), _ptr(y0), _ptr(dual0), C.byref(o), _ptr(y), _ptr(mult),
            _i32(it), _ptr(saved)))
        return y, mult, it, saved

    def dense_adjoint(self, saved, q, c, cot_y, *, values=None, cot_dual=None, tolerance=1e-6,
                      max_iterations=50, workspace=None):
        """The dense layer's backward (``purin_cp_dense_adjoint``): BiCGSTAB over the
        batch with the frozen prox.  Returns a QPAdjointOutput (valid/info None)."""
        batch = cot_y.shape[0]
        M = self.me + self.mi
        q = self._tensor(q, (batch, self.n), "q")
        c = self._tensor(c, (batch, self.n), "c")
        values = None if values is None else self._tensor(values, (batch, self.nnz), "values")
        cot = self._tensor(cot_y, (batch, self.n), "cotangent")
        cotd = None if cot_dual is None else self._tensor(cot_dual, (batch, M), "dual cotangent")
        o = _lib.default_adjoint_options()
        o.tolerance = float(tolerance)
        o.max_iterations = int(max_iterations)
        _set_workspace(o, workspace)
        gq, gc = self._empty(batch, self.n), self._empty(batch, self.n)
        gv = self._empty(batch, self.nnz)
        gr = self._empty(batch, M)
        gl, gu = self._empty(batch, self.n), self._empty(batch, self.n)
        _lib.check(self.lib.purin_cp_dense_adjoint(
            self.handle, _stream(), batch, _ptr(saved), _ptr(q), _ptr(c), _ptr(values), _ptr(cot),
            _ptr(cotd), C.byref(o), _ptr(gq), _ptr(gc), _ptr(gv), _ptr(gr), _ptr(gl), _ptr(gu)))
        return QPAdjointOutput(gq, gc, gv, gr, gl, gu, None, None, None)

    def qp_adjoint(self, saved, q, c, cot_y, *, values=None, cot_dual=None, tolerance=1e-9,
                   atol=0.0, restart=30, max_iterations=100, adjoint_tolerance=1e-8,
                   force_eligible=False, workspace=None):
        """Implicit VJP of ``qp_solve`` (``purin_cp_qp_adjoint``)."""
        batch = cot_y.shape[0]
        M = self.me + self.mi
        q = self._tensor(q, (batch, self.n), "q")
        c = self._tensor(c, (batch, self.n), "c")
        values = None if values is None else self._tensor(values, (batch, self.nnz), "values")
        cot = self._tensor(cot_y, (batch, self.n), "cotangent")
        cotd = None if cot_dual is None else self._tensor(cot_dual, (batch, M), "dual cotangent")
        o = _lib.default_adjoint_options()
        o.tolerance = float(tolerance)
        o.atol = float(atol)
        o.restart = int(restart)
        o.max_iterations = int(max_iterations)
        o.adjoint_tolerance = float(adjoint_tolerance)
        o.force_eligible = int(bool(force_eligible))
        _set_workspace(o, workspace)
        gq, gc = self._empty(batch, self.n), self._empty(batch, self.n)
        gv = self._empty(batch, self.nnz)
        gr = self._empty(batch, M)
        gl, gu = self._empty(batch, self.n), self._empty(batch, self.n)
        valid = self._empty(batch, dtype=torch.uint8)
        info = self._empty(batch, dtype=torch.int32)
        res = self._empty(batch)
        _lib.check(self.lib.purin_cp_qp_adjoint(
            self.handle, _stream(), batch, _ptr(saved), _ptr(q), _ptr(c), _ptr(values), _ptr(cot),
            _ptr(cotd), C.byref(o), _ptr(gq), _ptr(gc), _ptr(gv), _ptr(gr), _ptr(gl), _ptr(gu),
            _u8(valid), _i32(info), _ptr(res)))
        return QPAdjointOutput(gq, gc, gv, gr, gl, gu, _flags(valid), info, res)

    def adjoint(self, saved, target, rhs, cot_y, *, tolerance=1e-9, atol=0.0, restart=30,
                max_iterations=100, adjoint_tolerance=1e-8, force_eligible=False,
                bounds_grad=False, rhs_rows=None, values=None, workspace=None,
                return_steps=False):
        """Implicit VJP at a saved forward state (``purin_cp_adjoint``).

        ``values``: the per-sample coefficients of a ``project(..., values=...)``
        state (``purin_cp_adjoint_values``); the result then carries ``g_values``.
        ``workspace``: a caller workspace (``workspace_bytes("adjoint", B)``);
        ``return_steps``: fill ``steps`` with the per-sample Arnoldi steps.
        """
        batch = cot_y.shape[0]
        rows = rhs_rows if rhs_rows is not None else self.me + self.mi
        # target and rhs are held by the saved state; they are accepted for interface
        # parity with the reference's custom_vjp residuals and not re-read
        target = None if target is None else self._tensor(target, (batch, self.n), "target")
        rhs = None if rhs is None else self._tensor(rhs, (batch, rows), "rhs")
        cot = self._tensor(cot_y, (batch, self.n), "cotangent")
        o = _lib.default_adjoint_options()
        o.tolerance = float(tolerance)
        o.atol = float(atol)
        o.restart = int(restart)
        o.max_iterations = int(max_iterations)
        o.adjoint_tolerance = float(adjoint_tolerance)
        o.force_eligible = int(bool(force_eligible))
        _set_workspace(o, workspace)
        steps = self._empty(batch, dtype=torch.int32) if return_steps else None
        if steps is not None:
            o.arnoldi_iterations = _i32(steps)
        gt = self._empty(batch, self.n)
        gr = self._empty(batch, rows)
        gl = self._empty(batch, self.n) if bounds_grad else None
        gu = self._empty(batch, self.n) if bounds_grad else None
        valid = self._empty(batch, dtype=torch.uint8)
        info = self._empty(batch, dtype=torch.int32)
        res = self._empty(batch)
        if values is not None:
            values = self._tensor(values, (batch, self.nnz), "values")
            gv = self._empty(batch, self.nnz)
            _lib.check(self.lib.purin_cp_adjoint_values(
                self.handle, _stream(), batch, _ptr(saved), _ptr(values), _ptr(cot), C.byref(o),
                _ptr(gt), _ptr(gr), _ptr(gv), _u8(valid), _i32(info), _ptr(res)))
            return AdjointOutput(gt, gr, None, None, _flags(valid), info, res, gv, steps)
        _lib.check(self.lib.purin_cp_adjoint(
            self.handle, _stream(), batch, _ptr(saved), _ptr(target), _ptr(rhs), _ptr(cot),
            C.byref(o), _ptr(gt), _ptr(gr), _ptr(gl), _ptr(gu), _u8(valid), _i32(info),
            _ptr(res)))
        return AdjointOutput(gt, gr, gl, gu, _flags(valid), info, res, None, steps)
