"""Problem front ends producing shared-coefficient canonical rows.

* ``Projection``: the reference's symbolic builder (``add_parameter``,
  ``add_variable``, ``constraints.add(a == b, c <= d, e >= f)``) restricted to
  what the CP path consumes: constraints affine in the variables, with
  constant coefficients and right-hand sides affine in the parameters.
  Sign convention of reference src/purin/problems/expressions.py:298-309:
  ``a <= b`` is the residual ``a - b <= 0``, ``a >= b`` is ``b - a <= 0``,
  ``a == b`` is ``a - b == 0``.
* ``ParametricQP`` / ``MatrixProblem``: the matrix adapter of reference
  src/purin/problems/qp.py:83-402 (``A_eq y == b_eq0 + M_eq theta``,
  ``A_ineq y <= b_ineq0 + M_ineq theta``; the objective is unused by a distance
  projection).

Both canonicalise to ``CanonicalRows``: CSR rows (equalities first, columns
ascending, as reference src/purin/problems/problem.py:358-364) and
``rhs(theta) = rhs0 + rhs_map @ theta`` (= ``-[h(theta,0); g(theta,0)]``).
"""

from __future__ import annotations

import numbers
from dataclasses import dataclass

import numpy as np


@dataclass
class CanonicalRows:
    n: int
    me: int
    mi: int
    parameter_size: int
    indptr: np.ndarray
    indices: np.ndarray
    values: np.ndarray
    rhs0: np.ndarray
    rhs_map: np.ndarray          # (me+mi, parameter_size)
    variable_names: tuple = ()
    affine: bool = True
    parametric_coefficients: bool = False
    # per-entry coefficient map: values(theta) = values + theta @ value_map.T,
    # (nnz, parameter_size), when coefficients depend on parameters
    value_map: np.ndarray | None = None
    parameter_affine: bool = True  # rows (coefficients and rhs) affine in theta

    def coefficient_values(self, theta):
        """(B, nnz) coefficient values at theta (the plan's CSR entry order)."""
        theta = np.asarray(theta, np.float64).reshape(-1, self.parameter_size)
        if self.value_map is None:
            return np.broadcast_to(self.values, (theta.shape[0], self.values.size))
        return self.values[None, :] + theta @ self.value_map.T

    def rhs(self, theta):
        theta = np.asarray(theta, np.float64).reshape(-1, self.parameter_size)
        return self.rhs0[None, :] + theta @ self.rhs_map.T


# ---------------------------------------------------------------------------
# symbolic expressions
# ---------------------------------------------------------------------------


class Expression:
    """Polynomial of degree <= 2 in (variables, parameters) tracked exactly.

    ``var``: variable -> coefficient; ``par``: parameter -> coefficient;
    ``bil``: (variable, parameter) -> coefficient; ``const``; ``nonlinear``
    flags anything outside that set (e.g. ``y**2``, ``y*y``, ``abs(y)``).
    """

    __slots__ = ("var", "par", "bil", "const", "deps", "nonlinear", "par_nonlinear", "text")

    def __init__(self, var=None, par=None, bil=None, const=0.0, deps=frozenset(),
                 nonlinear=False, par_nonlinear=False, text=""):
        self.var = dict(var or {})
        self.par = dict(par or {})
        self.bil = dict(bil or {})
        self.const = float(const)
        self.deps = frozenset(deps)
        self.nonlinear = bool(nonlinear)
        self.par_nonlinear = bool(par_nonlinear)
        self.text = text

    # -- helpers ----------------------------------------------------------
    @staticmethod
    def lift(x):
        if isinstance(x, Expression):
            return x
        if isinstance(x, numbers.Real) or (isinstance(x, np.ndarray) and x.ndim == 0):
            return Expression(const=float(x), text=repr(float(x)))
        raise TypeError(f"cannot use {type(x).__name__} in a symbolic expression")

    def _has_vars(self):
        return bool(self.var or self.bil or self.deps)

    def _has_pars(self):
        return bool(self.par or self.bil)

    def _scaled(self, s):
        return Expression({k: v * s for k, v in self.var.items()},
                          {k: v * s for k, v in self.par.items()},
                          {k: v * s for k, v in self.bil.items()}, self.const * s, self.deps,
                          self.nonlinear, self.par_nonlinear, f"({s!r}*{self.text})")

    # -- arithmetic ----------------------------------------------------------
    def __add__(self, other):
        o = Expression.lift(other)
        out = Expression(self.var, self.par, self.bil, self.const + o.const, self.deps | o.deps,
                         self.nonlinear or o.nonlinear, self.par_nonlinear or o.par_nonlinear,
                         f"({self.text} + {o.text})")
        for src, dst in ((o.var, out.var), (o.par, out.par), (o.bil, out.bil)):
            for k, v in src.items():
                dst[k] = dst.get(k, 0.0) + v
        return out

    __radd__ = __add__

    def __neg__(self):
        return self._scaled(-1.0)

    def __sub__(self, other):
        return self + (-Expression.lift(other))

    def __rsub__(self, other):
        return Expression.lift(other) + (-self)

    def __mul__(self, other):
        o = Expression.lift(other)
        if not o._has_vars() and not o._has_pars() and not o.nonlinear:
            return self._scaled(o.const)
        if not self._has_vars() and not self._has_pars() and not self.nonlinear:
            return o._scaled(self.const)
        out = Expression(const=self.const * o.const, deps=self.deps | o.deps,
                         text=f"({self.text}*{o.text})")
        out.nonlinear = self.nonlinear or o.nonlinear
        out.par_nonlinear = self.par_nonlinear or o.par_nonlinear
        if self.bil or o.bil or (self.var and o.var):
            out.nonlinear = out.nonlinear or bool(self.var and o.var) or bool(
                (self.bil and (o.var or o.par or o.bil)) or (o.bil and (self.var or self.par)))
        for a, b in ((self, o), (o, self)):
            for k, v in a.var.items():
                out.var[k] = out.var.get(k, 0.0) + v * b.const
                for p, w in b.par.items():
                    out.bil[(k, p)] = out.bil.get((k, p), 0.0) + v * w
            for p, v in a.par.items():
                out.par[p] = out.par.get(p, 0.0) + v * b.const
        if self.par and o.par:
            out.par_nonlinear = True
        return out

    __rmul__ = __mul__

    def __truediv__(self, other):
        o = Expression.lift(other)
        if o._has_vars() or o._has_pars() or o.nonlinear:
            out = self * o
            out.nonlinear = out.nonlinear or o._has_vars()
            out.par_nonlinear = True
            return out
        return self._scaled(1.0 / o.const)

    def __pow__(self, k):
        if k == 1:
            return self
        out = self * self
        if self._has_vars():
            out.nonlinear = True
        return out

    def __abs__(self):
        out = Expression(self.var, self.par, self.bil, self.const, self.deps, self._has_vars(),
                         True, f"abs({self.text})")
        return out

    # -- comparisons -------------------------------------------------------
    def __le__(self, other):
        o = Expression.lift(other)
        return Constraint(self - o, "ineq", f"{self.text} <= {o.text}")

    def __ge__(self, other):
        o = Expression.lift(other)
        return Constraint(o - self, "ineq", f"{self.text} >= {o.text}")

    def __eq__(self, other):  # noqa: D105
        o = Expression.lift(other)
        return Constraint(self - o, "eq", f"{self.text} == {o.text}")

    __hash__ = object.__hash__

    def __bool__(self):
        raise TypeError("Symbolic expressions do not have a truth value. Use ==, <=, or >= "
                        "inside problem.constraints.add(...).")

    def __repr__(self):
        return f"Expression({self.text})"


class Constraint:
    def __init__(self, residual, kind, text):
        if kind not in {"eq", "ineq"}:
            raise ValueError(f"Constraint kind must be 'eq' or 'ineq'; got {kind!r}.")
        self.residual = residual
        self.kind = kind
        self.text = text

    def __bool__(self):
        raise TypeError("constraints have no truth value; add them with problem.constraints.add")


class ConstraintList:
    """``problem.constraints.add(...)`` (reference src/purin/problems/expressions.py:456-467)."""

    def __init__(self):
        self.items = []

    def add(self, *constraints):
        for c in constraints:
            if isinstance(c, (list, tuple)):
                self.add(*c)
                continue
            if not isinstance(c, Constraint):
                raise TypeError("constraints.add(...) expects symbolic comparisons created with "
                                "==, <=, or >=.")
            self.items.append(c)
        return self

    def equality(self, expression, *, name=None):
        r = Expression.lift(expression)
        self.items.append(Constraint(r, "eq", name or f"{r.text} == 0"))
        return self

    def inequality(self, expression, *, name=None):
        r = Expression.lift(expression)
        self.items.append(Constraint(r, "ineq", name or f"{r.text} <= 0"))
        return self

    def __iter__(self):
        return iter(self.items)

    def __len__(self):
        return len(self.items)


class _Namespace:
    def __init__(self, problem, kind):
        object.__setattr__(self, "_problem", problem)
        object.__setattr__(self, "_kind", kind)

    def __getattr__(self, name):
        p = object.__getattribute__(self, "_problem")
        kind = object.__getattribute__(self, "_kind")
        names = p.variable_names if kind == "variable" else p.parameter_names
        if name not in names:
            raise AttributeError(f"unknown {kind} {name!r}")
        i = names.index(name)
        if kind == "variable":
            return Expression(var={i: 1.0}, deps={i}, text=name)
        return Expression(par={i: 1.0}, text=name)

    def __getitem__(self, name):
        return self.__getattr__(name)

    def vector(self):
        p = object.__getattribute__(self, "_problem")
        kind = object.__getattribute__(self, "_kind")
        names = p.variable_names if kind == "variable" else p.parameter_names
        return [self.__getattr__(n) for n in names]


def _coerce_names(names):
    if isinstance(names, str):
        return [names]
    return [str(n) for n in names]


class Projection:
    """Symbolic constraint system (reference src/purin/problems/projection.py:9-35)."""

    def __init__(self, name="projection", *, method="chambolle-pock", config=None):
        self.name = str(name)
        self.method = str(method)
        self.config = config
        self.parameter_names = []
        self.variable_names = []
        self.parameter = _Namespace(self, "parameter")
        self.variable = _Namespace(self, "variable")
        self.parameters = self.parameter
        self.variables = self.variable
        self.constraints = ConstraintList()
        self._objective = None

    @property
    def objective(self):
        return self._objective

    @objective.setter
    def objective(self, expression):
        # a distance projection replaces the objective; keep it for inspection
        self._objective = expression

    def add_parameter(self, names):
        for n in _coerce_names(names):
            self._register(n, self.parameter_names)
        return self.parameter

    def add_variable(self, names):
        for n in _coerce_names(names):
            self._register(n, self.variable_names)
        return self.variable

    def _register(self, name, target):
        if name in self.parameter_names or name in self.variable_names:
            raise ValueError(f"Duplicate symbol name {name!r}.")
        target.append(name)

    def canonicalize(self):
        """Constant-coefficient affine rows and an affine rhs map."""
        n, p = len(self.variable_names), len(self.parameter_names)
        eq = [c for c in self.constraints if c.kind == "eq"]
        iq = [c for c in self.constraints if c.kind == "ineq"]
        rows, vals, vmaps, rhs0, rmap = [], [], [], [], []
        affine, parametric, par_affine = True, False, True
        for c in eq + iq:
            r = c.residual
            if r.nonlinear:
                affine = False
            if r.bil:
                parametric = True
            if r.par_nonlinear:
                par_affine = False
            cols = sorted(r.deps)
            rows.append(cols)
            vals.append([r.var.get(j, 0.0) for j in cols])
            for j in cols:  # coefficient of variable j: var[j] + sum_k bil[(j, k)] theta_k
                v = np.zeros(p)
                for (jj, k), w in r.bil.items():
                    if jj == j:
                        v[k] += w
                vmaps.append(v)
            rhs0.append(-r.const)
            m = np.zeros(p)
            for k, v in r.par.items():
                m[k] = -v
            rmap.append(m)
        indptr = np.zeros(len(rows) + 1, np.int64)
        indptr[1:] = np.cumsum([len(r) for r in rows])
        indices = np.asarray([c for r in rows for c in r], np.int32)
        values = np.asarray([v for r in vals for v in r], np.float64)
        value_map = np.asarray(vmaps, np.float64).reshape(len(values), p) if parametric else None
        return CanonicalRows(n, len(eq), len(iq), p, indptr, indices, values,
                             np.asarray(rhs0, np.float64), np.asarray(rmap, np.float64).reshape(len(rows), p),
                             tuple(self.variable_names), affine, parametric, value_map, par_affine)


# ---------------------------------------------------------------------------
# matrix adapter
# ---------------------------------------------------------------------------


def _rows_of(matrix, shape):
    import scipy.sparse as sp

    if matrix is None:
        return [[] for _ in range(shape[0])], [[] for _ in range(shape[0])]
    if sp.issparse(matrix):
        csr = sp.csr_matrix(matrix, dtype=np.float64)
        if csr.shape != shape:
            raise ValueError(f"matrix must have shape {shape}, got {csr.shape}")
        out_c, out_v = [], []
        for i in range(shape[0]):
            s, e = csr.indptr[i], csr.indptr[i + 1]
            order = np.argsort(csr.indices[s:e], kind="stable")
            out_c.append(csr.indices[s:e][order].tolist())
            out_v.append(csr.data[s:e][order].tolist())
        return out_c, out_v
    dense = np.asarray(matrix, np.float64)
    if dense.shape != shape:
        raise ValueError(f"matrix must have shape {shape}, got {dense.shape}")
    cols = [np.flatnonzero(r).tolist() for r in dense]
    return cols, [dense[i, c].tolist() for i, c in enumerate(cols)]


def _vec(v, size, name):
    if v is None:
        return np.zeros(size)
    a = np.asarray(v, np.float64)
    if a.shape != (size,):
        raise ValueError(f"{name} must have shape {(size,)}, got {a.shape}")
    return a


class ParametricQP:
    """Matrix-form problem (reference src/purin/problems/qp.py:83-235)."""

    def __init__(self, P, q0, q_parameter_map=None, A_eq=None, b_eq0=None,
                 b_eq_parameter_map=None, A_ineq=None, b_ineq0=None,
                 b_ineq_parameter_map=None, name="parametric_qp"):
        shape = np.shape(P) if not hasattr(P, "shape") else P.shape
        if len(shape) != 2 or shape[0] != shape[1]:
            raise ValueError("P must be square")
        self.n = int(shape[0])
        self.name = name
        maps = [m for m in (q_parameter_map, b_eq_parameter_map, b_ineq_parameter_map)
                if m is not None]
        self.parameter_size = int(np.shape(maps[0])[1]) if maps else 0
        if any(int(np.shape(m)[1]) != self.parameter_size for m in maps):
            raise ValueError("parameter maps must share one parameter dimension")
        self.me = 0 if A_eq is None else int(np.shape(A_eq)[0])
        self.mi = 0 if A_ineq is None else int(np.shape(A_ineq)[0])
        self.A_eq, self.A_ineq = A_eq, A_ineq
        self.b_eq0 = _vec(b_eq0, self.me, "b_eq0")
        self.b_ineq0 = _vec(b_ineq0, self.mi, "b_ineq0")
        p = self.parameter_size
        self.b_eq_parameter_map = (np.zeros((self.me, p)) if b_eq_parameter_map is None
                                   else np.asarray(b_eq_parameter_map, np.float64))
        self.b_ineq_parameter_map = (np.zeros((self.mi, p)) if b_ineq_parameter_map is None
                                     else np.asarray(b_ineq_parameter_map, np.float64))

    @classmethod
    def from_bounds(cls, *, P, q0, A, lower0, upper0, q_parameter_map=None,
                    lower_parameter_map=None, upper_parameter_map=None, name="parametric_qp"):
        """Two-sided rows ``lower <= A y <= upper`` (reference qp.py:308-398)."""
        import scipy.sparse as sp

        lower0 = np.asarray(lower0, np.float64)
        upper0 = np.asarray(upper0, np.float64)
        if lower0.shape != upper0.shape:
            raise ValueError("lower0 and upper0 shapes must match")
        eqm = np.isfinite(lower0) & np.isfinite(upper0) & (lower0 == upper0)
        um = np.isfinite(upper0) & ~eqm
        lm = np.isfinite(lower0) & ~eqm
        Am = sp.csr_matrix(A) if sp.issparse(A) else np.asarray(A, np.float64)
        p = 0
        for cand in (q_parameter_map, lower_parameter_map, upper_parameter_map):
            if cand is not None:
                p = int(np.shape(cand)[1])
                break
        eq_map = (np.zeros((int(eqm.sum()), p)) if upper_parameter_map is None
                  else np.asarray(upper_parameter_map)[eqm])
        parts, rhs, maps = [], [], []
        if um.any():
            parts.append(Am[um])
            rhs.append(upper0[um])
            maps.append(np.zeros((int(um.sum()), p)) if upper_parameter_map is None
                        else np.asarray(upper_parameter_map)[um])
        if lm.any():
            parts.append(-Am[lm])
            rhs.append(-lower0[lm])
            maps.append(np.zeros((int(lm.sum()), p)) if lower_parameter_map is None
                        else -np.asarray(lower_parameter_map)[lm])
        ncol = Am.shape[1]
        if sp.issparse(Am):
            A_ineq = sp.vstack(parts, format="csr") if parts else sp.csr_matrix((0, ncol))
        else:
            A_ineq = np.vstack(parts) if parts else np.zeros((0, ncol))
        return cls(P=P, q0=q0, q_parameter_map=q_parameter_map, A_eq=Am[eqm], b_eq0=upper0[eqm],
                   b_eq_parameter_map=eq_map, A_ineq=A_ineq,
                   b_ineq0=np.concatenate(rhs) if rhs else np.zeros(0),
                   b_ineq_parameter_map=np.vstack(maps) if maps else np.zeros((0, p)), name=name)

    def canonicalize(self):
        ce, ve = _rows_of(self.A_eq, (self.me, self.n))
        ci, vi = _rows_of(self.A_ineq, (self.mi, self.n))
        rows, vals = ce + ci, ve + vi
        indptr = np.zeros(len(rows) + 1, np.int64)
        indptr[1:] = np.cumsum([len(r) for r in rows])
        indices = np.asarray([c for r in rows for c in r], np.int32)
        values = np.asarray([v for r in vals for v in r], np.float64)
        return CanonicalRows(self.n, self.me, self.mi, self.parameter_size, indptr, indices,
                             values, np.concatenate((self.b_eq0, self.b_ineq0)),
                             np.vstack((self.b_eq_parameter_map, self.b_ineq_parameter_map)))

    compile = canonicalize


MatrixProblem = ParametricQP
ParametricLP = ParametricQP
