"""The device GMRES's raw-basis Gram--Schmidt against the oracle's CGS2 GMRES.

The HIP adjoint (``k_gm_tri`` in purin_amd/csrc/adjoint.hip) keeps the
Arnoldi basis as raw vectors Z with an upper-triangular map, v_j = sum_{i<=j}
Z_i Tm[i][j], so that each Arnoldi step reads the basis twice instead of three
times.  ``raw_basis_gmres`` below restates that scheme step for step in NumPy
(the same products, the lagged correction c = Hu u, the Pythagorean norm and
the masking).  In exact arithmetic it is the reference's two-pass classical
Gram--Schmidt GMRES (primal_dual_interior_point/operators.py:792-1125); these
tests check that in floating point it gives the oracle's solution, iteration
counts and info codes, and an orthonormal basis.
"""

import numpy as np
import pytest

from oracle import adjoint as oa


def raw_basis_gmres(matvec, rhs, *, tolerance, absolute_tolerance, restart, max_iterations,
                    return_basis=False):
    batch, width = rhs.shape
    dtype = rhs.dtype
    restart = int(min(restart, max_iterations, width))
    R = restart
    eps = dtype.type(1e-30)
    brk = dtype.type(1e-14)
    threshold = np.maximum(dtype.type(absolute_tolerance),
                           dtype.type(tolerance) * np.max(np.abs(rhs), axis=1, initial=0.0))
    x = np.zeros_like(rhs)
    residual_inf = np.max(np.abs(rhs - matvec(x)), axis=1, initial=0.0).astype(dtype)
    completed = 0
    row_iterations = np.zeros(batch, np.int32)
    bases = []
    while completed < max_iterations and np.any(residual_inf > threshold):
        cycle_limit = min(R, max_iterations - completed)
        residual = rhs - matvec(x)
        beta = np.sqrt(np.sum(residual * residual, axis=1))
        cycle_active = residual_inf > threshold
        Z = np.zeros((batch, R + 1, width), dtype)
        Z[:, 0] = residual * (dtype.type(1) / np.maximum(beta, eps))[:, None]
        Tm = np.zeros((batch, R + 1, R + 1), dtype)
        Tm[:, 0, 0] = 1
        Hu = np.zeros((batch, R + 1, R), dtype)
        U2 = np.zeros((batch, R + 1), dtype)
        H = np.zeros((batch, R + 1, R), dtype)
        cos = np.zeros((batch, R), dtype)
        sin = np.zeros((batch, R), dtype)
        g = np.zeros((batch, R + 1), dtype)
        g[:, 0] = beta
        steps = np.zeros(batch, np.int32)
        active = cycle_active.copy()
        it = 0
        while it < cycle_limit and np.any(active):
            nv = it + 1
            Tp = Tm[:, :nv, :nv]
            y = matvec(Z[:, it] * Tm[:, it, it][:, None])
            p = np.einsum("bid,bd->bi", Z[:, :nv], y)
            g1 = np.einsum("bij,bi->bj", Tp, p)                 # Tm^T p
            q1 = np.einsum("bij,bj->bi", Tp, g1)                # Tm g1
            y1 = y - np.einsum("bi,bid->bd", q1, Z[:, :nv])
            Z[:, it + 1] = y1
            p2 = np.einsum("bid,bd->bi", Z[:, :nv], y1)
            n1 = np.sum(y1 * y1, axis=1)
            g2 = np.einsum("bij,bi->bj", Tp, p2)
            c = np.einsum("bjk,bk->bj", Hu[:, :nv, :it], U2[:, :it])
            col = (g1 + g2) - c
            d2 = n1 - np.sum(g2 * g2, axis=1)
            next_norm = np.where(d2 < 0, dtype.type(0), np.sqrt(np.maximum(d2, 0)))
            next_norm = np.where(np.isnan(d2), d2, next_norm)
            Hu[:, :nv, it] = np.where(active[:, None], col, Hu[:, :nv, it])
            Hu[:, it + 1, it] = np.where(active, next_norm, Hu[:, it + 1, it])
            column = np.zeros((batch, R + 1), dtype)
            column[:, :nv] = col
            column[:, it + 1] = next_norm
            for ri in range(it):
                first, second = column[:, ri].copy(), column[:, ri + 1].copy()
                column[:, ri] = cos[:, ri] * first + sin[:, ri] * second
                column[:, ri + 1] = -sin[:, ri] * first + cos[:, ri] * second
            diag, sub = column[:, it], column[:, it + 1]
            rnorm = np.hypot(diag, sub)
            safe_r = np.maximum(rnorm, eps)
            nc = np.where(rnorm > eps, diag / safe_r, dtype.type(1))
            ns = np.where(rnorm > eps, sub / safe_r, dtype.type(0))
            cos[:, it] = np.where(active, nc, cos[:, it])
            sin[:, it] = np.where(active, ns, sin[:, it])
            column[:, it] = rnorm
            column[:, it + 1] = 0
            H[:, :, it] = np.where(active[:, None], column, H[:, :, it])
            pc, pn = g[:, it].copy(), g[:, it + 1].copy()
            rc, rn = nc * pc + ns * pn, -ns * pc + nc * pn
            g[:, it] = np.where(active, rc, pc)
            g[:, it + 1] = np.where(active, rn, pn)
            steps = np.where(active, it + 1, steps)
            est = np.abs(rn)
            finite = np.isfinite(est) & np.isfinite(rnorm) & np.isfinite(n1)
            inv = dtype.type(1) / np.maximum(next_norm, eps)
            Tm[:, it + 1, it + 1] = np.where(active, inv, 0)
            tg2 = np.einsum("bij,bj->bi", Tp, g2)
            Tm[:, :nv, it + 1] = np.where(active[:, None], -(tg2 * inv[:, None]), 0)
            U2[:, :nv] = np.where(active[:, None], g2 * inv[:, None], 0)
            active = active & finite & ~(next_norm <= brk) & (est > threshold)
            it += 1
        coeffs = np.zeros((batch, R), dtype)
        for row in range(R - 1, -1, -1):
            trailing = np.sum(H[:, row, :R] * coeffs, axis=1)
            d = H[:, row, row]
            safe = np.where(np.abs(d) > eps, d, dtype.type(1))
            coeffs[:, row] = np.where(row < steps, (g[:, row] - trailing) / safe, dtype.type(0))
        wc = np.zeros((batch, R), dtype)
        for b in range(batch):
            k = steps[b]
            wc[b, :k] = Tm[b, :k, :k] @ coeffs[b, :k]
        candidate = x + np.einsum("bi,bid->bd", wc, Z[:, :R])
        cand_norm = np.max(np.abs(rhs - matvec(candidate)), axis=1, initial=0.0).astype(dtype)
        x = np.where(cycle_active[:, None], candidate, x)
        residual_inf = np.where(cycle_active, cand_norm, residual_inf)
        completed += it
        row_iterations = row_iterations + steps
        if return_basis:
            bases.append((Z, Tm, steps))
    finite = np.all(np.isfinite(x), axis=1) & np.isfinite(residual_inf)
    info = np.where(~finite, 2, np.where(residual_inf <= threshold, 0, 1)).astype(np.int32)
    if return_basis:
        return x, info, residual_inf, row_iterations, bases
    return x, info, residual_inf, row_iterations


def _system(seed, batch, width, radius, dtype):
    """I - J^T with J a random contraction of spectral radius ``radius``, the
    shape of the CP fixed-point system (nonsymmetric, eigenvalues of I - J^T in
    the disc of radius ``radius`` about 1)."""
    rng = np.random.default_rng(seed)
    J = rng.normal(size=(batch, width, width))
    J *= radius / np.max(np.abs(np.linalg.eigvals(J)), axis=1)[:, None, None]
    A = (np.eye(width) - np.transpose(J, (0, 2, 1))).astype(dtype)
    rhs = rng.normal(size=(batch, width)).astype(dtype)
    return (lambda v: np.einsum("bij,bj->bi", A, v)), A, rhs


@pytest.mark.parametrize("restart,max_iterations,radius", [(10, 100, 0.9), (30, 100, 0.97),
                                                           (30, 300, 0.995), (7, 50, 0.6)])
def test_raw_basis_gmres_matches_cgs2_gmres(restart, max_iterations, radius):
    mv, A, rhs = _system(restart * 1000 + max_iterations, 6, 48, radius, np.float64)
    tol = dict(tolerance=1e-12, absolute_tolerance=0.0, restart=restart,
               max_iterations=max_iterations)
    x0, info0, r0, it0 = oa.batched_restarted_gmres(mv, rhs, **tol)
    x1, info1, r1, it1 = raw_basis_gmres(mv, rhs, **tol)
    np.testing.assert_array_equal(info1, info0)
    np.testing.assert_array_equal(it1, it0)
    assert np.max(np.abs(x1 - x0)) <= 1e-11 * np.max(np.abs(x0))
    exact = np.linalg.solve(A, rhs[..., None])[..., 0]
    conv = info0 == 0
    if conv.any():
        assert np.max(np.abs(x1[conv] - exact[conv])) <= 1e-9 * np.max(np.abs(exact))


def test_raw_basis_gmres_unconverged_iterate_matches():
    """Stopped by the iteration limit (info 1), the iterate is the Krylov
    minimiser of that many steps, fixed by the mathematics; both schemes agree."""
    mv, A, rhs = _system(5, 4, 64, 0.999, np.float64)
    tol = dict(tolerance=1e-14, absolute_tolerance=0.0, restart=30, max_iterations=45)
    x0, info0, r0, it0 = oa.batched_restarted_gmres(mv, rhs, **tol)
    x1, info1, r1, it1 = raw_basis_gmres(mv, rhs, **tol)
    assert np.all(info0 == 1)
    np.testing.assert_array_equal(info1, info0)
    assert np.max(np.abs(x1 - x0)) <= 1e-12 * np.max(np.abs(x0))
    assert np.max(np.abs(r1 - r0)) <= 1e-12 * np.max(np.abs(rhs))


def test_raw_basis_is_orthonormal():
    """The implied basis V = Z Tm is orthonormal to rounding error, and Tm's
    off-diagonal entries stay at rounding level (Z_{j+1} is nearly orthogonal
    to the prefix already)."""
    mv, A, rhs = _system(11, 3, 80, 0.99, np.float64)
    *_, bases = raw_basis_gmres(mv, rhs, tolerance=1e-14, absolute_tolerance=0.0, restart=30,
                                max_iterations=30, return_basis=True)
    Z, Tm, steps = bases[0]
    for b in range(Z.shape[0]):
        k = int(steps[b]) + 1
        V = np.einsum("id,ij->jd", Z[b, :k], Tm[b, :k, :k])
        assert np.max(np.abs(V @ V.T - np.eye(k))) <= 1e-13
        off = np.triu(Tm[b, :k, :k], 1) / np.abs(np.diag(Tm[b, :k, :k]))[None, :]
        assert np.max(np.abs(off)) <= 1e-12


def test_raw_basis_gmres_happy_breakdown_and_fp32():
    """A system solved exactly in few steps (low-rank perturbation of I) stops
    by happy breakdown in both schemes; fp32 agrees to its own precision."""
    rng = np.random.default_rng(3)
    batch, width = 5, 40
    Uv = rng.normal(size=(batch, width, 3))
    A = np.eye(width) + 0.3 * Uv @ np.transpose(Uv, (0, 2, 1)) / width
    rhs = rng.normal(size=(batch, width))
    mv = lambda v: np.einsum("bij,bj->bi", A, v)  # noqa: E731
    tol = dict(tolerance=1e-13, absolute_tolerance=0.0, restart=30, max_iterations=100)
    x0, info0, _, it0 = oa.batched_restarted_gmres(mv, rhs, **tol)
    x1, info1, _, it1 = raw_basis_gmres(mv, rhs, **tol)
    np.testing.assert_array_equal(info1, info0)
    np.testing.assert_array_equal(it1, it0)
    assert np.all(it0 <= 5)
    assert np.max(np.abs(x1 - x0)) <= 1e-13 * np.max(np.abs(x0))
    A32, rhs32 = A.astype(np.float32), rhs.astype(np.float32)
    mv32 = lambda v: np.einsum("bij,bj->bi", A32, v)  # noqa: E731
    tol32 = dict(tolerance=1e-5, absolute_tolerance=0.0, restart=30, max_iterations=100)
    y0, j0, _, _ = oa.batched_restarted_gmres(mv32, rhs32, **tol32)
    y1, j1, _, _ = raw_basis_gmres(mv32, rhs32, **tol32)
    np.testing.assert_array_equal(j1, j0)
    assert np.max(np.abs(y1 - y0)) <= 1e-5 * np.max(np.abs(y0))
