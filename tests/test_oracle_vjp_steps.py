"""What the adjoint's step sizes may change in the VJP, at the config5 state (CPU, oracle).

The reference draws the power-iteration start vector that sets the adjoint's
tau and sigma from ``jax.random.PRNGKey(42)`` (kernels.py:52-65, bounds.py:83-101);
JAX is absent here, so this build uses its own start vector and its tau, sigma
differ from the reference's in the last digits of the norm estimate.  What the
mathematics fixes instead:

* the converged VJP does not depend on tau, sigma (it is the implicit
  derivative of the fixed point, whatever the fixed-point map's steps):
  two start vectors give the same VJP to rounding;
* an unconverged GMRES iterate lambda with residual r = g - (I - J^T) lambda is
  within ||(I - J^T)^-1|| ||r|| of the solution, so the VJP (linear in lambda)
  is within C * rho of the converged VJP, rho = ||r||_inf / ||g||_inf, for any
  tau, sigma.  C is a property of the problem, measured here at the config5
  state (largest observed: about 7 for the candidates' gradient and 34 for the
  right-hand sides') and stated as C = 50.  Two step choices therefore give
  100-step VJPs within C (rho_a + rho_b) of each other, and the GPU is held to
  that bound against the oracle's converged VJP (tests/test_gpu_fullsize.py).

The 100-step iterates are accepted here with ``adjoint_tolerance = 1``: at the
default 1e-8 the reference marks them invalid and returns zero gradients
(bounds.py:148-153), which would make every comparison vacuous.
"""

import numpy as np
import pytest

from oracle import adjoint as oadj
from oracle import cloop
from oracle import projection as op
from purin_amd import workloads

C_BOUND = 50.0
PICK = np.array([0, 300, 700, 1023])


@pytest.fixture(scope="module")
def state():
    cloop.build()
    w = workloads.config5()
    cfg = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False)
    canon = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    S = len(PICK)
    prep = cloop.prepare(canon, w.target[PICK], np.tile(w.rhs, (S, 1)), cfg, np.float64)
    y, d, _ = cloop.run(prep, w.iterations, True, threads=4)
    pre = op.presolve(canon, w.rhs[None, :], cfg, np.float64)
    return dict(w=w, y=y, d=d, pre=pre, S=S)


def _vjp(st, seed, tol, maxit):
    w, pre, S = st["w"], st["pre"], st["S"]
    cfg = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False,
                    norm_seed=seed, gmres_tolerance=tol, gmres_max_iterations=maxit,
                    adjoint_tolerance=1.0)
    return oadj.adjoint(pre.kept_values[0], pre.support[pre.rows], pre.mask[pre.rows], w.me,
                        st["y"], st["d"], np.ones(S, bool), w.target[PICK],
                        np.tile(pre.kept_rhs, (S, 1)),
                        np.broadcast_to(pre.lower[0], (S, w.n)),
                        np.broadcast_to(pre.upper[0], (S, w.n)), w.cotangent[PICK], cfg)


def _rel(a, b):
    return np.max(np.abs(a - b), axis=1) / np.max(np.abs(b), axis=1)


def test_adjoint_steps_move_the_vjp_only_within_the_gmres_residual(state):
    conv = {s: _vjp(state, s, 1e-14, 1000) for s in (42, 7)}
    short = {s: _vjp(state, s, 1e-9, 100) for s in (42, 7)}
    assert not np.isclose(np.ravel(conv[42].tau)[0], np.ravel(conv[7].tau)[0], rtol=1e-6, atol=0)
    # converged: the step sizes do not matter
    assert np.all(conv[42].info == 0) and np.all(conv[7].info == 0)
    assert np.all(_rel(conv[7].g_target, conv[42].g_target) <= 1e-12)
    assert np.all(_rel(conv[7].g_rhs, conv[42].g_rhs) <= 1e-12)
    # 100 steps: within C * rho of the converged VJP, whatever the steps
    gscale = np.max(np.abs(state["w"].cotangent[PICK]), axis=1)
    for s in (42, 7):
        r = short[s]
        assert np.all(r.info == 1) and np.all(r.valid)
        assert np.all(np.asarray(r.iterations) == 100)
        rho = r.residual / gscale
        assert np.all(rho > 1e-7)      # a genuinely unconverged iterate
        assert np.all(_rel(r.g_target, conv[42].g_target) <= C_BOUND * rho)
        assert np.all(_rel(r.g_rhs, conv[42].g_rhs) <= C_BOUND * rho)
    # hence two step choices differ by at most C (rho_a + rho_b)
    both = (short[42].residual + short[7].residual) / gscale
    assert np.all(_rel(short[7].g_target, short[42].g_target) <= C_BOUND * both)
    assert np.all(_rel(short[7].g_rhs, short[42].g_rhs) <= C_BOUND * both)
