"""Count and iterate comparisons for early-stop parity tests (GPU vs oracle).

A sample's stop iteration is the first at which its stop-test margin
``max(residual, gap, stationarity) / tolerance`` (reference
src/purin/solvers/chambolle_pock/kernels.py:260-278) falls to 1 or below.  In
fp64 the GPU must stop every sample at the oracle's iteration.  In fp32 the
margin carries rounding error of its own, and the GPU sums in other orders
than the oracle, so a stop iteration is fixed by the recurrence only where
the margin crosses 1 cleanly.  The rule below measures that on the oracle
itself: it reruns the oracle with its steps changed by 1e-6 relative (safety
scaled by 1 +- 1e-6) and

* accepts a different count for a sample only where, at the earlier of the
  two stop iterations k, the oracle's margin lies within max(1e-4, 2 s) of 1,
  with s the largest change of that sample's margin over iterations
  k-2..k+2 under the perturbation (a borderline stop);
* allows at most 1 in 10 differing counts among samples whose stop iteration
  the perturbation leaves unchanged (stable samples), and no such limit among
  samples whose own stop iteration the 1e-6 perturbation moves (accelerated
  fp32 runs move some by tens to hundreds of iterations);
* holds the iterates of same-count samples to the parity bar, and of the
  others to max(10 bar, 2 d), with d the sample's distance (relative to the
  batch's largest entry) between the oracle and its perturbed runs.

A caller may add further perturbed runs (``alternates``): the same problem
solved another way, e.g. the oracle in fp64 on the fp32 inputs, whose margins
then measure the fp32 rounding noise of the margin itself (the objective sums
behind the gap carry rounding error of their own, which a change of the steps
does not show).  The perturbed runs are computed only when some count differs.
"""

from __future__ import annotations

import numpy as np


class Margins:
    """The oracle's result and stop margins, with its 1e-6-perturbed reruns on demand.

    ``solve(safety, trace)`` runs the oracle at the given safety factor,
    appending each iteration's (B,) margins to ``trace``, and returns its
    result (with ``.iterations`` and ``.y``).  ``alternates``: further
    callables ``alt(trace)`` solving the same problem another way (results
    and traces as ``solve``'s), counted among the perturbed runs.
    """

    def __init__(self, solve, dtype, safety=0.95, alternates=()):
        self._solve = solve
        self.dtype = np.dtype(dtype)
        self.safety = safety
        self._alternates = tuple(alternates)
        trace = []
        self.want = solve(safety, trace)
        self.trace = np.asarray(trace, np.float64)
        self._others = None

    @property
    def others(self):
        """[(result, trace)] of the runs with safety * (1 + 1e-6) and * (1 - 1e-6),
        then of the alternates."""
        if self._others is None:
            self._others = []
            for f in (1 + 1e-6, 1 - 1e-6):
                tr = []
                res = self._solve(self.safety * f, tr)
                self._others.append((res, np.asarray(tr, np.float64)))
            for alt in self._alternates:
                tr = []
                res = alt(tr)
                self._others.append((res, np.asarray(tr, np.float64)))
        return self._others


def check_counts(got, m: Margins, samples=None):
    """Per-sample iteration counts of the GPU (``got``) against the oracle's
    (``m.want.iterations``, restricted to ``samples`` of the GPU batch when the
    oracle ran on those only).  Returns the boolean mask of same-count samples."""
    want = np.asarray(m.want.iterations)
    got = np.asarray(got)
    if samples is not None:
        got = got[samples]
    diff = np.flatnonzero(got != want)
    msg = (f"{diff.size} samples differ: {diff.tolist()[:8]} got {got[diff][:8].tolist()} "
           f"want {want[diff][:8].tolist()}")
    if m.dtype == np.float64 or diff.size == 0:
        assert diff.size == 0, msg
        return got == want
    others = m.others
    unstable = np.zeros(want.shape, bool)
    for res, _ in others:
        unstable |= np.asarray(res.iterations) != want
    stable_diff = [b for b in diff if not unstable[b]]
    assert len(stable_diff) * 10 <= got.size, f"{msg}; stable samples differing: {stable_diff}"
    for b in diff:
        k = min(got[b], want[b]) - 1
        sens = 0.0
        for _, tr in others:
            lo, hi = max(k - 2, 0), min(k + 3, len(m.trace), len(tr))
            if hi > lo:
                sens = max(sens, float(np.max(np.abs(tr[lo:hi, b] - m.trace[lo:hi, b]))))
        assert abs(m.trace[k, b] - 1) <= max(1e-4, 2 * sens), (
            f"{msg}; sample {b} margin {m.trace[k, b]!r} sensitivity {sens!r}")
    return got == want


def check_iterates(got_y, m: Margins, same, bar, samples=None):
    """Iterates: same-count samples at ``bar``; the others at max(10 bar, 2 d)."""
    got_y = np.asarray(got_y, np.float64)
    if samples is not None:
        got_y = got_y[samples]
    want = np.asarray(m.want.y, np.float64)
    scale = max(float(np.max(np.abs(want))), 1e-300)
    err = np.max(np.abs(got_y - want), axis=1) / scale
    if np.any(same):
        assert np.max(err[same]) <= bar, (err[same].max(), bar)
    if np.all(same):
        return
    spread = np.zeros(want.shape[0])
    for res, _ in m.others:
        spread = np.maximum(spread, np.max(np.abs(np.asarray(res.y, np.float64) - want),
                                           axis=1) / scale)
    lim = np.maximum(10 * bar, 2 * spread)
    bad = ~same & (err > lim)
    assert not np.any(bad), (np.flatnonzero(bad), err[bad], lim[bad])
