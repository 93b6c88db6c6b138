"""The HIP path against the committed config1 fixture (tests/golden/config1.npz).

Fixed iterations (the configuration as stated: fixed-step CP, 1000 iterations):
fp64 y / multipliers / slacks within 1e-10 relative, fp32 within 1e-4; statuses,
iteration counts and active-set masks identical.  To convergence (tolerance 1e-9):
y within 1e-8 and the VJP w.r.t. target and rhs within 1e-8 (the adjoint is only
defined to the GMRES tolerance, 1e-9 relative residual).
"""

import numpy as np
import pytest

from tests import _golden
from tests._gpu import rel_err, require_gpu, to_np

pytestmark = pytest.mark.gpu


def plan(g, dtype):
    from purin_amd.plan import Plan

    return Plan(g["target"].shape[1], int(g["me"]), int(g["mi"]), g["indptr"], g["indices"],
                g["data"], dtype=dtype, device="cuda")


@pytest.mark.parametrize("tag,dtype,bar", [("f64", np.float64, 1e-10), ("f32", np.float32, 1e-4)])
@pytest.mark.parametrize("streaming", [False, True])
def test_fixed_iterations_match_fixture(tag, dtype, bar, streaming):
    require_gpu()
    g = _golden.load()
    p = plan(g, dtype)
    rhs = np.tile(g["rhs"], (32, 1)).astype(dtype)
    out = p.project(g["target"].astype(dtype), rhs, max_iterations=1000, early_stop=False,
                    streaming=streaming)
    y, mult, slacks = to_np(out.y), to_np(out.multipliers), to_np(out.slacks)
    assert rel_err(y, g[f"{tag}_y"]) <= bar
    assert rel_err(mult, g[f"{tag}_multipliers"]) <= bar
    assert rel_err(slacks, g[f"{tag}_slacks"]) <= bar
    np.testing.assert_array_equal(to_np(out.status), g[f"{tag}_status"])
    np.testing.assert_array_equal(to_np(out.iterations), g[f"{tag}_iterations"])
    mi_general = int(g["mi"]) - 128
    me = int(g["me"])
    for got, want in zip(_golden.masks(y, mult, me, mi_general),
                         _golden.masks(g[f"{tag}_y"], g[f"{tag}_multipliers"], me, mi_general)):
        np.testing.assert_array_equal(got, want)


def test_converged_projection_and_vjp_match_fixture():
    require_gpu()
    g = _golden.load()
    p = plan(g, np.float64)
    rhs = np.tile(g["rhs"], (32, 1))
    out = p.project(g["target"], rhs, max_iterations=10000, tolerance=1e-9, save=True)
    np.testing.assert_array_equal(to_np(out.status), g["conv_status"])
    np.testing.assert_array_equal(to_np(out.eligible), g["conv_eligible"])
    assert rel_err(to_np(out.y), g["conv_y"]) <= 1e-8
    adj = p.adjoint(out.saved, g["target"], rhs, g["cot"])
    np.testing.assert_array_equal(to_np(adj.valid), g["conv_valid"])
    assert rel_err(to_np(adj.g_target), g["conv_g_target"]) <= 1e-8
    assert rel_err(to_np(adj.g_rhs), g["conv_g_rhs"]) <= 1e-8
