"""ctypes binding of ``libpurin_cp.so`` (the C ABI in ``include/purin_cp.h``).

The library is required: importing this module raises if it has not been
built (``python -m purin_amd.build`` or ``__graft_entry__.build()``).  There is
no CPU fallback.
"""

from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpurin_cp.so")

F32, F64 = 0, 1
NOALLOC_SCRATCH_BYTES = 128 << 20  # PURIN_CP_NOALLOC_SCRATCH_BYTES
OK, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED, ERR_NOMEM = 0, 1, 2, 3, 4
# purin_cp_entry (purin_cp_workspace_bytes)
ENTRY = dict(spmm=0, solve=1, project=2, project_values=3, qp_solve=4, dense_solve=5,
             adjoint=6, adjoint_values=7, qp_adjoint=8, dense_adjoint=9)

# every symbol the header declares (checked by tests/test_abi.py)
SYMBOLS = (
    "purin_cp_default_options",
    "purin_cp_plan_create",
    "purin_cp_plan_destroy",
    "purin_cp_plan_get_info",
    "purin_cp_plan_kept_rows",
    "purin_cp_plan_set_metric",
    "purin_cp_spmm",
    "purin_cp_default_solve_options",
    "purin_cp_saved_bytes",
    "purin_cp_workspace_bytes",
    "purin_cp_last_timing",
    "purin_cp_last_adjoint_stats",
    "purin_cp_last_adjoint_iterations",
    "purin_cp_solve",
    "purin_cp_project",
    "purin_cp_project_noalloc",
    "purin_cp_project_values",
    "purin_cp_qp_solve",
    "purin_cp_dense_solve",
    "purin_cp_default_adjoint_options",
    "purin_cp_adjoint",
    "purin_cp_adjoint_values",
    "purin_cp_qp_adjoint",
    "purin_cp_dense_adjoint",
    "purin_cp_last_error",
    "purin_cp_build_info",
)


class Options(C.Structure):
    _fields_ = [
        ("accelerated", C.c_int32),
        ("row_scaling", C.c_int32),
        ("norm_bound", C.c_int32),
        ("norm_iterations", C.c_int32),
        ("norm_seed", C.c_int32),
        ("diagonal_preconditioning", C.c_int32),
        ("safety", C.c_double),
        ("bound_presolve", C.c_int32),
        ("reserved", C.c_int32),
    ]


class PlanInfo(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("n", C.c_int64), ("me", C.c_int64), ("mi", C.c_int64),
        ("kept_rows", C.c_int64), ("bound_rows", C.c_int64), ("nnz_kept", C.c_int64),
        ("norm", C.c_double), ("tau0", C.c_double), ("sigma0", C.c_double),
        ("adjoint_norm", C.c_double), ("adjoint_tau", C.c_double), ("adjoint_sigma", C.c_double),
        ("tolerance_factor", C.c_double),
        ("resident_stream_bytes", C.c_int64), ("resident_stream_bytes_early", C.c_int64),
        ("resident_row_slots", C.c_int64), ("resident_col_slots", C.c_int64),
        ("workspace_bytes", C.c_int64), ("adjoint_workspace_bytes", C.c_int64),
        ("resident_tile_samples", C.c_int64),
    ]


class SolveOptions(C.Structure):
    _fields_ = [
        ("tolerance", C.c_double),
        ("max_iterations", C.c_int64),
        ("early_stop", C.c_int32),
        ("check_every", C.c_int32),
        ("shared_bounds", C.c_int32),
        ("timing", C.c_int32),
        ("streaming", C.c_int32),
        ("reserved", C.c_int32),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_int64),
    ]


class Timing(C.Structure):
    _fields_ = [
        ("iterations", C.c_int64),
        ("row_ms", C.c_double),
        ("col_ms", C.c_double),
        ("diag_ms", C.c_double),
        ("loop_ms", C.c_double),
        ("resident", C.c_int32),
        ("linear_kybar", C.c_int32),
        ("narrow_columns", C.c_int32),
    ]


class AdjointStats(C.Structure):
    _fields_ = [("arnoldi_steps", C.c_int64), ("cycles", C.c_int32), ("reserved", C.c_int32)]


class AdjointOptions(C.Structure):
    _fields_ = [
        ("tolerance", C.c_double),
        ("atol", C.c_double),
        ("restart", C.c_int32),
        ("max_iterations", C.c_int32),
        ("adjoint_tolerance", C.c_double),
        ("force_eligible", C.c_int32),
        ("reserved", C.c_int32),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_int64),
        ("arnoldi_iterations", C.POINTER(C.c_int32)),
    ]


class PurinError(RuntimeError):
    """Error code and message returned by the HIP library."""

    def __init__(self, code, message):
        super().__init__(f"purin_cp error {code}: {message}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH):
    """Load the library (once) and declare argument types."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the HIP library first (python -m purin_amd.build)")
    lib = C.CDLL(path)
    vp, i64, i32, dbl = C.c_void_p, C.c_int64, C.c_int32, C.c_double
    u8p, i32p = C.POINTER(C.c_uint8), C.POINTER(C.c_int32)
    lib.purin_cp_default_options.argtypes = [C.POINTER(Options)]
    lib.purin_cp_default_options.restype = None
    lib.purin_cp_plan_create.argtypes = [C.POINTER(vp), i32, i64, i64, i64, C.POINTER(C.c_int64),
                                         C.POINTER(C.c_int32), C.POINTER(C.c_double),
                                         C.POINTER(Options)]
    lib.purin_cp_plan_create.restype = C.c_int
    lib.purin_cp_plan_destroy.argtypes = [vp]
    lib.purin_cp_plan_destroy.restype = None
    lib.purin_cp_plan_get_info.argtypes = [vp, C.POINTER(PlanInfo)]
    lib.purin_cp_plan_get_info.restype = C.c_int
    lib.purin_cp_plan_kept_rows.argtypes = [vp, C.POINTER(C.c_int64), C.POINTER(C.c_double)]
    lib.purin_cp_plan_kept_rows.restype = C.c_int
    lib.purin_cp_plan_set_metric.argtypes = [vp, C.POINTER(C.c_double)]
    lib.purin_cp_plan_set_metric.restype = C.c_int
    lib.purin_cp_spmm.argtypes = [vp, vp, i64, i32, i32, vp, vp]
    lib.purin_cp_spmm.restype = C.c_int
    lib.purin_cp_default_solve_options.argtypes = [C.POINTER(SolveOptions)]
    lib.purin_cp_default_solve_options.restype = None
    lib.purin_cp_saved_bytes.argtypes = [vp, i64]
    lib.purin_cp_saved_bytes.restype = C.c_int64
    lib.purin_cp_workspace_bytes.argtypes = [vp, i32, i64, C.POINTER(AdjointOptions)]
    lib.purin_cp_workspace_bytes.restype = C.c_int64
    lib.purin_cp_solve.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp, u8p, C.POINTER(SolveOptions),
                                   vp, vp, i32p, vp, vp, u8p, vp]
    lib.purin_cp_solve.restype = C.c_int
    lib.purin_cp_project.argtypes = [vp, vp, i64, vp, vp, vp, C.POINTER(SolveOptions), vp, vp, vp,
                                     i32p, i32p, vp, u8p, u8p, vp]
    lib.purin_cp_project.restype = C.c_int
    lib.purin_cp_project_noalloc.argtypes = lib.purin_cp_project.argtypes
    lib.purin_cp_project_noalloc.restype = C.c_int
    lib.purin_cp_project_values.argtypes = [vp, vp, i64, vp, vp, vp, vp, C.POINTER(SolveOptions),
                                            vp, vp, vp, i32p, i32p, vp, u8p, u8p, vp]
    lib.purin_cp_project_values.restype = C.c_int
    lib.purin_cp_qp_solve.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp, vp, vp,
                                      C.POINTER(SolveOptions), vp, vp, vp, i32p, i32p, vp, u8p,
                                      u8p, vp]
    lib.purin_cp_qp_solve.restype = C.c_int
    lib.purin_cp_dense_solve.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp, vp, vp,
                                         C.POINTER(SolveOptions), vp, vp, i32p, vp]
    lib.purin_cp_dense_solve.restype = C.c_int
    lib.purin_cp_last_timing.argtypes = [vp, C.POINTER(Timing)]
    lib.purin_cp_last_timing.restype = C.c_int
    lib.purin_cp_last_adjoint_stats.argtypes = [vp, C.POINTER(AdjointStats)]
    lib.purin_cp_last_adjoint_stats.restype = C.c_int
    lib.purin_cp_last_adjoint_iterations.argtypes = [vp, vp, i64, i32p]
    lib.purin_cp_last_adjoint_iterations.restype = C.c_int
    lib.purin_cp_default_adjoint_options.argtypes = [C.POINTER(AdjointOptions)]
    lib.purin_cp_default_adjoint_options.restype = None
    lib.purin_cp_adjoint.argtypes = [vp, vp, i64, vp, vp, vp, vp, C.POINTER(AdjointOptions), vp,
                                     vp, vp, vp, u8p, i32p, vp]
    lib.purin_cp_adjoint.restype = C.c_int
    lib.purin_cp_adjoint_values.argtypes = [vp, vp, i64, vp, vp, vp, C.POINTER(AdjointOptions),
                                            vp, vp, vp, u8p, i32p, vp]
    lib.purin_cp_adjoint_values.restype = C.c_int
    lib.purin_cp_qp_adjoint.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp,
                                        C.POINTER(AdjointOptions), vp, vp, vp, vp, vp, vp, u8p,
                                        i32p, vp]
    lib.purin_cp_qp_adjoint.restype = C.c_int
    lib.purin_cp_dense_adjoint.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp,
                                           C.POINTER(AdjointOptions), vp, vp, vp, vp, vp, vp]
    lib.purin_cp_dense_adjoint.restype = C.c_int
    lib.purin_cp_last_error.argtypes = []
    lib.purin_cp_last_error.restype = C.c_char_p
    lib.purin_cp_build_info.argtypes = []
    lib.purin_cp_build_info.restype = C.c_char_p
    _lib = lib
    return lib


def check(code):
    if code != OK:
        raise PurinError(code, load().purin_cp_last_error().decode())


def default_options():
    o = Options()
    load().purin_cp_default_options(C.byref(o))
    return o


def default_solve_options():
    o = SolveOptions()
    load().purin_cp_default_solve_options(C.byref(o))
    return o


def default_adjoint_options():
    o = AdjointOptions()
    load().purin_cp_default_adjoint_options(C.byref(o))
    return o
