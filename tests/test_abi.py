"""The C-ABI library loads and exports every function ``include/purin_cp.h`` declares.

CPU-only: no compute call is made (there may be no GPU here).
"""

import ctypes
import os
import re

from purin_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "purin_cp.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(purin_cp_\w+)\s*\(", text)))


def test_header_declares_the_binding_symbols():
    assert set(declared_functions()) == set(_lib.SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_functions() if not hasattr(lib, s)]
    assert not missing, missing


def test_defaults_match_reference_configs():
    """Defaults of ChambollePockConfig / LinearSolverConfig / ImplicitGradientConfig
    (reference src/purin/solvers/chambolle_pock/config.py:34-48, solvers/config.py:13-16, 94)."""
    o = _lib.default_options()
    assert (o.accelerated, o.row_scaling, o.norm_bound, o.norm_iterations, o.norm_seed,
            o.diagonal_preconditioning) == (0, 1, 1, 20, 42, 0)
    assert o.safety == 0.95
    s = _lib.default_solve_options()
    assert (s.tolerance, s.max_iterations, s.early_stop) == (1e-9, 10000, 1)
    a = _lib.default_adjoint_options()
    assert (a.tolerance, a.atol, a.restart, a.max_iterations, a.adjoint_tolerance) == (
        1e-9, 0.0, 30, 100, 1e-8)


def test_build_info_names_gfx950():
    assert b"gfx950" in _lib.load().purin_cp_build_info()


def test_invalid_plan_arguments_are_rejected_without_a_gpu():
    lib = _lib.load()
    handle = ctypes.c_void_p()
    indptr = (ctypes.c_int64 * 2)(0, 1)
    indices = (ctypes.c_int32 * 1)(5)   # column out of range for n = 2
    values = (ctypes.c_double * 1)(1.0)
    rc = lib.purin_cp_plan_create(ctypes.byref(handle), _lib.F64, 2, 1, 0, indptr, indices,
                                  values, None)
    assert rc == _lib.ERR_ARG
    assert b"out of range" in lib.purin_cp_last_error()
    rc = lib.purin_cp_plan_create(ctypes.byref(handle), 7, 2, 1, 0, indptr, indices, values, None)
    assert rc == _lib.ERR_ARG


def test_struct_layouts_match_the_header(tmp_path):
    """Every ctypes mirror of a header struct has the C compiler's size and
    field offsets (the binding passes these structs by pointer)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        import pytest

        pytest.skip("no C compiler")
    structs = {
        "purin_cp_options": _lib.Options,
        "purin_cp_plan_info": _lib.PlanInfo,
        "purin_cp_solve_options": _lib.SolveOptions,
        "purin_cp_timing": _lib.Timing,
        "purin_cp_adjoint_stats": _lib.AdjointStats,
        "purin_cp_adjoint_options": _lib.AdjointOptions,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "purin_cp.h"',
             "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        cname, what, value = line.split()
        got[(cname, what)] = int(value)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


def test_entry_codes_match_the_header():
    text = open(os.path.join(ROOT, "include", "purin_cp.h")).read()
    codes = {m.group(1).lower(): int(m.group(2))
             for m in re.finditer(r"PURIN_CP_ENTRY_(\w+)\s*=\s*(\d+)", text)}
    assert codes == _lib.ENTRY
