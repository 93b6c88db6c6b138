"""Build ``libpurin_cp.so`` (HIP, gfx950) in-tree with hipcc.

The library is the product: the C ABI of ``include/purin_cp.h``.  It is built
here, into ``purin_amd/``, so that the built ``.so`` travels with the source
tree to the GPU machine.  ``libpurin_probe.so`` (``include/purin_probe.h``)
holds the ceiling probes that ``bench.py`` times beside the resident kernel.

Each source compiles to its own object (in parallel, under ``_build/``), and
the objects link into the shared library; every call recompiles.
``resident_launch.hip`` compiles once per (element type, row-slot count) pair
(``RESIDENT_VARIANTS``), so the resident kernel's variants build in parallel.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(os.path.dirname(HERE), "_build")
LIB = os.path.join(HERE, "libpurin_cp.so")
SOURCES = ["plan.hip", "forward.hip", "adjoint.hip"]
RESIDENT_SOURCE = "resident_launch.hip"
RESIDENT_VARIANTS = [(f64, slr) for f64 in (1, 0) for slr in (1, 2, 3, 4)]
PROBE_LIB = os.path.join(HERE, "libpurin_probe.so")
PROBE_SOURCES = ["probe.hip"]
ARCH = os.environ.get("PURIN_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # no packed-fp32 (v_pk_*_f32) instructions in the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources(names=SOURCES):
    return [os.path.join(CSRC, s) for s in names if os.path.exists(os.path.join(CSRC, s))]


def _hipcc():
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed building {what}")


def _compile(job, verbose):
    src, defines, tag = job
    os.makedirs(OBJ, exist_ok=True)
    obj = os.path.join(OBJ, os.path.basename(src) + tag + ".o")
    tmp = obj + ".tmp"
    _run([_hipcc(), *FLAGS, *defines, "-c", src, "-o", tmp], os.path.basename(obj), verbose)
    os.replace(tmp, obj)
    return obj


def _jobs():
    """(source, defines, object tag) of the library's objects."""
    jobs = [(s, [], "") for s in sources()]
    res = os.path.join(CSRC, RESIDENT_SOURCE)
    for f64, slr in RESIDENT_VARIANTS:
        jobs.append((res, [f"-DPURIN_RES_F64={f64}", f"-DPURIN_RES_SLR={slr}"],
                     f".{'f64' if f64 else 'f32'}_r{slr}"))
    return jobs


def _link(objs, out, verbose):
    tmp = out + ".tmp"
    _run([_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp],
         os.path.basename(out), verbose)
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    lib_jobs = _jobs()
    probe_jobs = [(s, [], "") for s in sources(PROBE_SOURCES)]
    # the slowest objects first (the resident variants, then forward.hip)
    jobs = lib_jobs[len(SOURCES):] + lib_jobs[:len(SOURCES)][::-1] + probe_jobs
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(workers) as pool:
        objs = dict(zip([id(j) for j in jobs], pool.map(lambda j: _compile(j, verbose), jobs)))
    _link([objs[id(j)] for j in lib_jobs], LIB, verbose)
    _link([objs[id(j)] for j in probe_jobs], PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
