"""Build ``libpurin_cp.so`` (HIP, gfx950) in-tree with hipcc.

The library is the product: the C ABI of ``include/purin_cp.h``.  It is built
here, into ``purin_amd/``, so that the built ``.so`` travels with the source
tree to the GPU machine.  ``libpurin_probe.so`` (``include/purin_probe.h``)
holds the ceiling probes that ``bench.py`` times beside the resident kernel.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpurin_cp.so")
SOURCES = ["plan.hip", "forward.hip", "adjoint.hip"]
PROBE_LIB = os.path.join(HERE, "libpurin_probe.so")
PROBE_SOURCES = ["probe.hip"]
ARCH = os.environ.get("PURIN_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    # no packed-fp32 (v_pk_*_f32) instructions in the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources(names=SOURCES):
    return [os.path.join(CSRC, s) for s in names if os.path.exists(os.path.join(CSRC, s))]


def _hipcc(srcs, out, verbose):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = out + ".tmp"
    cmd = [hipcc, *FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed building {os.path.basename(out)}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    _hipcc(sources(), LIB, verbose)
    _hipcc(sources(PROBE_SOURCES), PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
