"""Guards on the compiled device code of this repository's own libraries (CPU only).

Packed FP32 arithmetic (v_pk_add_f32, v_pk_mul_f32, v_pk_fma_f32) is kept out
of the device code: some of its forms have given wrong results on the target
machines without any error.  hipcc -O3 forms these instructions by itself from
plain float code, so the build passes
``-Xclang -target-feature -Xclang -packed-fp32-ops`` (purin_amd/build.py) to
the device compilation (hipcc's host pass warns that it does not know the
feature; the device pass honours it).  These tests disassemble the gfx950
code objects embedded in the built libraries and check that none of the
instructions is present, and check the detection itself on a kernel compiled
with and without the flag.
"""

import os
import re
import struct
import subprocess

import pytest

from purin_amd import build as B

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
PACKED_F32 = re.compile(r"\bv_pk_(?:add|mul|fma)_f32\b")


def _code_objects(path):
    """The gfx950 code objects of a HIP shared library (its .hip_fatbin bundles)."""
    out = path + ".fatbin.tmp"
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={out}", path,
                    os.devnull], check=True, capture_output=True)
    try:
        data = open(out, "rb").read()
    finally:
        os.remove(out)
    objs, start = [], data.find(MAGIC)
    while start >= 0:
        p = start + len(MAGIC)
        (count,) = struct.unpack_from("<Q", data, p)
        p += 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + tlen].decode()
            p += tlen
            if "gfx950" in triple and size:
                objs.append(data[start + off:start + off + size])
        start = data.find(MAGIC, start + 1)
    return objs


def _disassemble(obj, tmp_path, name):
    f = tmp_path / f"{name}.co"
    f.write_bytes(obj)
    res = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", str(f)],
                         check=True, capture_output=True, text=True)
    return res.stdout


def _need_tools():
    for tool in ("llvm-objcopy", "llvm-objdump"):
        if not os.path.exists(f"{LLVM}/{tool}"):
            pytest.skip(f"{tool} not available")


@pytest.mark.parametrize("lib", [B.LIB, B.PROBE_LIB])
def test_built_device_code_has_no_packed_fp32(lib, tmp_path):
    _need_tools()
    if not os.path.exists(lib):
        pytest.skip(f"{os.path.basename(lib)} is not built")
    objs = _code_objects(lib)
    assert objs, "no gfx950 code object found in the library"
    for k, obj in enumerate(objs):
        text = _disassemble(obj, tmp_path, f"o{k}")
        assert "v_" in text  # a real disassembly
        found = sorted(set(PACKED_F32.findall(text)))
        assert not found, f"{os.path.basename(lib)} code object {k}: {found}"


def test_the_guard_detects_packed_fp32_and_the_flag_removes_it(tmp_path):
    """A float2 kernel: without the flag hipcc emits packed FP32 (so the scan
    above would see it); with the build's flags it emits none."""
    _need_tools()
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "pk.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "typedef float F2 __attribute__((ext_vector_type(2)));\n"
        "__global__ void k(const F2* a, const F2* b, F2* c, float s) {\n"
        "  int i = threadIdx.x + blockIdx.x * blockDim.x;\n"
        "  F2 x = a[i], y = b[i];\n"
        "  c[i] = x * y + s * x + y;\n"
        "}\n")
    base = ["-O3", f"--offload-arch={B.ARCH}", "--cuda-device-only", "-S"]
    flags = [f for f in B.FLAGS if f not in ("-shared", "-fPIC")]
    plain = tmp_path / "plain.s"
    guarded = tmp_path / "guarded.s"
    subprocess.run([hipcc, *base, str(src), "-o", str(plain)], check=True, capture_output=True)
    subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", str(src), "-o", str(guarded)],
                   check=True, capture_output=True)
    assert PACKED_F32.search(plain.read_text()), "control: expected packed FP32 without the flag"
    assert not PACKED_F32.search(guarded.read_text())


def _kernel_metadata(obj, tmp_path, name):
    """(kernel name, group_segment_fixed_size) of every kernel in a code object."""
    f = tmp_path / f"{name}.co"
    f.write_bytes(obj)
    notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", str(f)], check=True,
                           capture_output=True, text=True).stdout
    out, lds = [], None
    for line in notes.splitlines():
        m = re.search(r"\.group_segment_fixed_size:\s+(\d+)", line)
        if m:
            lds = int(m.group(1))
        m = re.search(r"\.name:\s+(\S+)", line)
        if m and lds is not None:
            out.append((m.group(1), lds))
            lds = None
    return out


def test_resident_kernels_have_no_static_lds(tmp_path):
    """The resident kernels address LDS by absolute byte offsets held in the
    matrix stream (their dynamic LDS must start at address 0), so no static LDS
    may enter them, including through a library helper such as a workgroup
    reduction."""
    _need_tools()
    if not os.path.exists(f"{LLVM}/llvm-readelf"):
        pytest.skip("llvm-readelf not available")
    if not os.path.exists(B.LIB):
        pytest.skip("libpurin_cp.so is not built")
    seen = 0
    for k, obj in enumerate(_code_objects(B.LIB)):
        for name, lds in _kernel_metadata(obj, tmp_path, f"m{k}"):
            if "k_resident" in name:
                seen += 1
                assert lds == 0, f"{name}: {lds} bytes of static LDS"
    assert seen > 0, "no resident kernel found"


def test_the_static_lds_guard_sees_a_workgroup_reduction(tmp_path):
    """Control: __syncthreads_and brings static LDS into a kernel, and the
    metadata read above reports it."""
    _need_tools()
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not os.path.exists(hipcc) or not os.path.exists(f"{LLVM}/llvm-readelf"):
        pytest.skip("hipcc or llvm-readelf not available")
    src = tmp_path / "red.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k_with_and(const int* a, int* b) {\n"
        "  b[threadIdx.x] = __syncthreads_and(a[threadIdx.x]);\n"
        "}\n"
        "__global__ void k_without(const int* a, int* b) { b[threadIdx.x] = a[threadIdx.x]; }\n")
    lib = tmp_path / "red.so"
    subprocess.run([hipcc, "-O3", "-fPIC", "-shared", f"--offload-arch={B.ARCH}", str(src),
                    "-o", str(lib)], check=True, capture_output=True)
    meta = {}
    for k, obj in enumerate(_code_objects(str(lib))):
        meta.update(dict(_kernel_metadata(obj, tmp_path, f"red{k}")))
    with_and = [v for n, v in meta.items() if "k_with_and" in n]
    without = [v for n, v in meta.items() if "k_without" in n]
    assert with_and and with_and[0] > 0
    assert without and without[0] == 0
