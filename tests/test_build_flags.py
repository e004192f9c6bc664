"""Checks of the HIP build's flags on the built library (no GPU needed):
the packed-fp32 guard, no register spills in the production GEMM and the
headline GEMV, and kernel-argument preloading on the decode kernels.

The packed-fp32 guard (webyiq_amd/build.py CFLAGS).

The library is compiled with `-Xclang -target-feature -Xclang
-packed-fp32-ops`.  hipcc's host pass does not know that feature and says
so; the device pass honours it.  These tests check both halves on the CPU:
the flag removes a packed fma from a probe kernel's gfx950 code (so it is
not ignored), and the built library's gfx950 code holds no v_pk_fma_f32,
v_pk_mul_f32 or v_pk_add_f32.
"""
import os
import re
import shutil
import subprocess

import pytest

from webyiq_amd import build as hipbuild

PK = re.compile(r"\bv_pk_(fma|mul|add)_f32\b")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
PROBE = r"""
#include <hip/hip_runtime.h>
__global__ void probe(float2* a, const float2* b, const float2* c, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float2 x = a[i], y = b[i], z = c[i];
        x.x = x.x * y.x + z.x;
        x.y = x.y * y.y + z.y;
        a[i] = x;
    }
}
"""


def device_asm(tmp_path, flags, tag):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / f"probe_{tag}.s"
    subprocess.run([hipbuild.HIPCC, "--offload-arch=gfx950", "-O3", *flags, "--cuda-device-only", "-S",
                    str(src), "-o", str(out)], check=True, capture_output=True)
    return out.read_text()


@pytest.mark.skipif(not os.path.exists(hipbuild.HIPCC), reason="hipcc not installed")
def test_flag_removes_packed_fp32_from_device_code(tmp_path):
    flag = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    assert all(f in hipbuild.CFLAGS for f in flag)
    without = device_asm(tmp_path, [], "default")
    with_flag = device_asm(tmp_path, flag, "flag")
    assert PK.search(without), "probe no longer yields a packed fma without the flag; pick another probe"
    assert not PK.search(with_flag)


@pytest.mark.skipif(not (os.path.exists(hipbuild.LIB) and os.path.exists(OBJDUMP)),
                    reason="library not built or llvm-objdump missing")
def test_library_device_code_has_no_packed_fp32(tmp_path):
    # llvm-objdump --offloading writes the bundles next to its input
    lib = tmp_path / "lib.so"
    shutil.copy(hipbuild.LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", str(lib)], check=True, capture_output=True, cwd=tmp_path)
    objs = sorted(p for p in tmp_path.iterdir() if "amdgcn" in p.name and "gfx950" in p.name)
    assert objs, "no gfx950 code object in the library"
    kernels = 0
    for o in objs:
        asm = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(o)], check=True, capture_output=True,
                             text=True).stdout
        kernels += asm.count(">:\n")
        hits = PK.findall(asm)
        assert not hits, f"{o.name}: packed fp32 ops {sorted(set(hits))}"
    assert kernels > 0


@pytest.mark.skipif(not (os.path.exists(hipbuild.LIB) and os.path.exists(OBJDUMP)),
                    reason="library not built or llvm-objdump missing")
def test_production_gemm_and_headline_gemv_use_no_scratch(tmp_path):
    """Register spills show up as a private segment: none in the GEMM
    instances that serve calls (the group-sum dump instances, a test hook,
    are exempt) nor in the headline decode GEMV."""
    lib = tmp_path / "lib.so"
    shutil.copy(hipbuild.LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", str(lib)], check=True, capture_output=True, cwd=tmp_path)
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    scratch = {}
    for o in sorted(p for p in tmp_path.iterdir() if "amdgcn" in p.name and "gfx950" in p.name):
        notes = subprocess.run([readelf, "--notes", str(o)], check=True, capture_output=True, text=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r"\s+\.name:\s+(\S+)", line)
            if m:
                name = m.group(1)
            m = re.match(r"\s+\.private_segment_fixed_size:\s+(\d+)", line)
            if m and name:
                scratch[name] = int(m.group(1))
    gemm = {k: v for k, v in scratch.items() if "gemm_kernel" in k and k.endswith("ELb0EEEvNS0_10GemmParamsE")}
    assert len(gemm) >= 30
    assert not {k: v for k, v in gemm.items() if v}, "spilling GEMM instances"
    head = [k for k in scratch if "gemv_kernelILi1ELi0ELi128ELb1ELi2ELb0ELb0E" in k]
    assert head and all(scratch[k] == 0 for k in head)


def kernel_bodies(tmp_path):
    """{mangled kernel name: [instruction mnemonics with operands]} of the
    built library's gfx950 code objects."""
    lib = tmp_path / "lib.so"
    shutil.copy(hipbuild.LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", str(lib)], check=True, capture_output=True, cwd=tmp_path)
    bodies, name = {}, None
    for o in sorted(p for p in tmp_path.iterdir() if "amdgcn" in p.name and "gfx950" in p.name):
        asm = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", "--no-show-raw-insn", str(o)], check=True,
                             capture_output=True, text=True).stdout
        for line in asm.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
            if m:
                name = m.group(1)
                bodies[name] = []
            elif name and line.startswith("\t"):
                bodies[name].append(line.split("//")[0].strip())
    return bodies


@pytest.mark.skipif(not (os.path.exists(hipbuild.LIB) and os.path.exists(OBJDUMP)),
                    reason="library not built or llvm-objdump missing")
def test_decode_kernels_issue_their_first_load_without_an_argument_wait(tmp_path):
    """The decode-path kernels take the arguments their first loads need as
    leading arguments preloaded into SGPRs (build.py SOURCE_FLAGS): their
    code starts with the preload's compatibility preamble (scalar loads of
    those arguments, a wait and a branch over padding, run only where the
    firmware does not preload), and after it the first global load comes
    before any wait for a scalar load (one merely issued is no stall)."""
    bodies = kernel_bodies(tmp_path)
    wanted = ["gemv_kernelILi1ELi0ELi128ELb1ELi2ELb0ELb0E",   # the headline GEMV
              "gemv_kernelILi1ELi2ELi128ELb1ELi3ELb0ELb1E",   # fused norm + quant + gate_up
              "quant_split_kernelILb1ELb1ELi128ELi8E",        # norm + quantiser
              "attn_combine_kernelILi2E",                     # chunk merge
              "gemv_mfma_rows_kernelILi8ELi0ELb1E"]           # lm_head at 3..8 tokens
    for w in wanted:
        names = [n for n in bodies if w in n]
        assert names, f"{w}: kernel not found"
        ins = bodies[names[0]]
        br = next(i for i, s in enumerate(ins) if s.startswith("s_branch"))
        assert all(s.startswith(("s_load", "s_waitcnt")) for s in ins[:br]), f"{w}: no preload preamble"
        body = [s for s in ins[br + 1:] if not s.startswith("s_nop")]
        first = next(i for i, s in enumerate(body) if s.startswith("global_load"))
        early = [s for s in body[:first] if "s_waitcnt" in s and "lgkmcnt" in s]
        assert not early, f"{w}: a wait for argument loads before the first global load: {early}"
