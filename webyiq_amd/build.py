"""Build libwebyiq_q4q8.so (gfx950) in-tree with hipcc.

  python -m webyiq_amd.build          # compile every kernel + the C ABI

Each .hip translation unit is compiled in parallel into webyiq_amd/_build/,
then linked into webyiq_amd/libwebyiq_q4q8.so next to this file; the C++ host
side (host/webyiq_graph.cpp, g++) follows as libwebyiq_graph.so.  Flags:
  --offload-arch=gfx950 only (no other targets, no CUDA/HIP dual paths);
  -Xclang -target-feature -Xclang -packed-fp32-ops: the device pass emits
  no packed fp32 ops (v_pk_fma/mul/add_f32); the host pass does not know
  the feature and prints "'-packed-fp32-ops' is not a recognized feature for
  this target (ignoring feature)", which is filtered from the log (that
  line only).  tests/test_build_flags.py checks both halves: the flag takes
  a packed fma out of a probe kernel's device code, and the built
  library's device code holds no packed fp32 op;
  -mllvm -amdgpu-mfma-vgpr-form: MFMA results in ordinary VGPRs, which the
  VALU epilogues read directly (accumulation registers would need a copy
  instruction per element);
  no fast-math: divisions and the fp32 epilogues keep IEEE semantics that
  the CPU oracle reproduces bit for bit.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libwebyiq_q4q8.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HOST_LIB = os.path.join(HERE, "libwebyiq_graph.so")
# timing build: the same library with the GEMV's per-workgroup stamps (-DWQ_TIMELINE)
TIMELINE_LIB = os.path.join(HERE, "libwebyiq_q4q8_timeline.so")
TIMELINE_SOURCE = "gemv_q4q8.hip"
CXX = os.environ.get("CXX", "g++")

SOURCES = ["capi.hip", "quant_act.hip", "gemv_q4q8.hip", "gemv_mfma.hip", "gemm_q4q8.hip", "argmax.hip", "embed.hip",
           "attn_combine.hip"]
CFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
# Per-source flags: kernel-argument preloading.  The leading arguments of the
# GEMV (nine, 14 SGPRs), the MFMA GEMV of 3..8 tokens (eight, 13 SGPRs), the
# activation quantisers (four, 6 SGPRs) and the chunk merge (five, 7 SGPRs)
# are what their first global loads need; preloaded, they arrive in SGPRs
# with the wave, so no scalar load of the argument segment precedes the
# first load.  (Kernels whose first argument is a parameter struct preload
# nothing.)
SOURCE_FLAGS = {"gemv_q4q8.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
                "gemv_mfma.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
                "quant_act.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=4"],
                "attn_combine.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=5"]}
# what the host pass prints for the device-only feature above (harmless)
HOST_PASS_NOTE = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [HIPCC, *CFLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    tl_obj = os.path.join(BUILD, "gemv_q4q8_timeline.o")
    cmd = [HIPCC, *CFLAGS, *SOURCE_FLAGS.get(TIMELINE_SOURCE, []), "-DWQ_TIMELINE", "-c",
           os.path.join(CSRC, TIMELINE_SOURCE), "-o", tl_obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    procs.append((TIMELINE_SOURCE + " (timeline)", subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines()
                         if l.strip() != HOST_PASS_NOTE)
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        for src, text in failed:
            print(f"--- {src} failed ---\n{text}", file=sys.stderr)
        raise RuntimeError("hipcc failed for " + ", ".join(s for s, _ in failed))
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], check=True)
    os.replace(tmp, LIB)
    tl_objs = [tl_obj if os.path.basename(o) == TIMELINE_SOURCE.replace(".hip", ".o") else o for o in objs]
    tmp = TIMELINE_LIB + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *tl_objs, "-o", tmp], check=True)
    os.replace(tmp, TIMELINE_LIB)
    build_host(verbose)
    return LIB


def build_host(verbose=False):
    """The C++ host side (host/webyiq_graph.cpp): plain C++17 over the C ABI,
    linked against libwebyiq_q4q8.so next to it."""
    tmp = HOST_LIB + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", os.path.join(HERE, "host", "webyiq_graph.cpp"),
           "-o", tmp, "-L" + HERE, "-lwebyiq_q4q8", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
