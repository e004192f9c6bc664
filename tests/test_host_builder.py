"""The C++ host side (webyiq_amd/host/webyiq_graph.hpp): Builder, OpDef and
encode, the restatement of the engine's operator layer
(crates/engine/src/graph.rs:117-222, lib.rs:222-228) above the C ABI.

tests/cpp/builder_test.cpp does the checking; these tests run it.
  --cpu  build-time shape and size checks with the engine's messages
         ("missing tensor {name}"), matmul's dispatch by Path, and encode's
         error propagation ("{op}: {wq_last_error()}"), launching nothing
  --gpu  an MLP block (fused norm+quant gate_up in silu mode, quant, down
         accumulated into the residual) and the greedy head (norm_quant,
         lm_head + argmax) built with Builder and replayed by encode on the
         Decode (1 token), Spec (2) and Prefill (128, GEMM, no head) paths,
         every intermediate compared with the CPU oracle: bit for bit, except
         the silu * up output (device expf) and the Prefill GEMM's per-token
         G = 128 output (min term folded on an f16 MFMA), both within rel
         1e-5, the tolerance of the kernels' own parity tests; then embed,
         the chunk merge feeding a per-32 o projection and the MTP input
         stage (graph.rs:439-443, 289-291, 500-504), bit for bit.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
EXE = os.path.join(HERE, "cpp", "builder_test")
LIBS = [os.path.join(ROOT, "webyiq_amd", "libwebyiq_q4q8.so"), os.path.join(ROOT, "webyiq_amd", "libwebyiq_graph.so"),
        os.path.join(ROOT, "oracle", "liboracle_q4q8.so")]


def run(mode, timeout):
    out = subprocess.run([EXE, mode], capture_output=True, text=True, timeout=timeout)
    print(out.stdout, out.stderr, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert f"builder_test {mode[2:]} ok" in out.stdout


@pytest.mark.skipif(shutil.which("make") is None or shutil.which("g++") is None, reason="needs make and g++")
def test_builder_host_checks():
    missing = [p for p in LIBS if not os.path.exists(p)]
    assert not missing, f"build first (python -c 'import __graft_entry__ as g; g.build()'): {missing}"
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)
    run("--cpu", 60)


@pytest.mark.gpu
def test_builder_mlp_and_head_match_oracle():
    assert os.path.exists(EXE), "tests/cpp/builder_test is not built (make -C tests/cpp after the build)"
    run("--gpu", 110)
