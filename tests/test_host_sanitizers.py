"""CPU: the decode launch planner (tiny-llm_amd/csrc/attn_plan.cpp) and the
oracle (oracle/kv_oracle.c) built with g++/gcc under the address and
undefined-behaviour sanitizers and driven by tests/cpp/test_host_sanitized.cpp
(random and extreme plans; every oracle entry point on small inputs).  Any
sanitizer report fails the run."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tiny-llm_amd", "csrc")
ORACLE = os.path.join(ROOT, "oracle")
CHECKS = ["planner_random", "oracle_kv_and_attention", "oracle_prefill_softmax_weights",
          "oracle_w8a16_and_fp16"]


@pytest.fixture(scope="module")
def program(tmp_path_factory):
    gxx, gcc = shutil.which("g++"), shutil.which("gcc")
    if gxx is None or gcc is None:
        pytest.skip("g++/gcc not found")
    d = tmp_path_factory.mktemp("san")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-g", "-O1"]
    obj = str(d / "kv_oracle.o")
    subprocess.run([gcc, "-std=c11", "-fopenmp", "-ffp-contract=off", "-Wall", "-Wextra", *san,
                    "-c", os.path.join(ORACLE, "kv_oracle.c"), "-o", obj],
                   check=True, capture_output=True, text=True)
    exe = str(d / "test_host_sanitized")
    subprocess.run([gxx, "-std=c++17", "-Wall", "-Wextra", "-Werror", *san, "-I", CSRC,
                    "-I", ORACLE, os.path.join(ROOT, "tests", "cpp", "test_host_sanitized.cpp"),
                    os.path.join(CSRC, "attn_plan.cpp"), obj, "-fopenmp", "-lm", "-o", exe],
                   check=True, capture_output=True, text=True)
    return exe


def test_planner_and_oracle_under_sanitizers(program):
    env = dict(os.environ, OMP_NUM_THREADS="2", ASAN_OPTIONS="detect_leaks=1")
    r = subprocess.run([program], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert [ln.split()[1] for ln in r.stdout.splitlines() if ln.startswith("ok ")] == CHECKS
