"""GPU: the C++ drop-in (tests/cpp/test_dropin_decode.cpp, built by
__graft_entry__.build() with hipcc in the drop-in's include order): the
decode branch of TransformerLayer::attention (src/transformer.cpp:222-237)
restated against tiny_llm::KVCacheManager and kernels::attention_decode,
its error paths through fmt-style TLLM_ERROR calls of the caller's logger,
and the batched DecodeBatch replacement -- each against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "test_dropin_decode")
LIB = os.path.join(ROOT, "tiny-llm_amd", "_build", "libtinyllm_kv.so")


def test_cpp_dropin_decode_branch():
    assert os.path.exists(EXE), "run __graft_entry__.build() first"
    print("step: C++ drop-in", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    lib = [ln.split(None, 1)[1] for ln in lines if ln.startswith("library ")]
    assert lib and os.path.realpath(lib[0]) == os.path.realpath(LIB), lib
    assert [ln.split()[1] for ln in lines if ln.startswith("ok ")] == [
        "reference_decode_branch", "caller_logger_fmt", "batched_gqa_decode"]
    # the caller's logger printed the fmt-formatted errors
    assert "forward: invalid seq_id 999 for layer 0" in r.stderr
    assert "forward: invalid position 165 for layer 0, max_seq_len=160" in r.stderr
