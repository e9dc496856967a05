"""CPU: the block-granular pool's host bookkeeping (csrc/block_allocator.cpp).

Builds tests/cpp/test_block_allocator.cpp with g++ under the address and
undefined-behaviour sanitizers and runs it; the program checks the
allocator's contract and, over random operation sequences, the invariants of
the reference's slot-allocator property tests (tests/test_kv_cache.cpp:
298-440) restated for blocks."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tiny-llm_amd", "csrc")
TESTS = [
    "fresh_pool_is_empty", "ensure_maps_in_order_and_records_updates", "ensure_is_all_or_nothing",
    "release_returns_blocks_and_resets_entries", "updates_coalesce_to_the_final_value",
    "shortfall_counts_missing_blocks", "invalid_geometry_throws",
    "random_operations_keep_invariants",
]


@pytest.fixture(scope="module")
def program(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path_factory.mktemp("blocks") / "test_block_allocator")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-I", CSRC,
           os.path.join(ROOT, "tests", "cpp", "test_block_allocator.cpp"),
           os.path.join(CSRC, "block_allocator.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def test_block_allocator_host_suite(program):
    r = subprocess.run([program], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert [ln.split()[1] for ln in r.stdout.splitlines() if ln.startswith("ok ")] == TESTS
