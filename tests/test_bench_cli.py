"""CPU: bench.py's command line -- the one-GPU refusal of --gpus N > 1 and the
options of the W8A16 and prefill paths (parsing only; no GPU work)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line


def test_parse_paths_and_weight_layouts(monkeypatch):
    sys.path.insert(0, ROOT)
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py", "--path", "project", "--weights", "reference"])
    a = bench.parse()
    assert (a.path, a.weights, a.gpus, a.config) == ("project", "reference", 1, 3)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--path", "prefill", "--prefill-seqs", "16",
                                      "--prefill-tokens", "512"])
    a = bench.parse()
    assert (a.path, a.prefill_seqs, a.prefill_tokens, a.weights) == ("prefill", 16, 512, "packed")
    monkeypatch.setattr(sys, "argv", ["bench.py", "--weights", "int4"])
    with pytest.raises(SystemExit):
        bench.parse()
