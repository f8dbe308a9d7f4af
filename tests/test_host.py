"""Host-side behaviour that needs no GPU: the loader's failure modes and bench.py's one-GPU contract."""
import os
import subprocess
import sys

import pytest

from conftest import ROOT


def test_load_gpuq_fails_loudly_without_a_device(monkeypatch):
    import gpuq
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError):
        gpuq.load_gpuq(0, required=True)
    assert gpuq.load_gpuq(0, required=False, quiet=True) is None


def test_missing_library_is_an_error(monkeypatch, tmp_path):
    import gpuq
    monkeypatch.setenv("GPUQ_DIR", str(tmp_path))
    with pytest.raises(FileNotFoundError):
        gpuq.open_lib()


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
