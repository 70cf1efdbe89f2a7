"""The C++20 host API (sdxl-end2end_amd/cpp): Runtime / Tensor / Ops (attention, layer_norm, linear,
E4M3 packing, attention_sublayer) over the C ABI.

Runs the CTest-style executable like the reference runs tests/cuda/cuda_ops_test.cu:
host-only cases here, every case on the GPU box.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "sdxl-end2end_amd", "bin")


def _run(name, *args, timeout=120):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} not built; run __graft_entry__.build()")
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)


def test_host_only_cases():
    r = _run("sdxl_hip_ops_test", "--host-only")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host cases passed" in r.stdout


@pytest.mark.gpu
def test_device_cases():
    r = _run("sdxl_hip_ops_test")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "device cases passed" in r.stdout
    assert "sublayer cases passed" in r.stdout
    assert "out-projection cases passed" in r.stdout  # the level-2 out-projection shape (K-split kernel)
    assert "graph capture cases passed" in r.stdout  # Ops::attention captured in a HIP graph


@pytest.mark.gpu
def test_attention_bench_cli_small_shapes():
    """The reference's ATTENTION_BENCHMARK.bat shape list, with few iterations."""
    for args in (("77", "77", "20", "2", "5"), ("4096", "77", "10", "2", "3"), ("1024", "1024", "20", "2", "3")):
        r = _run("sdxl_hip_attention_bench", *args)
        assert r.returncode == 0, r.stdout + r.stderr
        line = [l for l in r.stdout.splitlines() if l.startswith("flash error")][0]
        max_abs = float(line.split("max_abs=")[1].split()[0])
        assert max_abs < 2e-3, r.stdout
