"""bench.py's command-line contract, without a GPU: more than one GPU is
refused with a message before anything touches the device, and the five
workload presets name the benchmark configurations."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_workload_presets():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    w = bench.WORKLOADS
    assert sorted(bench.CPU_SAMPLE) == sorted(w)
    assert sorted(w) == [1, 2, 3, 4, 5]
    assert w[4] == ("qwen3-8b-q4km", 512, 512, False)  # the headline configuration
    assert w[5] == ("qwen3-32b-q4km", 4096, 256, True)  # sampled decode
    assert w[2][0] == "qwen3-0.6b-q8_0" and w[2][1] + w[2][2] == 176  # KV up to 176 positions
    import rlh
    for name, _, _, _ in w.values():
        assert name in rlh.SPECS
