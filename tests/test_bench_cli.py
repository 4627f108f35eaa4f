"""bench.py's command-line contract on the CPU: more than one GPU is refused with a message (this
build measures one GPU), and the per-workload option names the configured shapes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_workload_option_lists_the_configured_shapes():
    r = _bench("--help")
    assert r.returncode == 0
    for name in ("c_proj", "turbo", "cfg1", "cfg4_up", "cfg4_down", "oja"):
        assert name in r.stdout
    bad = _bench("--workload", "nope")
    assert bad.returncode != 0 and "invalid choice" in bad.stderr


def test_workload_table_matches_the_configs():
    sys.path.insert(0, ROOT)
    import bench

    shapes = {k: v[1:5] for k, v in bench.WORKLOADS.items()}
    assert shapes["cfg1"] == (4096, 768, 3072, 8)
    assert shapes["c_proj"] == (8192, 4096, 1024, 8)
    assert shapes["turbo"] == (8192, 1280, 5120, 8)
    assert shapes["cfg4_up"] == (32768, 2048, 8192, 16) and shapes["cfg4_down"] == (32768, 8192, 2048, 16)
    assert bench.WORKLOADS["turbo"][5] == 0.0 and bench.WORKLOADS["cfg1"][7]["dtype"] == "fp32"
