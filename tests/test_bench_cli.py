"""CPU checks of bench.py's command line (no GPU needed): a multi-GPU request
is refused with a message before any device work, and the workload names
the profiles use exist."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, env=env, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode != 0
    assert "no multi-GPU path" in r.stderr
    assert r.stdout.strip() == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2", RANK="0", LOCAL_RANK="0")
    r = _bench("--gpus", "1", env=env)
    assert r.returncode != 0
    assert "no multi-GPU path" in r.stderr


def test_workload_names():
    sys.path.insert(0, ROOT)
    import bench
    names = set(bench.ALL + bench.EXTRA)
    assert "gemm_bf16_8192" == bench.ALL[0]   # the headline `value`
    for n in bench.WORKLOAD_KERNEL:
        assert n in names, n
