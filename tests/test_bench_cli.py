"""CPU tests of bench.py's command-line contract: more than one GPU is refused with a
message (this build runs on one GPU), before anything touches a GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_multi_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert p.returncode == 2
    assert "one GPU" in p.stderr and "--gpus 2" in p.stderr


def test_world_size_env_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=300,
                       cwd=ROOT, env=env)
    assert p.returncode == 2
