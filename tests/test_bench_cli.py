"""bench.py's command-line contract on the CPU: one GPU only (this build has no
multi-GPU path), and the committed HBM-traffic figure that its roofline object
reports."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py")] + args, cwd=REPO,
                          env=e, capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None),
                                      (["--gpus", "1"], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_exits_with_a_message(args, env):
    r = _run(args, env)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU only" in r.stderr
    assert r.stdout == ""      # no JSON line


def test_traffic_figure_comes_from_the_committed_profile():
    sys.path.insert(0, REPO)
    import bench
    t = bench.traffic_from_profiles()
    assert isinstance(t, int)
    # the dominant launch's algorithmic bytes: 2 x (N*K/2 + 4*N*K/64) + 2*K + 2*N
    N, K = 8192, 3072
    alg = 2 * (N * K // 2 + 4 * N * K // 64) + 2 * K + 2 * N
    assert alg == 28334080
    assert 1.0 <= t / alg < 1.05
