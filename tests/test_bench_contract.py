"""bench.py's refusal of more than one GPU, on the CPU: the build measures one
GPU's share, so `--gpus N` with N > 1 (or a multi-rank launch) must exit with a
message before any GPU work, not print a line for a configuration it did not
run."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, env=env,
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None),
                                      ([], {"WORLD_SIZE": "2"})],
                         ids=["gpus2", "gpus8", "world_size2"])
def test_bench_refuses_more_than_one_gpu(args, env):
    r = _run(args, env)
    assert r.returncode == 2, (r.returncode, r.stdout[-500:], r.stderr[-500:])
    assert "one GPU only" in r.stderr
    assert '"metric"' not in r.stdout  # no result line for a run that did not happen
