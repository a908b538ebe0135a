"""bench.py's command line: the requests it refuses before touching a GPU (one GPU only, at least
one timed step), with exit status 2 and a message on stderr and nothing on stdout (the driver reads
stdout's last line as the result)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, cwd=ROOT, env=e)


@pytest.mark.parametrize("args,env,needle", [
    (("--gpus", "2"), None, "one GPU only"),
    (("--gpus", "8", "--steps", "5"), None, "one GPU only"),
    ((), {"WORLD_SIZE": "2"}, "one GPU only"),
    (("--steps", "0"), None, "--steps must be >= 1"),
])
def test_refused_requests(args, env, needle):
    r = run_bench(*args, env=env)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert needle in r.stderr
    assert r.stdout == ""
