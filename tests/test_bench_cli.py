"""bench.py's contract that needs no GPU: the build measures one
GPU only, so any --gpus above 1 exits with status 2 and says so, before any
GPU work; a non-zero rank (a launcher's extra processes) prints nothing; and
the profile summaries its JSON line cites are committed."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused_with_a_message():
    for n in ("2", "8"):
        res = _bench("--gpus", n)
        assert res.returncode == 2
        assert "one GPU only" in res.stderr and f"--gpus {n}" in res.stderr
        assert res.stdout == ""


def test_non_zero_rank_prints_nothing():
    env = dict(os.environ, RANK="1")
    res = _bench("--gpus", "1", env=env)
    assert res.returncode == 0
    assert res.stdout == ""


def test_profiles_cited_by_bench_exist():
    """Every profiles/ summary bench.py cites in its JSON line is committed."""
    import re
    text = open(os.path.join(ROOT, "bench.py")).read()
    cited = set(re.findall(r"profiles/[\w.\-]+\.(?:md|json|txt)", text))
    cited |= {"profiles/" + m for m in re.findall(r'"profiles",\s*"([\w.\-]+)"', text)}
    assert cited
    for path in sorted(cited):
        assert os.path.exists(os.path.join(ROOT, path)), path
