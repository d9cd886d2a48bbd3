"""bench.py's command-line contract on the host: more than one GPU is refused
with a message, and config a (the reference's CPU plumbing case) runs without
a GPU and prints one JSON line with its figures."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run(*args, timeout=300):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run("--gpus", "2", timeout=120)
    assert "one GPU" in (r.stdout + r.stderr)
    assert not r.stdout.strip().startswith("{")  # no result line


def test_config_a_runs_on_the_host_and_prints_one_json_line():
    r = run("--config", "a")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.strip().startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    a = d["configs"]["a"]
    assert d["metric"].startswith("KV path HBM GB/s")
    assert a["prefix_reuse"] == 512  # the 512-token cached prefix is matched
    assert a["finite"] is True
    assert a["decode_ms_1thread"] > 0 and a["append_us"] > 0 and a["prefix_match_us"] > 0


def test_config_b_legs_are_checked_before_any_gpu_work():
    r = run("--config", "b", "--b-legs", "decode,bogus", timeout=120)
    assert r.returncode != 0
    assert "--b-legs takes a comma list" in (r.stdout + r.stderr)
    assert not r.stdout.strip().startswith("{")
