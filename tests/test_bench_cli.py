"""bench.py's command line without a GPU: the flags parse, and a request for
more than one GPU ends with a message (this build measures one GPU)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                          timeout=120)


def test_help_lists_the_contract_flags():
    r = run("--help")
    assert r.returncode == 0, r.stderr
    for flag in ("--gpus", "--steps", "--warmup", "--config", "--no-others", "--short-record"):
        assert flag in r.stdout, flag


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no bench line


def test_unknown_configuration_is_rejected():
    r = run("--config", "7")
    assert r.returncode != 0
    assert "invalid choice" in r.stderr
