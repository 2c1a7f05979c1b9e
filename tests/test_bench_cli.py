"""bench.py's command-line contract that needs no GPU: more than one GPU is
refused with a message (this build measures one MI355X), and the profile
modes are the documented ones."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""


def test_help_lists_the_profile_modes():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 0
    for mode in ("decode", "decode8", "prefill", "traffic", "moe"):
        assert mode in r.stdout
