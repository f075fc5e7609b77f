"""The GPU softmax's expf (wm_expf.h) against the host libm expf.

The reference's f32::exp is the platform libm's expf; on x86_64 Linux that
is glibc's.  wm_expf.h restates glibc's published expf algorithm; this test
compiles the same header for the host and compares bit patterns over
[-128, 0] (the softmax domain, x - max <= 0): every 13th float by default,
every float with WM_EXPF_EXHAUSTIVE=1 (about a minute on 8 cores).
"""
import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "tests" / "_build"


def test_expf_restatement_matches_libm():
    BUILD.mkdir(exist_ok=True)
    exe = BUILD / "expf_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread",
                    f"-I{ROOT / 'project-willamette_amd' / 'csrc'}", str(ROOT / "tests" / "expf_check.cpp"),
                    "-o", str(exe), "-lm"], check=True)
    stride = "1" if os.environ.get("WM_EXPF_EXHAUSTIVE") else "13"
    r = subprocess.run([str(exe), stride], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
