"""Calibration of the fast f32 exp behind the certified increments: its
relative error over every input of its domain must stay far below the band
ZS_EXP_EPS = 2^-18 the kernels assume.

The sweep is a test program (tests/c/calib_exp.hip), not part of the
library: this test compiles it with the library's flags when the binary is
missing or older than its source."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "c", "calib_exp.hip")
EXE = os.path.join(HERE, "c", "calib_exp")


def build_calibration():
    from zllm_amd.build import FLAGS, HIPCC
    if os.path.exists(EXE) and os.path.getmtime(EXE) >= os.path.getmtime(SRC):
        return EXE
    flags = [f for f in FLAGS if f not in ("-fPIC", "-shared")]
    r = subprocess.run([HIPCC] + flags + [SRC, "-o", EXE], capture_output=True, text=True)
    assert r.returncode == 0, "hipcc failed building the calibration sweep:\n" + r.stdout + r.stderr
    return EXE


def test_fast_exp_error_bound():
    exe = build_calibration()
    print("[case] fast exp sweep", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
