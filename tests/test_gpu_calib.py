"""Calibration of the fast f32 exp behind the certified increments: its
relative error over every input of its domain must stay far below the band
ZS_EXP_EPS = 2^-18 the kernels assume."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_fast_exp_error_bound():
    exe = os.path.join(HERE, "c", "calib_exp")
    assert os.path.exists(exe), "build() compiles tests/c/calib_exp"
    print("[case] fast exp sweep", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
