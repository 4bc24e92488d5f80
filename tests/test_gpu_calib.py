"""Calibrations of the fast approximations behind certified results: the
fast f32 exp of the exact sums (relative error below 2^-22 over every input
of its domain, for the band ZS_EXP_EPS = 2^-21),
the cheaper exp of the grid predictions (below 2^-17; only the predictions
use it, so a larger error would cost time, never exactness) and the fast
Gumbel term of the lane's BSAMPLE (within ZS_GUMBEL_EPS / 4 of the exact term
for all 2^24 uniforms). The sweeps print the measured exponents.

The sweeps are test programs (tests/c/calib_*.hip), not part of the
library: this test compiles each with the library's flags when the binary is
missing or older than its source."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def build_calibration(name="calib_exp"):
    from zllm_amd.build import FLAGS, HIPCC
    src = os.path.join(HERE, "c", name + ".hip")
    exe = os.path.join(HERE, "c", name)
    if os.path.exists(exe) and os.path.getmtime(exe) >= os.path.getmtime(src):
        return exe
    flags = [f for f in FLAGS if f not in ("-fPIC", "-shared")]
    r = subprocess.run([HIPCC] + flags + [src, "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, "hipcc failed building the calibration sweep:\n" + r.stdout + r.stderr
    return exe


def test_fast_exp_error_bound():
    exe = build_calibration()
    print("[case] fast exp sweep", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_fast_gumbel_error_bound():
    exe = build_calibration("calib_gumbel")
    print("[case] fast gumbel sweep", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
