"""Host checks of the scalar arithmetic the kernels share with the host
(zllm_amd/csrc/zs_math.h): glibc-identical expf and the exact sequential-sum
increment rule. CPU only."""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def test_expf_and_increments_match_libm():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "check_math")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "c", "check_math.c"), "-lm"],
                       check=True)
        r = subprocess.run([exe, "97"], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0 and "ok" in r.stdout, r.stdout
