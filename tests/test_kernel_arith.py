"""CPU checks of arithmetic identities the HIP kernels rely on."""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_shared_divisor_quotient_is_ieee(tmp_path):
    """The row kernels divide by the row scale with one reciprocal, a multiply
    and two FMAs; that must equal IEEE x / scale wherever it can change a code."""
    exe = tmp_path / "div_shared_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    str(HERE / "csrc" / "div_shared_check.c"), "-lm"], check=True)
    res = subprocess.run([str(exe), "20000000", "12345"], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout
    n, bad = (int(tok.split("=")[1]) for tok in res.stdout.split())
    assert n > 19_000_000 and bad == 0
