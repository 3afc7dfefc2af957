"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer: every
function of oracle/mx_oracle.c driven over seeded random and edge-case inputs
(oracle/sanitize_check.c, `make -C oracle sanitize`), with the contracts each
states checked on the way.  Host code only; no GPU."""
import shutil
import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parent.parent / "oracle"


def test_oracle_clean_under_asan_and_ubsan():
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    res = subprocess.run(["make", "-C", str(ORACLE), "sanitize", "CC=gcc"], capture_output=True, text=True,
                         timeout=300)
    if res.returncode != 0 and "cannot find" in res.stderr and "asan" in res.stderr:
        pytest.skip("gcc has no AddressSanitizer runtime here")
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "sanitize_check: clean" in res.stdout
