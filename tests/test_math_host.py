"""Host checks of the kernels' numeric building blocks (mxs_math.h): the
reciprocal-based f32 division of the repetition penalty, the composed bias
and penalty stage, the f64 exps used for weights (64- and 16-entry tables,
table-free), and the total-order key."""
import os
import subprocess
import tempfile
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def results():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "math_host_check")
        subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                        str(HERE / "math_host_check.cpp"), "-o", exe, "-lm"], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    res = {}
    for line in out.splitlines():
        if line.startswith("#"):
            print(line)
            continue
        name, fail, cases, *rest = line.split()
        res[name] = (int(fail), int(cases), rest)
    return res


@pytest.mark.parametrize("name", ["division", "penalize", "exp_neg", "exp_neg16", "exp_neg_p", "okey"])
def test_math(results, name):
    fail, cases, rest = results[name]
    assert cases > 1000
    assert fail == 0, f"{name}: {fail} of {cases} cases differ {rest}"
