"""The FMA-corrected reciprocal division of the kernels (x * r, then one Markstein
correction) must equal IEEE x / T bit for bit for |x| in [2^-100, 2^100) and T in
[2^-20, 2^20] (sample.rs:373-375 divides). A strided sample of every f32 in that range
(one in 997, about 2.5 million values) for temperatures across the range, on the CPU with
libm fmaf."""
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def div_check(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("div") / "div_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "div_check.c"), "-lm"],
                   check=True)
    return exe


def test_fma_corrected_division_is_ieee(div_check):
    rng = np.random.default_rng(21)
    temps = [2.0 ** -20, 2.0 ** 20, 0.2, 0.7, 1.0, 1.3, 1.5, 3.0, 1e-3, 7e3] + list(
        (2.0 ** rng.uniform(-20, 20, 6)).astype(np.float32))
    out = subprocess.run([div_check, "997"] + [repr(float(np.float32(t))) for t in temps], check=True,
                         capture_output=True, text=True).stdout.split("\n")
    rows = [l.split() for l in out if l.strip()]
    assert len(rows) == len(temps)
    for t, count, bad in rows:
        assert int(count) > 2_000_000, (t, count)
        assert int(bad) == 0, f"T={t}: {bad} of {count} quotients differ from IEEE division"


def test_planted_mistake_is_caught(div_check, tmp_path):
    # without the correction step (plain x * (1/T)) many quotients differ: the check has teeth
    src = open(os.path.join(HERE, "div_check.c")).read().replace("return e != e ? q : s;", "return q;")
    c = tmp_path / "mut.c"
    c.write_text(src)
    exe = str(tmp_path / "mut")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, str(c), "-lm"], check=True)
    out = subprocess.run([exe, "9973", "0.7"], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[2]) > 0
