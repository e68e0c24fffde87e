"""Native host checks under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only): the
host C-ABI helpers (builderforce-inference_amd/host/bfi_host.cpp) and the C oracle, built
with g++/gcc from source with -fsanitize=address,undefined and driven by
tests/native/host_checks.cpp, which also restates the mix_decode known answers
(engine/mod.rs:663-707). No GPU code is built or run here."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="no host compiler")
def test_host_helpers_and_oracle_under_sanitizers(tmp_path):
    obj = str(tmp_path / "oracle.o")
    exe = str(tmp_path / "host_checks")
    subprocess.run(["gcc", "-std=c11", "-ffp-contract=off", "-fno-fast-math", *SAN, "-c", "-o", obj,
                    os.path.join(ROOT, "oracle", "bfi_oracle.c")], check=True, timeout=300)
    subprocess.run(["g++", "-std=c++17", *SAN, "-o", exe, os.path.join(ROOT, "tests", "native", "host_checks.cpp"),
                    os.path.join(ROOT, "builderforce-inference_amd", "host", "bfi_host.cpp"), obj, "-lm", "-lpthread"],
                   check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    assert r.stdout.strip() == "ok"
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
