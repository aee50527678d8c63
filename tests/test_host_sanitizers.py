"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer: csrc/plan.cpp (the plan authority's
admission arithmetic, partition rules, workspace layouts and rotary tables) and the CPU oracle (oracle/*.c), built
with g++/gcc -fsanitize=address,undefined -fno-sanitize-recover=all and driven over valid, invalid and edge inputs
by tests/sanitizer_driver.cpp.  Any report ends the driver with a non-zero status.  Host only: no HIP code is
built or run here."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="needs gcc and g++")
def test_plan_authority_and_oracle_under_asan_and_ubsan(tmp_path):
    objs = []
    for src in ("pvlc_oracle.c", "blake3_spec.c"):
        obj = str(tmp_path / (src + ".o"))
        subprocess.run(["gcc", "-std=c11", "-ffp-contract=off", *SAN, "-c", os.path.join(REPO, "oracle", src),
                        "-o", obj], check=True, capture_output=True, text=True)
        objs.append(obj)
    exe = str(tmp_path / "sanitizer_driver")
    build = subprocess.run(["g++", "-std=c++17", *SAN, "-I", os.path.join(REPO, "include"),
                            "-I", os.path.join(REPO, "paddleocr-vl-webgpu_amd", "csrc"), "-I", os.path.join(REPO, "oracle"),
                            os.path.join(HERE, "sanitizer_driver.cpp"),
                            os.path.join(REPO, "paddleocr-vl-webgpu_amd", "csrc", "plan.cpp"), *objs, "-lm",
                            "-o", exe], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    run = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    print(run.stdout[-500:], run.stderr[-3000:])
    assert run.returncode == 0, run.stderr[-3000:]
    assert "checks passed" in run.stdout
