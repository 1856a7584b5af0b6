"""Opt-in (FSK_SANITIZE=1): builds tests/fuzz_capi.cpp with the library's
source under AddressSanitizer and UndefinedBehaviorSanitizer on the host pass
and runs it.  The fuzz calls every C-ABI entry point with random and
perturbed-valid arguments; every call must return a status without a
sanitizer report.

CPU only.  Perturbed-valid calls carry fake device addresses, so they are safe
only while no GPU is visible (they stop at their first HIP call).  The child
runs with every device hidden by its environment, refuses to run if the HIP
runtime still reports a device (exit code 3), and this test then skips.  The
build takes a few minutes, so the default CPU run skips it too; neither file
is shipped to GPU boxes."""
import os
import subprocess

import pytest

from fasterkernels_amd import build

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Hides every GPU from the fuzz process (HIP and the ROCm runtime underneath).
NO_DEVICE_ENV = {"HIP_VISIBLE_DEVICES": "-1", "ROCR_VISIBLE_DEVICES": "-1", "CUDA_VISIBLE_DEVICES": "-1",
                 "GPU_DEVICE_ORDINAL": "-1"}


@pytest.mark.skipif(os.environ.get("FSK_SANITIZE") != "1", reason="set FSK_SANITIZE=1 to run the sanitizer fuzz")
def test_capi_fuzz_under_sanitizers(tmp_path):
    exe = str(tmp_path / "fuzz_capi")
    cmd = [build.hipcc(), "--offload-arch=gfx950", "-O1", "-g", "-std=c++17",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-omit-frame-pointer",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(REPO, "include"), build.SRC, os.path.join(REPO, "tests", "fuzz_capi.cpp"), "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=1800)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, UBSAN_OPTIONS="print_stacktrace=1", ASAN_OPTIONS="detect_leaks=0")
    env.update(NO_DEVICE_ENV)
    run = subprocess.run([exe], capture_output=True, text=True, timeout=1800, env=env)
    out = run.stdout + run.stderr
    if run.returncode == 3 and "device visible" in out:
        pytest.skip("a GPU is visible to the fuzz process; the fuzz runs only without one")
    assert run.returncode == 0, out[-3000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-3000:]
    assert "returned" not in out and "null last_error" not in out, out[-3000:]
    assert out.rstrip().endswith("done"), out[-3000:]
