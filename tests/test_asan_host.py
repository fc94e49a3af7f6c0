"""Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the C ABI.

``tests/asan/run_host_asan.sh`` compiles the library's sources host-only with
both sanitizers, links them with ``tests/asan/abi_host_check.cpp`` and runs
it: every size helper over extreme arguments, the codebook classifier on
exact-size heap tables, every entry point's argument errors, and (no GPU
visible) the launch paths' HIP-error reporting.  Any sanitizer report, leak
or failed expectation fails the test.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="needs hipcc")
def test_c_abi_under_host_sanitizers():
    env = dict(os.environ)
    env.pop("HIP_VISIBLE_DEVICES", None)
    r = subprocess.run(["bash", os.path.join(HERE, "asan", "run_host_asan.sh")], capture_output=True, text=True,
                       timeout=900, env=env)
    out = r.stdout + r.stderr
    print(out[-4000:])
    assert r.returncode == 0, out[-4000:]
    assert "0 failed" in r.stdout
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out
