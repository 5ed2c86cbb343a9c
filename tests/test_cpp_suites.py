"""The C++ suites over the lh:: drop-in headers (tests/cpp), run as
subprocesses: the host-side dtype suite on the CPU, the kernel suites
(quantizers, quantized GEMMs, fp32 GEMMs through liblonghorn_kernels.so on
the GPU) with the gpu marker.  Both compare against the oracle library."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin")


def _run(name: str, timeout: int) -> str:
    exe = os.path.join(BIN, name)
    assert os.path.exists(exe), f"{exe} is not built (run __graft_entry__.build())"
    print(f"running {name}", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=timeout)
    out = r.stdout + r.stderr
    print(out[-4000:], flush=True)
    assert r.returncode == 0, f"{name} failed:\n{out[-4000:]}"
    return out


def test_cpp_dtypes_suite():
    out = _run("lh_dtypes_tests", 120)
    assert "[  PASSED  ] 11 tests." in out


@pytest.mark.gpu
def test_cpp_kernel_suites():
    out = _run("lh_kernel_tests", 110)
    assert "FAILED" not in out
