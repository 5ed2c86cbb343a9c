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
    assert "[  PASSED  ] 3 tests." in out


@pytest.mark.gpu
def test_cpp_kernel_suites():
    out = _run("lh_kernel_tests", 110)
    assert "FAILED" not in out


def _bench(args, timeout):
    exe = os.path.join(ROOT, "longhornai_amd", "bin", "lh_bench")
    assert os.path.exists(exe), f"{exe} is not built (run __graft_entry__.build())"
    print("running lh_bench " + " ".join(args), flush=True)
    r = subprocess.run([exe] + args, capture_output=True, text=True, timeout=timeout)
    out = r.stdout + r.stderr
    print(out[-3000:], flush=True)
    assert r.returncode == 0, f"lh_bench failed:\n{out[-3000:]}"
    return out


@pytest.mark.gpu
def test_lh_bench_hip_timing(tmp_path):
    """The benchmark driver's HIP timing mode: event-timed launches of the
    decode GEMV with rotating weight sets, table + roofline + CSV."""
    csv = tmp_path / "bench.csv"
    roof = tmp_path / "roofline.csv"
    out = _bench(["--timing", "hip", "--filter", "w4a16/decode", "--iters", "20", "--warmup", "3",
                  "--csv", str(csv), "--roofline", str(roof)], 100)
    assert "w4a16/decode[1x8192x28672]" in out
    rows = csv.read_text().strip().splitlines()
    assert rows[0].startswith("name,timing,mean_us")
    name, timing, mean_us = rows[1].split(",")[:3]
    assert timing == "hip" and float(mean_us) > 0
    r = roof.read_text().strip().splitlines()[1].split(",")
    assert r[5] == "memory"  # AI of a decode GEMV is far below the bf16 ridge


@pytest.mark.gpu
def test_lh_bench_host_timing():
    """Host timing over the synchronous lh:: drop-in, as the reference's driver."""
    out = _bench(["--timing", "host", "--filter", "lh/c1_w8_gemv", "--iters", "3", "--warmup", "1"], 100)
    assert "lh/c1_w8_gemv[1x4096x4096]" in out
