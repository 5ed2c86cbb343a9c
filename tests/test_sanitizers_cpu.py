"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

* The prepacked-W4 file reader (longhornai_amd/csrc/w4file.cpp), the one
  parser of untrusted input in the library, built with both sanitizers into
  tests/cpp/bin/w4file_asan and run over valid files and every kind of
  damaged or hostile file the format tests use.
* The CPU oracle (oracle/lhq_oracle.c) built the same way
  (oracle/_asan/liboracle.so) and driven through its own pin suites in a
  child Python process with the sanitizer runtimes preloaded.

Any sanitizer report fails the test (the builds use
-fno-sanitize-recover=all, so a report also ends the process non-zero)."""
import os
import subprocess
import sys

import numpy as np
import pytest

from longhornai_amd import capi
from tests import test_weights_io_cpu as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "cpp", "bin", "w4file_asan")
ASAN_ORACLE = os.path.join(ROOT, "oracle", "_asan", "liboracle.so")
REPORT = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def lib():
    return capi.load()


def _files(lib, d):
    """(path, want_ok) for valid files, the BAD mutations and hostile headers."""
    out = []
    for i, (K, N, G, asym) in enumerate([(256, 48, 128, True), (4096, 40, 64, False)]):
        p = str(d / f"ok{i}.safetensors")
        W.write(p, W.tensors(lib, K, N, G, asym), W.meta_for(K, N, G))
        out.append((p, True))
    K, N, G = 256, 48, 128
    for name, mutate, _ in W.BAD:
        t, m = W.tensors(lib, K, N, G, True), W.meta_for(K, N, G)
        mutate(t, m)
        p = str(d / f"bad_{name}.safetensors")
        W.write(p, t, m)
        out.append((p, False))
    raw = open(out[0][0], "rb").read()
    hlen = int.from_bytes(raw[:8], "little")
    q = lib.lhq_w4_qweight_bytes(K, N)
    hostile = {
        "truncated": raw[:-1],
        "trailing": raw + b"\0",
        "short_header": raw[:20],
        "empty": b"",
        "huge_hlen": (1 << 40).to_bytes(8, "little") + raw[8:],
        "brace_flood": raw[:8] + b"{" * hlen + raw[8 + hlen:],
        "wrapped": W._rewrite_header(raw, lambda h: h["qweight"].update(data_offsets=[2 ** 64 - 1 - q, 2 ** 64 - 1])),
        "huge_dims": W._rewrite_header(raw, lambda h: h["__metadata__"].update(K=str(2 ** 20), N=str(2 ** 20))),
        "deep": raw[:8] + (b"[" * 64).ljust(hlen, b" ") + raw[8 + hlen:],
        "bad_escape": W._rewrite_header(raw, lambda h: h["__metadata__"].update(format="\u0001")),
    }
    for name, data in hostile.items():
        p = str(d / f"hostile_{name}.safetensors")
        open(p, "wb").write(data)
        out.append((p, False))
    return out


def test_w4file_reader_under_asan_ubsan(lib, tmp_path):
    assert os.path.exists(CHECK), f"{CHECK} is not built (run __graft_entry__.build())"
    files = _files(lib, tmp_path)
    r = subprocess.run([CHECK] + [p for p, _ in files], capture_output=True, text=True, timeout=120,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=1"})
    assert not any(s in r.stderr for s in REPORT), r.stderr[-4000:]
    assert r.returncode == 0, r.stderr[-4000:]
    lines = r.stdout.strip().splitlines()
    assert len(lines) == len(files)
    for (path, ok), line in zip(files, lines):
        status = int(line.split(" ", 1)[0])
        assert (status == 0) == ok, line


@pytest.mark.skipif(_runtime("libasan.so") is None or _runtime("libubsan.so") is None,
                    reason="gcc sanitizer runtimes not found")
def test_oracle_pin_suites_under_asan_ubsan():
    assert os.path.exists(ASAN_ORACLE), f"{ASAN_ORACLE} is not built (run __graft_entry__.build())"
    env = {**os.environ, "LD_PRELOAD": f"{_runtime('libasan.so')}:{_runtime('libubsan.so')}",
           "ASAN_OPTIONS": "detect_leaks=0", "LHO_ORACLE_SO": ASAN_ORACLE}
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        "tests/test_oracle_pins.py", "tests/test_moe_oracle.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert not any(s in out for s in REPORT), out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out and "failed" not in out
