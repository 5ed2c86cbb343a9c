"""bench.py's command-line contract, checked without a GPU: a request for
more than one GPU is refused before any device work, and the JSON line's
builder functions that need no device agree with the byte and op counts the
roofline uses."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    for env_extra, args in (({}, ["--gpus", "2"]), ({"WORLD_SIZE": "2"}, [])):
        env = dict(os.environ, **env_extra)
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, env=env,
                           capture_output=True, text=True, timeout=120)
        assert r.returncode != 0
        assert "one GPU" in r.stdout + r.stderr


def test_algorithmic_bytes_of_the_headline_shape():
    sys.path.insert(0, ROOT)
    import bench
    # K*N/2 codes + (K/G)*N*2 fp16 scales + (K/G)*N/2 u4 zeros + M*K*2 + M*N*2
    assert bench.w4a16_bytes(1, 8192, 28672, 128) == 122_101_760
    assert bench.w4a16_bytes(1, 4096, 4096, 128) == 8_732_672
