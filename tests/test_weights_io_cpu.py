"""The prepacked-W4 file format (lhq_w4_file_info) on the CPU: files written
by the safetensors package itself (an independent writer) are accepted, and
each kind of damage or mismatch is rejected with the right status.  No GPU:
lhq_w4_file_info reads and checks files on the host only."""
import ctypes
import os

import numpy as np
import pytest

from longhornai_amd import capi

safetensors_np = pytest.importorskip("safetensors.numpy")


def fnv1a64(data: bytes) -> int:
    h = 1469598103934665603
    for b in data:
        h = ((h ^ b) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def sizes(lib, K, N, G, asym):
    return (lib.lhq_w4_qweight_bytes(K, N), lib.lhq_w4_scales_bytes(K, N, G, 1 if asym else 0),
            lib.lhq_w4_zeros_bytes(K, N, G) if asym else 0)


def tensors(lib, K, N, G, asym, seed=0):
    q, s, z = sizes(lib, K, N, G, asym)
    g = np.random.default_rng(seed)
    t = {"qweight": g.integers(0, 256, q, dtype=np.uint8)}
    t["scales"] = (g.standard_normal(s // 2).astype(np.float16) if asym
                   else g.standard_normal(s // 4).astype(np.float32))
    if asym:
        t["zeros"] = g.integers(0, 2 ** 32, z // 4, dtype=np.uint32)
    return t


def write(path, t, meta, checksum=True):
    """safetensors file with a correct fnv1a64 over its data section (unless
    `checksum` is False, or meta already holds one)."""
    meta = dict(meta)
    if "fnv1a64" not in meta:
        meta["fnv1a64"] = "0" * 16
    safetensors_np.save_file(t, path, metadata=meta)
    if checksum and meta["fnv1a64"] == "0" * 16:
        raw = open(path, "rb").read()
        hlen = int.from_bytes(raw[:8], "little")
        digest = "%016x" % fnv1a64(raw[8 + hlen:])
        header = raw[8:8 + hlen].replace(b'"fnv1a64":"' + b"0" * 16 + b'"', b'"fnv1a64":"' + digest.encode() + b'"')
        assert len(header) == hlen
        open(path, "wb").write(raw[:8] + header + raw[8 + hlen:])


def meta_for(K, N, G, **over):
    m = {"format": "lhq-w4-prepacked", "version": "1", "layout": "w4-tile16x128-v1",
         "K": str(K), "N": str(N), "group_size": str(G)}
    m.update(over)
    return {k: v for k, v in m.items() if v is not None}


@pytest.fixture(scope="module")
def lib():
    return capi.load()


def info(lib, path):
    vals = [ctypes.c_int(-1) for _ in range(4)]
    st = lib.status("lhq_w4_file_info", str(path).encode(), *[ctypes.addressof(v) for v in vals])
    return st, [v.value for v in vals]


@pytest.mark.parametrize("K,N,G,asym", [(256, 48, 128, True), (4096, 40, 64, False), (384, 16, 384, True)])
def test_valid_files(lib, tmp_path, K, N, G, asym):
    p = tmp_path / "w.safetensors"
    write(str(p), tensors(lib, K, N, G, asym), meta_for(K, N, G))
    st, v = info(lib, p)
    assert st == capi.LHQ_OK, lib.last_error()
    assert v == [K, N, G, 1 if asym else 0]


BAD = [
    # (name, mutation, expected status)
    ("format", lambda t, m: m.update(format="something-else"), capi.LHQ_ERR_INVALID),
    ("version", lambda t, m: m.update(version="2"), capi.LHQ_ERR_UNSUPPORTED),
    ("layout", lambda t, m: m.update(layout="w4-tile32x64-v1"), capi.LHQ_ERR_UNSUPPORTED),
    ("no_version", lambda t, m: m.pop("version"), capi.LHQ_ERR_UNSUPPORTED),
    ("K_text", lambda t, m: m.update(K="25x"), capi.LHQ_ERR_INVALID),
    ("K_mismatch", lambda t, m: m.update(K="512"), capi.LHQ_ERR_INVALID),
    ("G_not_dividing", lambda t, m: m.update(group_size="100"), capi.LHQ_ERR_INVALID),
    # divides K, but no W4A16 GEMM takes it (32, 64 or a multiple of 128)
    ("G_unsupported", lambda t, m: m.update(group_size="16"), capi.LHQ_ERR_UNSUPPORTED),
    ("scales_dtype", lambda t, m: t.update(scales=t["scales"].astype(np.float32)), capi.LHQ_ERR_INVALID),
    ("qweight_short", lambda t, m: t.update(qweight=t["qweight"][:-16]), capi.LHQ_ERR_INVALID),
    ("missing_zeros", lambda t, m: t.pop("zeros"), capi.LHQ_ERR_INVALID),
    ("extra_tensor", lambda t, m: t.update(extra=np.zeros(4, np.uint8)), capi.LHQ_ERR_INVALID),
    ("checksum", lambda t, m: m.update(fnv1a64="0123456789abcdef"), capi.LHQ_ERR_INVALID),
]


@pytest.mark.parametrize("name,mutate,status", BAD, ids=[b[0] for b in BAD])
def test_rejects(lib, tmp_path, name, mutate, status):
    K, N, G = 256, 48, 128
    t = tensors(lib, K, N, G, True)
    m = meta_for(K, N, G)
    mutate(t, m)
    p = tmp_path / "w.safetensors"
    write(str(p), t, m)
    st, _ = info(lib, p)
    assert st == status, (name, st, lib.last_error())
    assert lib.last_error()


def test_rejects_damaged_bytes(lib, tmp_path):
    K, N, G = 256, 48, 128
    p = tmp_path / "w.safetensors"
    write(str(p), tensors(lib, K, N, G, True), meta_for(K, N, G))
    raw = open(p, "rb").read()
    cases = {
        "flipped_data_byte": raw[:-100] + bytes([raw[-100] ^ 1]) + raw[-99:],
        "truncated_data": raw[:-1],
        "trailing_bytes": raw + b"\0",
        "truncated_header": raw[:20],
        "empty": b"",
        "huge_header_length": (1 << 40).to_bytes(8, "little") + raw[8:],
        "garbage_header": raw[:8] + b"{" * int.from_bytes(raw[:8], "little") + raw[8 + int.from_bytes(raw[:8], "little"):],
    }
    for name, data in cases.items():
        q = tmp_path / f"{name}.safetensors"
        open(q, "wb").write(data)
        st, _ = info(lib, q)
        assert st == capi.LHQ_ERR_INVALID, (name, st, lib.last_error())
    st, _ = info(lib, tmp_path / "does_not_exist.safetensors")
    assert st == capi.LHQ_ERR_INVALID


def _rewrite_header(raw: bytes, edit) -> bytes:
    """The same file with its JSON header replaced by edit(header dict)."""
    import json
    hlen = int.from_bytes(raw[:8], "little")
    h = json.loads(raw[8:8 + hlen])
    edit(h)
    hb = json.dumps(h, separators=(",", ":")).encode()
    hb += b" " * ((8 - (8 + len(hb)) % 8) % 8)
    return len(hb).to_bytes(8, "little") + hb + raw[8 + hlen:]


def test_rejects_hostile_headers(lib, tmp_path):
    """Header claims that would index outside the data section or size a
    buffer from a length the file does not hold are rejected before any
    allocation: wrapped 64-bit offsets, offsets past the data, swapped
    offsets, and dims implying far more bytes than the file has."""
    K, N, G = 256, 48, 128
    p = tmp_path / "w.safetensors"
    write(str(p), tensors(lib, K, N, G, True), meta_for(K, N, G))
    raw = open(p, "rb").read()
    q, _, _ = sizes(lib, K, N, G, True)
    big = 2 ** 64 - 1

    def set_off(name, b, e):
        return lambda h: h[name].update(data_offsets=[b, e])

    def claim(k, n):
        def f(h):
            h["__metadata__"].update(K=str(k), N=str(n))
        return f

    cases = {
        "wrapped_offsets": set_off("qweight", big - q, big),
        "offsets_past_data": set_off("qweight", 10 ** 12, 10 ** 12 + q),
        "swapped_offsets": set_off("qweight", q, 0),
        "huge_dims": claim(2 ** 20, 2 ** 20),
        "max_int_dims": claim(2 ** 31 - 2, 2 ** 31 - 1),
    }
    for name, edit in cases.items():
        f = tmp_path / f"{name}.safetensors"
        open(f, "wb").write(_rewrite_header(raw, edit))
        st, _ = info(lib, f)
        assert st == capi.LHQ_ERR_INVALID, (name, st, lib.last_error())
    # the untouched rewrite is still a valid file (the helper itself is sound)
    f = tmp_path / "same.safetensors"
    open(f, "wb").write(_rewrite_header(raw, lambda h: None))
    assert info(lib, f)[0] == capi.LHQ_OK, lib.last_error()
