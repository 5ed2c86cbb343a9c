"""Prepacked W4 weights saved and loaded through the library (lhq_w4_save /
lhq_w4_load) on the GPU: byte-exact round trips, interoperation with the
safetensors package in both directions, and the GEMM on loaded weights equal
to the GEMM on the originals."""
import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu

safetensors_np = pytest.importorskip("safetensors.numpy")


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _asym(oracle, ops, K, N, G, seed):
    p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed), G)
    return ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)


def _sym(oracle, ops, K, N, G, seed):
    p, s = oracle.q4_quantize_groupwise(D.normal((K, N), 0.02, seed), G)
    return ops.prepack_w4_sym(ops.dev(p), ops.dev(s), K, N, G)


def _save(ops, w, path):
    ops.run("lhq_w4_save", str(path).encode(), w.qweight, w.scales, w.zeros, w.K, w.N, w.G, 1 if w.asym else 0)


def _load(ops, path, K, N, G, asym):
    q, s, z = ops.w4_buffers(K, N, G, asym)
    ops.run("lhq_w4_load", str(path).encode(), q, s, z, K, N, G, 1 if asym else 0)
    return ops.W4Weights(q, s, z, K, N, G, asym)


def _bytes(t):
    return t.detach().cpu().numpy().view(np.uint8)


@pytest.mark.parametrize("K,N,G,asym", [(4096, 1040, 128, True), (512, 72, 64, True), (1024, 48, 32, False)])
def test_round_trip_and_gemm(oracle, ops, tmp_path, K, N, G, asym):
    w = (_asym if asym else _sym)(oracle, ops, K, N, G, 7 + K)
    path = tmp_path / "w.safetensors"
    _save(ops, w, path)
    v = _load(ops, path, K, N, G, asym)
    assert np.array_equal(_bytes(v.qweight), _bytes(w.qweight))
    assert np.array_equal(_bytes(v.scales), _bytes(w.scales))
    if asym:
        assert np.array_equal(_bytes(v.zeros), _bytes(w.zeros))
        A = ops.dev(D.to_bf16_bits(oracle, D.normal((64, K), 1.0, 3)))
        c0, c1 = ops.gemm_w4a16_bf16(A, w), ops.gemm_w4a16_bf16(A, v)
    else:
        A = ops.dev(D.uniform((8, K), -1, 1, 3))
        c0, c1 = ops.gemm_w4a16(A, w), ops.gemm_w4a16(A, v)
    assert np.array_equal(_bytes(c0), _bytes(c1))


def test_file_is_safetensors(oracle, ops, tmp_path):
    """A file the library writes reads back with the safetensors package."""
    K, N, G = 1024, 96, 128
    w = _asym(oracle, ops, K, N, G, 11)
    path = tmp_path / "w.safetensors"
    _save(ops, w, path)
    t = safetensors_np.load_file(str(path))
    assert set(t) == {"qweight", "scales", "zeros"}
    assert t["scales"].dtype == np.float16 and t["zeros"].dtype == np.uint32
    assert np.array_equal(t["qweight"], _bytes(w.qweight))
    assert np.array_equal(t["scales"].view(np.uint8), _bytes(w.scales))
    assert np.array_equal(t["zeros"].view(np.uint8), _bytes(w.zeros))


def test_loads_file_written_by_safetensors(oracle, ops, tmp_path):
    """A file the safetensors package writes (with the metadata and checksum
    of the format) loads into the same device bytes."""
    from tests.test_weights_io_cpu import meta_for, write
    K, N, G = 512, 40, 128
    w = _asym(oracle, ops, K, N, G, 13)
    t = {"qweight": _bytes(w.qweight).copy(), "scales": _bytes(w.scales).view(np.float16).copy(),
         "zeros": _bytes(w.zeros).view(np.uint32).copy()}
    path = tmp_path / "w.safetensors"
    write(str(path), t, meta_for(K, N, G))
    v = _load(ops, path, K, N, G, True)
    for a, b in ((v.qweight, w.qweight), (v.scales, w.scales), (v.zeros, w.zeros)):
        assert np.array_equal(_bytes(a), _bytes(b))


def test_load_rejects_other_dims(oracle, ops, lib, tmp_path):
    from longhornai_amd.capi import LHQ_ERR_INVALID
    K, N, G = 512, 40, 128
    w = _asym(oracle, ops, K, N, G, 17)
    path = tmp_path / "w.safetensors"
    _save(ops, w, path)
    q, s, z = ops.w4_buffers(K, N, G, True)
    st = lib.status("lhq_w4_load", str(path).encode(), q.data_ptr(), s.data_ptr(), z.data_ptr(), K, 48, G, 1,
                    ops.stream())
    assert st == LHQ_ERR_INVALID and "holds K=512 N=40" in lib.last_error()
    st = lib.status("lhq_w4_load", str(path).encode(), q.data_ptr(), s.data_ptr(), z.data_ptr(), K, N, G, 0,
                    ops.stream())
    assert st == LHQ_ERR_INVALID
