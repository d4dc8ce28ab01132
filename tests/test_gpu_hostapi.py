"""The reference's host-pointer entry points as exported by the product library (the drop-ins
reference src/llama.c:876-884 calls unchanged): sgl_matmul_nt (reference src/ops.c:243-279) and
sgl_matmul_w8a16 (reference src/quant.c:44-89), against the oracle on the same inputs, ragged N
and K, with and without bias, several row counts; repeated calls reuse the device copy of the
weight, and a weight changed in place is picked up after sgl_qcache_release.
Tolerance (BASELINE): max|y - y_ref| / max|y_ref| <= 1e-3."""
import ctypes as C

import numpy as np
import pytest

import synth
from linear_cases import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
SHAPES = [(72, 100), (300, 1000), (1000, 4096), (4864, 896)]


def _lib():
    import sgl_qlinear as q
    L = q._L
    L.sgl_qcache_release.argtypes = [C.c_void_p]
    L.sgl_qcache_release.restype = C.c_int
    L.sgl_qcache_clear.restype = C.c_int
    return q, L


@pytest.mark.parametrize("N,K", SHAPES)
def test_matmul_nt_host(orc, N, K):
    q, L = _lib()
    W = synth.normal(7 + N, (N, K), 0.05)
    b = synth.normal(8 + N, N, 0.1)
    for M in (1, 8, 33):
        A = synth.normal(9 + M, (M, K))
        for bias in (None, b):
            print(f"[gpu] sgl_matmul_nt N={N} K={K} M={M} bias={bias is not None}", flush=True)
            y = q.matmul_nt(A, W, bias)
            ref = orc.matmul_nt(A, W, bias)
            e = rel_err(y, ref)
            assert e <= TOL, (M, e)
            # the second call reuses the resident weight and gives the same bits
            assert np.array_equal(q.matmul_nt(A, W, bias), y)
    assert L.sgl_qcache_release(C.c_void_p(W.ctypes.data)) >= 1


@pytest.mark.parametrize("N,K", SHAPES)
def test_matmul_w8a16_host(orc, N, K):
    q, L = _lib()
    q8, s8 = synth.quant_rows_i8(synth.normal(11 + N, (N, K), 0.02))
    b = synth.normal(12 + N, N, 0.1)
    for M in (1, 8, 33):
        A = synth.normal(13 + M, (M, K))
        for bias in (None, b):
            print(f"[gpu] sgl_matmul_w8a16 N={N} K={K} M={M} bias={bias is not None}",
                  flush=True)
            y = q.matmul_w8a16(A, q8, s8, bias)
            ref = orc.matmul_w8a16(A, q8, s8, bias)
            e = rel_err(y, ref)
            assert e <= TOL, (M, e)
            assert np.array_equal(q.matmul_w8a16(A, q8, s8, bias), y)
    L.sgl_qcache_release(C.c_void_p(q8.ctypes.data))


def test_weight_changed_in_place(orc):
    """A weight buffer rewritten after use: released, the next call uploads the new contents;
    a different shape on the same pointer is a different entry."""
    q, L = _lib()
    N, K = 256, 512
    W = synth.normal(21, (N, K), 0.05)
    A = synth.normal(22, (4, K))
    assert rel_err(q.matmul_nt(A, W), orc.matmul_nt(A, W)) <= TOL
    W[:] = synth.normal(23, (N, K), 0.05)
    assert L.sgl_qcache_release(C.c_void_p(W.ctypes.data)) == 1
    assert rel_err(q.matmul_nt(A, W), orc.matmul_nt(A, W)) <= TOL
    q8, s8 = synth.quant_rows_i8(synth.normal(24, (N, K), 0.02))
    assert rel_err(q.matmul_w8a16(A, q8, s8), orc.matmul_w8a16(A, q8, s8)) <= TOL
    s8 *= 2  # scales rewritten in place: every scale is in the fingerprint
    assert rel_err(q.matmul_w8a16(A, q8, s8), orc.matmul_w8a16(A, q8, s8)) <= TOL
    assert L.sgl_qcache_clear() >= 2


def test_empty_sum_and_rows(orc):
    """K = 0 writes the bias (or zeros), as the reference's empty sum does; M = 0 writes
    nothing."""
    q, L = _lib()
    b = synth.normal(31, 40, 0.1)
    for fn in ("nt", "w8"):
        out = np.full((3, 40), 7.0, np.float32)
        A = np.zeros((3, 1), np.float32)
        if fn == "nt":
            L.sgl_matmul_nt(A.ctypes.data, np.zeros(40, np.float32).ctypes.data, b.ctypes.data,
                            out.ctypes.data, 3, 40, 0)
        else:
            L.sgl_matmul_w8a16(A.ctypes.data, np.zeros(40, np.int8).ctypes.data,
                               np.ones(40, np.float32).ctypes.data, b.ctypes.data,
                               out.ctypes.data, 3, 40, 0)
        assert np.array_equal(out, np.tile(b, (3, 1))), fn
    out = np.full((2, 5), 7.0, np.float32)
    L.sgl_matmul_nt(None, None, None, out.ctypes.data, 0, 5, 3)
    assert (out == 7.0).all()
