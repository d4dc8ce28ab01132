"""sgl_qlinear_forward_noalloc (the forward that allocates nothing: its prefill GEMM works in
the library's per-GPU scratch array) against sgl_qlinear_forward, through the C ABI: the same
kernels, so the outputs must be bit-identical.  Two calls in a row, the second with fewer rows,
for the GEMM (f32 and bf16 rows, bias), the split-row GEMV and the one-row GEMV; a batch that
needs more than the scratch array is refused with -1."""
import ctypes as C

import numpy as np
import pytest

import synth
from linear_cases import build, product

pytestmark = pytest.mark.gpu


def _noalloc(ql, A, bias=None, out=None):
    import torch
    import sgl_qlinear as q
    f = q._L.sgl_qlinear_forward_noalloc
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_void_p,
                  C.c_void_p]
    f.restype = C.c_int
    A = A.contiguous()
    if out is None:
        out = torch.empty((A.shape[0], ql.N), dtype=torch.float32, device=A.device)
    rc = f(ql.h, C.c_void_p(A.data_ptr()), q._dtype_code(A), A.shape[0],
           None if bias is None else C.c_void_p(bias.data_ptr()), C.c_void_p(out.data_ptr()),
           q._stream())
    return rc, out


@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4", "w8"])
def test_noalloc_matches_forward(fmt):
    import torch
    N, K = 1000, 4096
    kind, a = build(fmt, N, K, seed=71)
    ql = product(kind, a, N, K)
    bias = torch.from_numpy(synth.normal(72, N, 0.1)).cuda()
    for dt in (torch.float32, torch.bfloat16):
        for M in (700, 300, 20, 1):  # each call smaller than the one before
            A = torch.from_numpy(synth.normal(73 + M, (M, K))).cuda().to(dt)
            print(f"[gpu] noalloc {fmt} M={M} {dt}", flush=True)
            rc, y = _noalloc(ql, A, bias)
            torch.cuda.synchronize()
            assert rc == 0
            ref = ql.forward(A, bias=bias)
            assert torch.equal(y, ref), (fmt, M, dt)


def test_noalloc_refuses_oversized_batch():
    import torch
    N, K = 64, 16384
    kind, a = build("gptq4", N, K, seed=74)
    ql = product(kind, a, N, K)
    A = torch.zeros((2048, K), dtype=torch.float32, device="cuda")  # 2048 x 16384 f32 operands
    rc, _ = _noalloc(ql, A)
    assert rc == -1
