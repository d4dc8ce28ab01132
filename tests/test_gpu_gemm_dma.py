"""Prefill GEMM shapes that take k_gemm_dma (direct formats, K <= 4096, at least 200 tiles of
128 rows x 192 columns for bf16 rows, of 64 rows for f32 rows; 8 waves of 384 columns when
those alone give 200 tiles), against the reference CPU path (oracle dequant +
sgl_matmul_nt).  Covers 8-bit codes, MXFP4, f32 rows (two A pieces), ragged M and N, K that
is not a whole number of four-chunk loop bodies (chunks past the end computed with zero
scales), bias, the 8-wave tile, at most 64 rows (64-row tiles, K split over workgroups), and
the 64-row tiles that run two workgroups per CU where 128-row tiles are too few.  Tolerance (BASELINE): max|y - y_ref| / max|y_ref| <= 1e-3."""
import numpy as np
import pytest

import synth
from linear_cases import build, oracle_forward, oracle_weight, product, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3

CASES = [
    # fmt, N, K, M, dtype, bias
    ("gptq4", 9616, 1408, 520, "bf16", True),    # 11 chunks: one zero-scale chunk; ragged M, N
    ("gptq8", 9600, 2048, 520, "bf16", False),   # 8-bit codes (2 steps per chunk)
    ("mxfp4", 9616, 1024, 520, "bf16", True),    # e2m1 with block and column exponents
    ("gptq4", 7696, 2048, 300, "f32", True),     # f32 rows: hi + lo pieces on 64-row tiles
    ("awq4", 8000, 1024, 2000, "bf16", False),   # 16 x 21 tiles of 384 columns: 8 waves
    # at most 64 rows: 64-row tiles, K split over workgroups, k_splitk_reduce adds the slices
    ("gptq4", 4000, 4096, 40, "bf16", True),     # 21 column blocks (ragged), K in 8 slices
    ("gptq4", 4000, 2048, 64, "f32", True),      # f32 rows on the 64-row tile
    ("mxfp4", 3000, 1408, 33, "bf16", True),     # 11 chunks over the slices, e2m1
    ("mxfp4", 7700, 1024, 4100, "bf16", True),   # 33 x 21 tiles of 384 columns: 8 waves, e2m1
    # too few 128-row tiles, enough 64-row ones: 64 x 192 tiles, two workgroups per CU
    ("gptq4", 7000, 2048, 300, "bf16", True),    # 5 x 37 tiles, ragged M and N
    ("gptq8", 6000, 1024, 350, "bf16", False),   # 8-bit codes
    ("mxfp4", 9000, 1408, 250, "bf16", True),    # e2m1, 11 chunks
]


@pytest.mark.parametrize("fmt,N,K,M,dt,bias", CASES)
def test_gemm_dma_shapes(orc, fmt, N, K, M, dt, bias):
    import torch
    kind, a = build(fmt, N, K, seed=7)
    ql = product(kind, a, N, K)
    W = oracle_weight(orc, kind, a, N, K)
    A = synth.normal(0x5EED0DA0 + M, (M, K))
    b = synth.normal(0x5EED0DA1, (N,)) if bias else None
    if dt == "bf16":
        Ab = synth.bf16_bits_to_f32(synth.to_bf16_bits(A))
        tA = torch.from_numpy(Ab).cuda().to(torch.bfloat16)
    else:
        Ab, tA = A, torch.from_numpy(A).cuda()
    tb = torch.from_numpy(b).cuda() if bias else None
    print(f"[gpu] gemm dma {fmt} [{N},{K}] M={M} {dt} bias={bias}", flush=True)
    y = ql.forward(tA, bias=tb).cpu().numpy()
    ref = oracle_forward(orc, kind, a, W, Ab, b)
    e = rel_err(y, ref)
    print(f"[gpu]   max rel err {e:.3e}", flush=True)
    assert e <= TOL, e
    # repeat: identical (no atomics in the tile, fixed order)
    y2 = ql.forward(tA, bias=tb).cpu().numpy()
    assert np.array_equal(y, y2)
