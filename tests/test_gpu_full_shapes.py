"""Parity at the BASELINE configurations' own shapes (configs 1-4): the product forward
against the reference CPU path (oracle dequant + sgl_matmul_nt, or sgl_matmul_w8a16 for W8)
on the same seeded inputs, every row compared.  Tolerance (BASELINE): max|y - y_ref| /
max|y_ref| <= 1e-3.  Each case prints its measured error; with SGLQ_PARITY_LOG set, the
errors are also appended to that file (one JSON object per case)."""
import json
import os

import numpy as np
import pytest

import synth
from linear_cases import build, oracle_forward, oracle_weight, product, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
_cache = {}


def _weight(orc, fmt, N, K, seed):
    key = (fmt, N, K, seed)
    if key not in _cache:
        _cache.clear()  # one full-size weight at a time
        kind, a = build(fmt, N, K, seed=seed)
        _cache[key] = (kind, a, product(kind, a, N, K), oracle_weight(orc, kind, a, N, K))
    return _cache[key]


def _case(orc, fmt, N, K, M, dt, seed):
    import torch
    kind, a, ql, W = _weight(orc, fmt, N, K, seed)
    A = synth.normal(seed + 1000 + M, (M, K))
    if dt == "bf16":
        Ab = synth.bf16_bits_to_f32(synth.to_bf16_bits(A))
        tA = torch.from_numpy(Ab).cuda().to(torch.bfloat16)
    else:
        Ab, tA = A, torch.from_numpy(A).cuda()
    print(f"[gpu] full shape {fmt} [{N},{K}] M={M} {dt}", flush=True)
    y = ql.forward(tA).cpu().numpy()
    ref = oracle_forward(orc, kind, a, W, Ab)
    e = rel_err(y, ref)
    print(f"[gpu]   max rel err {e:.3e}", flush=True)
    log = os.environ.get("SGLQ_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"fmt": fmt, "N": N, "K": K, "M": M, "dtype": dt,
                                "max_rel_err": e}) + "\n")
    assert e <= TOL, (fmt, N, K, M, dt, e)


@pytest.mark.parametrize("M", [1, 8])
def test_config1_w8(orc, M):
    """W8 per-channel [4864, 896] (Qwen2.5-0.5B MLP), f32 rows."""
    _case(orc, "w8", 4864, 896, M, "f32", 0x5EED0001)


@pytest.mark.parametrize("N,K", [(11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_config2_gptq_decode(orc, N, K, M, dt):
    """GPTQ int4 g128 decode, gate/up [11008, 4096] and down [4096, 11008]."""
    _case(orc, "gptq4", N, K, M, dt, 0x5EED0002)


@pytest.mark.parametrize("fmt", ["gptq4", "awq4", "gptq4_act", "marlin4_asym"])
@pytest.mark.parametrize("M", [64, 512, 2048])
def test_config3_prefill(orc, fmt, M):
    """Prefill GEMM at [11008, 4096], bf16 rows: GPTQ, AWQ (gemm layout), GPTQ act-order and
    the Marlin layout, through the 128 x 64 (M = 512) and 256 x 128 (M = 2048) tilings."""
    _case(orc, fmt, 11008, 4096, M, "bf16", 0x5EED0003)


@pytest.mark.parametrize("M", [512, 2048])
def test_config3_prefill_long_k(orc, M):
    """The down shape [4096, 11008]: the longest K, where the prescaled f16 weights of the
    LDS kernel accumulate the most rounding."""
    _case(orc, "gptq4", 4096, 11008, M, "bf16", 0x5EED0004)


@pytest.mark.parametrize("M", [1, 16, 512])
def test_config4_mxfp4(orc, M):
    """MXFP4 [8192, 8192], bf16 rows: decode GEMV (M = 1, 16) and prefill GEMM (M = 512)."""
    _case(orc, "mxfp4", 8192, 8192, M, "bf16", 0x5EED0005)
