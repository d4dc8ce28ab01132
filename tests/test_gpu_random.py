"""Seeded random shapes through sgl_qlinear_forward against the oracle (dequant + the
reference's f32 matmul, reference src/ops.c:243-279): formats, ragged N and K, every decode
and prefill plan (M from 1 to 300 crosses the GEMV / GEMM boundary and the GEMM tilings), f32 /
bf16 / f16 activations, with and without bias.  Tolerance: max|y - y_ref| / max|y_ref| <= 1e-3.
Each case prints its parameters before it runs, so a failure names it."""
import numpy as np
import pytest

import synth
from linear_cases import build, oracle_forward, oracle_weight, product, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
FMTS = ["gptq4", "gptq4_act", "gptq8", "gptq4_g32", "gptq4_v2", "gptq4_row", "awq4",
        "awq4_gemv", "awq4_noz", "marlin4_asym", "marlin4_sym", "marlin8_sym", "ct4", "ct8",
        "ct4_g64", "mxfp4", "w8", "gptq8_g32"]
MS = [1, 2, 5, 8, 9, 16, 17, 40, 64, 65, 130, 300]


def _cases(n, seed=0x5EED0900):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = FMTS[i % len(FMTS)]
        N = int(rng.integers(16, 700))
        K = int(rng.integers(32, 3000))
        if fmt.startswith("awq") or fmt.startswith("gptq"):  # zeros packed 8 (4) per word
            N = -(-N // 8) * 8
        if fmt.startswith("marlin"):
            N, K = -(-N // 64) * 64, -(-K // 16) * 16
        M = int(rng.choice(MS))
        while M * N * K > 2e8 and M > 1:
            M //= 2
        dt = ["f32", "bf16", "f16"][int(rng.integers(0, 3))]
        out.append((fmt, N, K, M, dt, bool(rng.integers(0, 2)), 1000 + i))
    return out


@pytest.mark.parametrize("case", _cases(72), ids=lambda c: "-".join(map(str, c[:5])))
def test_random_shape(orc, case):
    import torch
    fmt, N, K, M, dt, bias, seed = case
    print(f"[gpu] random case {case}", flush=True)
    kind, a = build(fmt, N, K, seed=seed)
    ql = product(kind, a, N, K)
    W = oracle_weight(orc, kind, a, N, K)
    A = synth.normal(seed + 1, (M, K))
    if dt == "bf16":
        Ab = synth.bf16_bits_to_f32(synth.to_bf16_bits(A))
        tA = torch.from_numpy(Ab).cuda().to(torch.bfloat16)
    elif dt == "f16":
        Ab = A.astype(np.float16).astype(np.float32)
        tA = torch.from_numpy(Ab).cuda().to(torch.float16)
    else:
        Ab = A
        tA = torch.from_numpy(A).cuda()
    b = synth.normal(seed + 2, N, 0.1) if bias else None
    y = ql.forward(tA, bias=None if b is None else torch.from_numpy(b).cuda()).cpu().numpy()
    e = rel_err(y, oracle_forward(orc, kind, a, W, Ab, b))
    assert e <= TOL, (case, e)


def _moe_cases(n, seed=0x5EED0A00):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = ["gptq4", "mxfp4", "gptq8"][i % 3]
        n_exp = int(rng.integers(2, 12))
        E = int(rng.integers(2, 12)) * 64
        mi = int(rng.integers(2, 20)) * 16
        T = int(rng.choice([1, 2, 3, 4, 7, 33, 90]))
        k = int(rng.integers(1, min(n_exp, 4) + 1))
        dt = ["f32", "bf16"][int(rng.integers(0, 2))]
        out.append((fmt, n_exp, E, mi, T, k, dt, 2000 + 10 * i))
    return out


@pytest.mark.parametrize("case", _moe_cases(12), ids=lambda c: "-".join(map(str, c[:7])))
def test_random_moe(orc, case):
    """Routed-expert FFN (reference src/deepseek.c:655-677) at seeded random sizes: decode
    (T <= 4, grouped GEMV) and prefill (grouped GEMM) with ragged expert blocks."""
    from test_gpu_moe import _check
    fmt, n_exp, E, mi, T, k, dt, seed = case
    print(f"[gpu] random moe {case}", flush=True)
    _check(orc, n_exp, E, mi, T, k, seed, dtypes=(dt,), fmt=fmt)


def _route_cases(n, seed=0x5EED0B00):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        ne = int(rng.choice([2, 4, 8, 16, 24, 32, 64, 96, 128, 160, 256]))
        divs = [g for g in (0, 2, 4, 8) if g == 0 or (ne % g == 0 and ne // g >= 2)]
        ng = int(rng.choice(divs))
        tg = int(rng.integers(1, ng + 1)) if ng else 0
        cap = ne if not ng else tg * (ne // ng)
        k = int(rng.integers(1, min(cap, 8) + 1))
        out.append((ne, k, bool(rng.integers(0, 2)), ng, tg, bool(rng.integers(0, 2)),
                    bool(rng.integers(0, 2)), float(rng.choice([1.0, 2.5])), 3000 + i))
    return out


@pytest.mark.parametrize("case", _route_cases(24), ids=lambda c: "-".join(map(str, c[:7])))
def test_random_route(orc, case):
    """Routing (reference src/deepseek.c:593-633) at seeded random expert counts, group
    limits, top-k, sigmoid / softmax, correction bias, normalisation and scale: ids bit-exact,
    weights within 2e-6 relative."""
    import torch
    import sgl_qlinear as q
    ne, k, sig, ng, tg, bias, norm, scale, seed = case
    print(f"[gpu] random route {case}", flush=True)
    rng = np.random.default_rng(seed)
    lg = (rng.standard_normal((int(rng.integers(1, 70)), ne)) * 2).astype(np.float32)
    b = (rng.standard_normal(ne) * 0.1).astype(np.float32) if bias else None
    ids, w = q.qmoe_route(torch.from_numpy(lg).cuda(), k,
                          None if b is None else torch.from_numpy(b).cuda(), sig, ng, tg, norm,
                          scale)
    rid, rw = orc.moe_route(lg, k, b, sig, ng, tg, norm, scale)
    assert np.array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=0)
