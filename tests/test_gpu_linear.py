"""Forward parity on the GPU: sgl_qlinear_forward against the reference CPU path (the oracle's
dequant + sgl_matmul_nt, or sgl_matmul_w8a16 for W8) on the same seeded inputs.
Tolerance (BASELINE): max|y - y_ref| / max|y_ref| <= 1e-3."""
import numpy as np
import pytest

import synth
from linear_cases import build, oracle_forward, oracle_weight, product, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3

FORMATS = ["gptq4", "gptq4_act", "gptq4_v2", "gptq4_noz", "gptq4_row", "gptq8", "awq4",
           "awq4_gemv", "awq4_noz", "marlin4_asym", "marlin4_sym", "marlin8_asym", "marlin8_sym",
           "ct4", "ct8", "mxfp4", "w8", "gptq4_g32", "gptq4_g64", "awq4_g256", "gptq8_g32",
           "ct4_g64"]


def _run(orc, fmt, N, K, Ms, dtypes=("f32", "bf16"), bias=False, seed=3):
    import torch
    kind, a = build(fmt, N, K, seed=seed)
    ql = product(kind, a, N, K)
    W = oracle_weight(orc, kind, a, N, K)
    b = synth.normal(seed + 7, N, 0.1) if bias else None
    for M in Ms:
        A = synth.normal(seed + 100 + M, (M, K))
        for dt in dtypes:
            if dt == "bf16":
                Ab = synth.bf16_bits_to_f32(synth.to_bf16_bits(A))
                tA = torch.from_numpy(Ab).cuda().to(torch.bfloat16)
            elif dt == "f16":
                Ab = A.astype(np.float16).astype(np.float32)
                tA = torch.from_numpy(Ab).cuda().to(torch.float16)
            else:
                Ab = A
                tA = torch.from_numpy(A).cuda()
            print(f"[gpu] forward {fmt} N={N} K={K} M={M} {dt}", flush=True)
            tb = None if b is None else torch.from_numpy(b).cuda()
            y = ql.forward(tA, bias=tb).cpu().numpy()
            ref = oracle_forward(orc, kind, a, W, Ab, b)
            e = rel_err(y, ref)
            assert e <= TOL, (fmt, M, dt, e)
    return ql


@pytest.mark.parametrize("fmt", FORMATS)
def test_small_shapes(orc, fmt):
    N, K = (256, 1024) if not fmt.startswith("gptq4_row") else (80, 1000)
    _run(orc, fmt, N, K, [1, 3, 16, 17, 64, 100])


def test_dtypes_and_bias(orc):
    _run(orc, "gptq4", 128, 512, [1, 7], dtypes=("f32", "bf16", "f16"), bias=True)
    _run(orc, "w8", 128, 512, [2], dtypes=("f32", "f16"), bias=True)


def test_ragged_n_and_k(orc):
    # N not a multiple of 16 and K not a multiple of 128: padded tiles must not leak
    _run(orc, "gptq4", 72, 384, [1, 5])
    _run(orc, "mxfp4", 40, 160, [1, 3])
    _run(orc, "w8", 50, 100, [1, 9])


def test_marlin_equals_natural(orc):
    """A Marlin repack of identical codes gives the identical device result (bit for bit)."""
    import torch
    import sgl_qlinear as q
    kind, a = build("marlin4_asym", 256, 1024, seed=11)
    mar = product(kind, a, 256, 1024)
    c, z, s = a["natural"]
    qw, qz = synth.gptq_pack(c, z)
    nat = q.QLinear.from_awq_gptq(q.make_cfg(method=2, bits=4, group_size=128, zero_point=1), qw,
                                  s, 256, 1024, qzeros=qz)
    A = torch.from_numpy(synth.normal(12, (8, 1024))).cuda()
    assert torch.equal(mar.forward(A), nat.forward(A))
    assert torch.equal(mar.dequant(), nat.dequant())


@pytest.mark.parametrize("fmt", ["gptq4", "awq4", "mxfp4", "w8", "gptq8"])
def test_prefill_split_over_k(orc, fmt):
    """Prefill GEMM tilings at K = 4096 and ragged N: 64 x 128 tiles split 6 ways over K
    (M <= 64), 128 x 64 tiles split 3 ways (M = 100) and unsplit (M = 200); slice partials are
    reduced in order."""
    _run(orc, fmt, 1000, 4096, [33, 64, 100, 200], dtypes=("bf16",), bias=True)


@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4", "gptq8", "awq4_gemv"])
def test_prefill_large_tiles(orc, fmt):
    """256 x 128 tiles (M >= 1024) with ragged M and N, and the M boundaries between the
    tilings (64 / 65, 1023 / 1024) and between GEMV and GEMM (16 / 17)."""
    _run(orc, fmt, 1000, 1024, [16, 17, 65, 1023, 1030], dtypes=("bf16",), bias=True)


def test_prefill_large_tiles_f32(orc):
    """f32 activations (two A pieces) through every tiling."""
    _run(orc, "gptq4", 520, 1024, [40, 300, 1100], dtypes=("f32",))


@pytest.mark.parametrize("fmt", ["gptq4", "gptq4_act", "gptq8", "mxfp4", "w8", "gptq4_row"])
def test_gemv_rows_long_k(orc, fmt):
    """Decode GEMV of 8-16 rows over a long K: eight tiles per workgroup with up to 128 KiB of
    staging (one workgroup per CU) and eight activation items held per thread; the K range
    split over workgroups with partial sums; ragged N."""
    K = 8192 if fmt == "mxfp4" else 11008 if fmt != "gptq4_row" else 11000
    _run(orc, fmt, 200, K, [8, 12, 16], bias=True)


def test_prefill_prep_fallbacks(orc):
    """Activation prep paths other than the one-launch row prep: rows whose byte length is not
    a multiple of 16 (K = 100, 16-bit and f32 activations) and K beyond what one workgroup
    holds in registers (K = 33024 > 32768), both through the two-launch exponent + operand
    prep."""
    _run(orc, "w8", 50, 100, [20, 70])
    _run(orc, "gptq4", 48, 33024, [17, 70], bias=True)


def test_graph_replay_matches_eager(orc):
    """Split-K arrival counters reset themselves: repeated graph replays, with eager work and
    synchronisations between them, all equal the eager result bit for bit."""
    import torch
    kind, a = build("gptq4", 4096, 11008, seed=21)
    ql = product(kind, a, 4096, 11008)
    A = torch.from_numpy(synth.normal(22, (1, 11008))).cuda()
    ref = ql.forward(A).clone()
    out = torch.empty_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ql.forward(A, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ql.forward(A, out=out)
    for i in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        assert torch.equal(ql.forward(A), ref)


def test_deterministic_split_k(orc):
    """Two launches on the same input give bit-identical outputs (no atomics on C)."""
    import torch
    kind, a = build("gptq4", 4096, 11008, seed=23)
    ql = product(kind, a, 4096, 11008)
    for M in (16, 64, 256):
        A = torch.from_numpy(synth.normal(24, (M, 11008))).cuda()
        assert torch.equal(ql.forward(A), ql.forward(A)), M


@pytest.mark.parametrize("fmt", ["gptq4", "gptq4_act", "mxfp4", "w8", "gptq8"])
def test_gemv_split_rows(orc, fmt):
    """17-32 rows (f32) and 17-24 rows (16-bit activations) run as two decode GEMVs, rows 0-15
    and the rest, on offset A / C; the rows either side of both limits take the GEMM."""
    _run(orc, fmt, 200, 4096, [17, 20, 24, 25, 32, 33], dtypes=("f32", "bf16", "f16"),
         bias=True)


@pytest.mark.parametrize("fmt", ["gptq4", "gptq4_g32", "gptq8", "w8", "mxfp4", "awq4", "ct4_g64",
                                 "gptq4_noz"])
def test_gemv_one_row_wave_staging(orc, fmt):
    """One row takes the wave-staged GEMV (each wave stages its own K slice and power of two)
    with the slice length of the one-row plan: 4 chunks up to 32 chunks (K = 2200 with a partial
    last chunk, 4096), 8 up to 64 (6000, 8192; 8-bit codes 4096), 12 over 65-96 chunks of 4-bit
    codes (11008), and 4 on two tiles with K split over workgroups beyond (16384; 8-bit codes
    5120, 11008);
    ragged N, bias, every activation dtype."""
    u8 = fmt in ("gptq8", "w8")
    for K in ([2176, 4096, 8192, 11008, 16384] if fmt == "mxfp4" else
              [2200, 4096, 5120, 11008] if u8 else [2200, 4096, 6000, 8192, 11008, 16384]):
        _run(orc, fmt, 200, K, [1], dtypes=("f32", "bf16", "f16"), bias=True)


@pytest.mark.parametrize("fmt", ["gptq4", "gptq8", "w8", "mxfp4", "gptq4_g32"])
def test_gemv_two_rows_wave_staging(orc, fmt):
    """Two rows over K of 17-32 chunks take the two-row wave-staged GEMV (one workgroup
    range; a partial last chunk at K = 2200); three rows and a longer K stay on k_gemv."""
    for K in ([2176, 4096] if fmt == "mxfp4" else [2200, 4096, 5000]):
        _run(orc, fmt, 200, K, [2, 3], dtypes=("f32", "bf16", "f16"), bias=True)
