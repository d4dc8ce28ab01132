"""Routed-expert FFN on the GPU (sgl_qmoe_forward) against the reference CPU composition
(oracle: dequant every expert, then reference src/deepseek.c:655-677 per token and slot).
Tolerance: max|y - y_ref| / max|y_ref| <= 1e-3."""
import numpy as np
import pytest

import synth
from linear_cases import rel_err
from oracle.oracle import make_cfg as ocfg

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _experts(orc, n_exp, E, mi, seed, fmt="gptq4", std=0.02):
    import sgl_qlinear as q
    from linear_cases import build, oracle_weight, product
    cfg = dict(method=2, bits=4, group_size=128, zero_point=1)
    gu, dn, wgu, wdn = [], [], [], []
    for e in range(n_exp):
        for (N, K, lst, wl, sd) in ((2 * mi, E, gu, wgu, seed + 2 * e),
                                    (E, mi, dn, wdn, seed + 2 * e + 1)):
            if fmt == "gptq4":
                c, z, s = synth.quantize_groups(synth.normal(sd, (N, K), std), 128)
                qw, qz = synth.gptq_pack(c, z)
                lst.append(q.QLinear.from_awq_gptq(q.make_cfg(**cfg), qw, s, N, K, qzeros=qz))
                rc, W = orc.dequant(ocfg(**cfg), qw, s, N, K, qzeros=qz)
                assert rc == 0
            else:
                kind, a = build(fmt, N, K, seed=sd)
                lst.append(product(kind, a, N, K))
                W = oracle_weight(orc, kind, a, N, K)
            wl.append(W)
    return gu, dn, wgu, wdn


def _check(orc, n_exp, E, mi, T, k, seed, dtypes=("bf16", "f32"), drop=False, fmt="gptq4",
           std=0.02, repeat=False):
    import torch
    import sgl_qlinear as q
    gu, dn, wgu, wdn = _experts(orc, n_exp, E, mi, seed, fmt, std)
    ids, wts = synth.moe_routing(seed + 999, T, n_exp, k)
    if drop == "all":  # no routed slot at all: the output is zero
        ids[:] = -1
    elif drop:  # unrouted slots (id -1) are skipped
        ids[::3, -1] = -1
    if repeat:  # every token lists token 0's first expert in its first two slots
        ids[:, :2] = ids[0, 0]
    h = synth.normal(seed + 1000, (T, E))
    for dt in dtypes:
        if dt == "bf16":
            hb = synth.bf16_bits_to_f32(synth.to_bf16_bits(h))
            th = torch.from_numpy(hb).cuda().to(torch.bfloat16)
        elif dt == "f16":
            hb = h.astype(np.float16).astype(np.float32)
            th = torch.from_numpy(hb).cuda().to(torch.float16)
        else:
            hb, th = h, torch.from_numpy(h).cuda()
        print(f"[gpu] moe {fmt} n_exp={n_exp} E={E} mi={mi} T={T} k={k} {dt}", flush=True)
        y = q.qmoe_forward(gu, dn, th, torch.from_numpy(ids).cuda(),
                           torch.from_numpy(wts).cuda()).cpu().numpy()
        ref = orc.moe_ffn(hb, wgu, wdn, ids, wts)
        e = rel_err(y, ref)
        print(f"[gpu]   max rel err {e:.3e}", flush=True)
        assert e <= TOL, (dt, e)
        y2 = q.qmoe_forward(gu, dn, th, torch.from_numpy(ids).cuda(),
                            torch.from_numpy(wts).cuda()).cpu().numpy()
        assert np.array_equal(y, y2), "MoE forward is not deterministic"


def test_moe_small(orc):
    _check(orc, 8, 256, 128, 20, 2, seed=31)


def test_moe_unrouted_slots(orc):
    _check(orc, 6, 256, 256, 9, 3, seed=41, dtypes=("f32",), drop=True)


def test_moe_prefill_mxfp4(orc):
    """MXFP4 experts: the fused SwiGLU epilogue applies the gate and up column exponents."""
    _check(orc, 8, 256, 128, 40, 2, seed=61, fmt="mxfp4")


def test_moe_prefill_gptq8_ragged(orc):
    """8-bit experts (2-step chunks) with an intermediate size of 11 tiles and a hidden size of
    24 tiles: the last column block of the gate/up pairs and of the down output is partial."""
    _check(orc, 6, 384, 176, 40, 2, seed=81, fmt="gptq8")


def test_moe_prefill_unfused(orc):
    """Group scales below 2^-14 cannot prescale f16 codes: those experts take the register
    unpack GEMM, with SwiGLU formed by its own operand prep."""
    _check(orc, 8, 256, 128, 40, 2, seed=71, std=2e-5)


def test_moe_decode_batch_f32(orc):
    """Decode batches (T <= 4) take the grouped-GEMV path; f32 and bf16 tokens."""
    _check(orc, 16, 512, 256, 3, 4, seed=51)


def test_moe_decode_deepseek_shape(orc):
    """BASELINE config 5, decode: one token, 6 of 64 experts, hidden 2048, inter 1408."""
    _check(orc, 64, 2048, 1408, 1, 6, seed=0x5EED0005, dtypes=("bf16",))


def test_moe_prefill_deepseek_shape(orc):
    """BASELINE config 5, prefill: 512 tokens, top-6 of 64 experts, hidden 2048, inter 1408."""
    _check(orc, 64, 2048, 1408, 512, 6, seed=0x5EED0005, dtypes=("bf16",))


@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4", "gptq8"])
def test_moe_decode_one_token(orc, fmt):
    """One token: segments straight from the routing (no routing launch), one row per slot.
    GPTQ4 (f16 scales, one group per chunk) takes the grouped one-row kernel, MXFP4 and GPTQ8
    (two chunks per group) the grouped wave-staged kernel: token rows gathered for gate/up,
    SwiGLU rows formed while loading for down, and the weighted combine done by the last slot
    of each tile; with and without unrouted slots, and with none routed at all (zero
    output)."""
    _check(orc, 8, 512, 256, 1, 3, seed=91, fmt=fmt)
    _check(orc, 6, 256, 384, 1, 4, seed=93, fmt=fmt, dtypes=("f32",), drop=True)
    _check(orc, 4, 256, 128, 1, 2, seed=95, fmt=fmt, dtypes=("bf16",), drop="all")


def test_moe_decode_one_token_many_slots(orc):
    """One token routed to 10 experts: more slots than the in-workgroup combine holds (8), so
    the down launch keeps one workgroup per (tile, slot) and the last slot of each tile
    combines; with and without unrouted slots."""
    _check(orc, 16, 256, 128, 1, 10, seed=97)
    _check(orc, 16, 256, 128, 1, 10, seed=98, dtypes=("f32",), drop=True)


def test_moe_decode_one_token_u8_g64(orc):
    """One token over 8-bit experts with 64-element groups (one group per 64-element chunk):
    both launches take the grouped one-row kernel's 8-bit form."""
    _check(orc, 8, 512, 256, 1, 4, seed=99, fmt="gptq8_g64")
    _check(orc, 8, 512, 256, 1, 4, seed=100, fmt="gptq8_g64", dtypes=("f32",), drop=True)



@pytest.mark.parametrize("T", [2, 4])
@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4", "gptq8"])
def test_moe_decode_tokens(orc, T, fmt):
    """2 and 4 tokens: routing launch, grouped wave-staged GEMVs over the experts' row blocks
    (at most T rows each), then the combine; with and without unrouted slots, and with none
    routed at all."""
    _check(orc, 8, 512, 256, T, 3, seed=101 + T, fmt=fmt)
    _check(orc, 6, 256, 384, T, 4, seed=111 + T, fmt=fmt, dtypes=("f32",), drop=True)
    _check(orc, 4, 256, 128, T, 2, seed=121 + T, fmt=fmt, dtypes=("bf16",), drop="all")


@pytest.mark.parametrize("T", [1, 2, 4])
def test_moe_decode_repeated_experts(orc, T):
    """Tokens that list one expert twice (and share it): that expert has more pairs than
    there are tokens, so the routing cuts its rows into blocks of at most T rows, the rows the
    decode GEMVs stage.  (One token takes slot-per-segment launches where its weights allow.)"""
    _check(orc, 8, 256, 128, T, 3, seed=131 + T, repeat=True)


def test_moe_decode_deepseek_shape_four_tokens(orc):
    """BASELINE config 5, decode of four tokens (the bench's T = 4 line)."""
    _check(orc, 64, 2048, 1408, 4, 6, seed=0x5EED0006, dtypes=("bf16",))


def test_moe_decode_many_pairs(orc):
    """Four tokens of 20 slots (80 pairs: more row blocks than experts)."""
    _check(orc, 32, 256, 128, 4, 20, seed=141, dtypes=("f32",))


@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4"])
def test_moe_decode_one_token_repeated_experts(orc, fmt):
    """One token listing an expert twice on the launches that take segments straight from the
    routing (GPTQ4: the one-row kernel with the in-workgroup combine; MXFP4: the wave-staged
    kernel with the fused combine): each slot stays its own segment."""
    _check(orc, 8, 512, 256, 1, 3, seed=151, fmt=fmt, repeat=True)


def test_moe_prefill_repeated_experts(orc):
    """Prefill rows where every token lists one shared expert twice: that expert's 80 rows
    span two 64-row blocks."""
    _check(orc, 8, 256, 128, 40, 3, seed=161, repeat=True)


@pytest.mark.parametrize("T", [1, 3, 9])
def test_moe_single_expert(orc, T):
    """One expert, one slot per token: decode and prefill launches with a single segment."""
    _check(orc, 1, 256, 128, T, 1, seed=171 + T, dtypes=("f32",))


@pytest.mark.parametrize("T", [1, 4, 40])
def test_moe_one_intermediate_tile(orc, T):
    """An intermediate size of one 16-column tile (gate/up of two tiles, down K of 16)."""
    _check(orc, 4, 128, 16, T, 2, seed=181 + T, dtypes=("bf16",))


def test_moe_every_expert(orc):
    """Every token routed to every expert (k = n_exp): every segment holds every token."""
    _check(orc, 6, 256, 128, 2, 6, seed=191)
    _check(orc, 6, 256, 128, 20, 6, seed=192, dtypes=("f32",))


@pytest.mark.parametrize("T", [1, 3, 40])
@pytest.mark.parametrize("fmt", ["gptq4", "mxfp4"])
def test_moe_f16_tokens(orc, T, fmt):
    """f16 token rows: one token (slot-per-segment launches), a decode batch, and prefill."""
    _check(orc, 8, 512, 256, T, 3, seed=201 + T, fmt=fmt, dtypes=("f16",))


def test_moe_prefill_short_intermediate(orc):
    """An intermediate size of one tile (16) with 8-bit experts: the down products are too few
    to average the rounding of one-piece f16 operands (1.06e-3 on one piece), so below 256
    intermediate columns the down operands keep hi + lo pieces.  Found by a randomized sweep."""
    _check(orc, 17, 384, 16, 64, 4, seed=499866, fmt="gptq8", dtypes=("bf16",), repeat=True)
