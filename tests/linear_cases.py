"""Shared builders for the forward-parity tests: one synthetic weight per format, packed the
way the reference loader receives it, plus its oracle dequant (f32 [N, K])."""
import numpy as np

import synth
from oracle.oracle import make_cfg as ocfg


def build(fmt, N, K, seed=1, G=128):
    """Returns (kind, args dict, oracle-side callable producing f32 W)."""
    W = synth.normal(seed, (N, K), 0.02)
    if "_g" in fmt and fmt.rsplit("_g", 1)[1].isdigit():  # e.g. gptq4_g32: other group size
        fmt, G = fmt.rsplit("_g", 1)[0], int(fmt.rsplit("_g", 1)[1])
    if fmt in ("gptq4", "gptq4_act", "gptq4_v2", "gptq4_noz", "gptq8", "gptq4_row"):
        bits = 8 if fmt == "gptq8" else 4
        gi = synth.act_order_gidx(seed + 1, K, G) if fmt == "gptq4_act" else None
        Ge = 0 if fmt == "gptq4_row" else G
        c, z, s = synth.quantize_groups(W, Ge, bits=bits, g_idx=gi)
        pack = 32 // bits
        Kp = -(-K // pack) * pack
        cp = np.zeros((N, Kp), np.uint8)
        cp[:, :K] = c
        qw, qz = synth.gptq_pack(cp, z, bits=bits, v2=fmt == "gptq4_v2")
        if fmt == "gptq4_noz":
            qz = None
        cfg = dict(method=2, bits=bits, group_size=-1 if fmt == "gptq4_row" else G, zero_point=1,
                   desc_act=int(gi is not None), v2=int(fmt == "gptq4_v2"))
        return "awq_gptq", dict(cfg=cfg, qweight=qw, scales=s, qzeros=qz, g_idx=gi)
    if fmt in ("awq4", "awq4_gemv", "awq4_noz"):
        c, z, s = synth.quantize_groups(W, G)
        qw, qz = synth.awq_pack(c, z, transposed=fmt == "awq4_gemv")
        cfg = dict(method=1, bits=4, group_size=G, zero_point=int(fmt != "awq4_noz"),
                   transposed=int(fmt == "awq4_gemv"))
        return "awq_gptq", dict(cfg=cfg, qweight=qw, scales=s,
                                qzeros=None if fmt == "awq4_noz" else qz, g_idx=None)
    if fmt.startswith("marlin"):
        bits = 8 if "8" in fmt else 4
        withz = fmt.endswith("asym")
        c, z, s = synth.quantize_groups(W, G, bits=bits, sym=not withz)
        qw, qz, sc = synth.marlin_pack(c, z, s, bits=bits, with_zeros=withz)
        cfg = dict(method=2, bits=bits, group_size=G, zero_point=1, layout=1)
        return "marlin", dict(cfg=cfg, qweight=qw, scales=sc, qzeros=qz, natural=(c, z, s))
    if fmt in ("ct4", "ct8"):
        bits = 4 if fmt == "ct4" else 8
        half = 1 << (bits - 1)
        ng = -(-K // G)
        Wp = np.zeros((N, ng * G), np.float32)
        Wp[:, :K] = W
        sc = (np.abs(Wp).reshape(N, ng, G).max(axis=2) / (half - 1)).astype(np.float16)
        sc = np.maximum(sc.astype(np.float32), 1e-6).astype(np.float16).astype(np.float32)
        sq = np.clip(np.round(Wp / np.repeat(sc, G, axis=1)), -half, half - 1).astype(np.int32)
        wp = synth.ct_pack(sq, bits)
        cfg = dict(method=3, bits=bits, group_size=G, offset=half, packed_dim=1)
        return "ct", dict(cfg=cfg, wpacked=wp, scales=sc)
    if fmt == "mxfp4":
        Kp = -(-K // 32) * 32
        Wp = np.zeros((N, Kp), np.float32)
        Wp[:, :K] = W
        blocks, scales = synth.mxfp4_quantize(Wp)
        return "mxfp4", dict(blocks=blocks, scales=scales)
    if fmt == "w8":
        q, s = synth.quant_rows_i8(W)
        return "w8", dict(W8=q, sw=s)
    raise ValueError(fmt)


def product(kind, a, N, K):
    import sgl_qlinear as q
    if kind == "awq_gptq":
        return q.QLinear.from_awq_gptq(q.make_cfg(**a["cfg"]), a["qweight"], a["scales"], N, K,
                                       qzeros=a["qzeros"], g_idx=a["g_idx"])
    if kind == "marlin":
        return q.QLinear.from_marlin(q.make_cfg(**a["cfg"]), a["qweight"], a["scales"], N, K,
                                     qzeros=a["qzeros"])
    if kind == "ct":
        return q.QLinear.from_ct(q.make_cfg(**a["cfg"]), a["wpacked"], a["scales"], N, K)
    if kind == "mxfp4":
        return q.QLinear.from_mxfp4(a["blocks"], a["scales"], N, K)
    return q.QLinear.from_w8(a["W8"], a["sw"])


def oracle_weight(orc, kind, a, N, K):
    if kind == "awq_gptq":
        rc, W = orc.dequant(ocfg(**a["cfg"]), a["qweight"], a["scales"], N, K, qzeros=a["qzeros"],
                            g_idx=a["g_idx"])
    elif kind == "marlin":
        rc, W = orc.dequant_marlin(ocfg(**a["cfg"]), a["qweight"], a["scales"], N, K,
                                   qzeros=a["qzeros"])
    elif kind == "ct":
        rc, W = orc.dequant_ct(ocfg(**a["cfg"]), a["wpacked"], a["scales"], N, K)
    elif kind == "mxfp4":
        rc, W = orc.dequant_mxfp4(a["blocks"], a["scales"], N, K)
    else:
        return None
    assert rc == 0
    return W


def oracle_forward(orc, kind, a, W, A, bias=None):
    """The reference CPU path: W8 -> sgl_matmul_w8a16; otherwise dequant + sgl_matmul_nt."""
    if kind == "w8":
        return orc.matmul_w8a16(A, a["W8"], a["sw"], bias)
    return orc.matmul_nt(A, W, bias)


def rel_err(y, ref):
    """max |y - ref| / max |ref|  (the tolerance metric for every forward test: <= 1e-3)"""
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))
