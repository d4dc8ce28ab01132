"""Dequant parity on the GPU: every reference dequant entry point of the product (host API,
computed by HIP kernels) and the device twin sgl_qlinear_dequant must reproduce the reference's
golden vectors bit for bit."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, golden
from oracle.oracle import make_cfg as ocfg

pytestmark = pytest.mark.gpu

DEQUANT = sorted(f[8:-4] for f in os.listdir(GOLDEN) if f.startswith("dequant_"))


def cfg_from(arr):
    import sgl_qlinear as q
    return q.make_cfg(**dict(zip([n for n, _ in q.QCfg._fields_], [int(v) for v in arr])))


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("name", DEQUANT)
def test_host_api_dequant(name):
    import sgl_qlinear as q
    g = golden("dequant_" + name)
    print(f"[gpu] dequant {name}", flush=True)
    rc, out = q.qweight_dequant(cfg_from(g["cfg"]), g["qweight"], g["scales"], int(g["N"]),
                                int(g["K"]), qzeros=g.get("qzeros"), g_idx=g.get("g_idx"))
    assert rc == 0 and bits_equal(out, g["expected"])


@pytest.mark.parametrize("name", DEQUANT)
def test_device_twin_dequant(name):
    import sgl_qlinear as q
    g = golden("dequant_" + name)
    ql = q.QLinear.from_awq_gptq(cfg_from(g["cfg"]), g["qweight"], g["scales"], int(g["N"]),
                                 int(g["K"]), qzeros=g.get("qzeros"), g_idx=g.get("g_idx"))
    assert bits_equal(ql.dequant().cpu().numpy(), g["expected"])


@pytest.mark.parametrize("name", ["marlin4_asym", "marlin4_sym", "marlin8_asym", "marlin8_sym"])
def test_marlin(name):
    import sgl_qlinear as q
    g = golden(name)
    rc, out = q.qweight_dequant_marlin(cfg_from(g["cfg"]), g["qweight"], g["scales"],
                                       int(g["N"]), int(g["K"]), qzeros=g.get("qzeros"))
    assert rc == 0 and bits_equal(out, g["expected"])
    ql = q.QLinear.from_marlin(cfg_from(g["cfg"]), g["qweight"], g["scales"], int(g["N"]),
                               int(g["K"]), qzeros=g.get("qzeros"))
    assert bits_equal(ql.dequant().cpu().numpy(), g["expected"])


def test_marlin_unit_known_answers():
    import sgl_qlinear as q
    g = golden("marlin_unit")
    for name in g["names"]:
        p = str(name) + "_"
        cfg = q.make_cfg(method=1, bits=int(g[p + "bits"]), group_size=int(g[p + "G"]), layout=1)
        N, K = int(g[p + "N"]), int(g[p + "K"])
        qz = g[p + "qzeros"] if int(g[p + "has_z"]) else None
        rc, out = q.qweight_dequant_marlin(
            cfg, g[p + "qweight"], g[p + "scales"], N, K, qzeros=qz,
            shapes=dict(qw=(int(g[p + "qw_rows"]), int(g[p + "qw_cols"])),
                        qz=(int(g[p + "qz_rows"]), int(g[p + "qz_cols"])),
                        sc=(int(g[p + "sc_rows"]), N)))
        assert rc == 0
        assert np.abs(out.reshape(-1).astype(np.float64) - g[p + "expected"]).max() == 0.0, name


@pytest.mark.parametrize("bits", [4, 8])
def test_ct(bits):
    import sgl_qlinear as q
    g = golden(f"ct{bits}")
    rc, out = q.qweight_dequant_ct(cfg_from(g["cfg"]), g["wpacked"], g["scales"], int(g["N"]),
                                   int(g["K"]))
    assert rc == 0 and bits_equal(out, g["expected"])


@pytest.mark.parametrize("name", ["mxfp4", "mxfp4_ragged"])
def test_mxfp4(name):
    import sgl_qlinear as q
    g = golden(name)
    rc, out = q.qweight_dequant_mxfp4(g["blocks"], g["scales"], int(g["N"]), int(g["K"]))
    assert rc == 0 and bits_equal(out, g["expected"])


def test_mxfp4_exhaustive(orc):
    """All 16 codes x 256 e8m0 bytes, product vs oracle (incl. 255 -> 0, subnormal scales)."""
    import sgl_qlinear as q
    codes = np.arange(16)
    blocks = np.zeros((256, 16), np.uint8)
    blocks[:, :8] = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    scales = np.arange(256, dtype=np.uint8)[:, None]
    rc, out = q.qweight_dequant_mxfp4(blocks, scales, 256, 32)
    rc2, ref = orc.dequant_mxfp4(blocks, scales, 256, 32)
    assert rc == rc2 == 0 and bits_equal(out, ref)


def test_quant_i8_golden():
    import sgl_qlinear as q
    g = golden("quant_i8")
    s, qq = q.quant_rows_i8(g["X"])
    assert np.array_equal(qq, g["q"]) and bits_equal(s, g["s"])
    s, qq = q.quant_rows_i8(g["Xr"])
    assert np.array_equal(qq, g["qr"]) and bits_equal(s, g["sr"])
    s1, q1 = q.quant_row_i8(g["X"][2])
    assert bits_equal(s1, g["s"][2]) and np.array_equal(q1, g["q"][2])
    for i in range(4):
        assert bits_equal(q.dequant_row_i8(g["qr"][i], g["sr"][i]), g["dq"][i])


def test_quant_i8_full_size(orc):
    """BASELINE config 1 weights [4864, 896] N(0, 0.02): codes and scales bit-identical."""
    import synth
    import sgl_qlinear as q
    W = synth.normal(0x5EED0001, (4864, 896), 0.02)
    s, qq = q.quant_rows_i8(W)
    s2, q2 = orc.quant_rows_i8(W)
    assert np.array_equal(qq, q2) and bits_equal(s, s2)


def test_fresh_gptq_act_order_vs_oracle(orc):
    """A fresh act-order GPTQ weight at a non-trivial shape, bit-exact vs the oracle."""
    import synth
    import sgl_qlinear as q
    W = synth.normal(901, (96, 1024), 0.02)
    gi = synth.act_order_gidx(902, 1024, 128)
    c, z, s = synth.quantize_groups(W, 128, g_idx=gi)
    qw, qz = synth.gptq_pack(c, z)
    cfg = q.make_cfg(method=2, bits=4, group_size=128, zero_point=1, desc_act=1)
    rc, out = q.qweight_dequant(cfg, qw, s, 96, 1024, qzeros=qz, g_idx=gi)
    rc2, ref = orc.dequant(ocfg(method=2, bits=4, group_size=128, zero_point=1, desc_act=1), qw,
                           s, 96, 1024, qzeros=qz, g_idx=gi)
    assert rc == rc2 == 0 and bits_equal(out, ref)
