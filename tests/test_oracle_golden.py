"""The CPU oracle against the reference's golden vectors (bit-exact) and its known answers.

Golden vectors come from the reference's own compiled C (tests/golden/make_golden.py).  Known
answers are the inline cases of reference tests/test_qweight.c:130-225 and the Marlin file
reference tests/_marlin_unit.json (as tests/golden/marlin_unit.npz)."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, golden
from oracle.oracle import QCfg, have_reference, make_cfg, qcfg_from_json, Reference


def cfg_from(arr):
    c = QCfg()
    for (n, _), v in zip(QCfg._fields_, arr):
        setattr(c, n, int(v))
    return c


DEQUANT = sorted(f[8:-4] for f in os.listdir(GOLDEN) if f.startswith("dequant_"))


@pytest.mark.parametrize("name", DEQUANT)
def test_dequant_golden(orc, name):
    g = golden("dequant_" + name)
    rc, out = orc.dequant(cfg_from(g["cfg"]), g["qweight"], g["scales"], int(g["N"]),
                          int(g["K"]), qzeros=g.get("qzeros"), g_idx=g.get("g_idx"))
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))


@pytest.mark.parametrize("name", ["marlin4_asym", "marlin4_sym", "marlin8_asym", "marlin8_sym"])
def test_marlin_golden(orc, name):
    g = golden(name)
    rc, out = orc.dequant_marlin(cfg_from(g["cfg"]), g["qweight"], g["scales"], int(g["N"]),
                                 int(g["K"]), qzeros=g.get("qzeros"))
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))
    # closed form on the natural codes the packer started from: (q - z) * s, g = k / G
    q, z, s = g["codes"].astype(np.int64), g["zeros"].astype(np.int64), g["nat_scales"]
    G = int(g["cfg"][2])
    K = int(g["K"])
    gi = np.arange(K) // G
    bits = int(g["cfg"][1])
    zz = z[gi].T if "qzeros" in g else (1 << (bits - 1))
    ref = ((q - zz).astype(np.float32) * s[gi].T).astype(np.float32)
    assert np.array_equal(out, ref)


def test_marlin_unit_known_answers(orc):
    g = golden("marlin_unit")
    for name in g["names"]:
        p = str(name) + "_"
        cfg = make_cfg(method=1, bits=int(g[p + "bits"]), group_size=int(g[p + "G"]), layout=1)
        N, K = int(g[p + "N"]), int(g[p + "K"])
        qz = g[p + "qzeros"] if int(g[p + "has_z"]) else None
        rc, out = orc.dequant_marlin(
            cfg, g[p + "qweight"], g[p + "scales"], N, K, qzeros=qz,
            shapes=dict(qw=(int(g[p + "qw_rows"]), int(g[p + "qw_cols"])),
                        qz=(int(g[p + "qz_rows"]), int(g[p + "qz_cols"])),
                        sc=(int(g[p + "sc_rows"]), N)))
        assert rc == 0
        assert np.abs(out.reshape(-1).astype(np.float64) - g[p + "expected"]).max() == 0.0, name


@pytest.mark.parametrize("bits", [4, 8])
def test_ct_golden(orc, bits):
    g = golden(f"ct{bits}")
    rc, out = orc.dequant_ct(cfg_from(g["cfg"]), g["wpacked"], g["scales"], int(g["N"]),
                             int(g["K"]))
    assert rc == 0 and np.array_equal(out, g["expected"])


@pytest.mark.parametrize("name", ["mxfp4", "mxfp4_ragged"])
def test_mxfp4_golden(orc, name):
    g = golden(name)
    rc, out = orc.dequant_mxfp4(g["blocks"], g["scales"], int(g["N"]), int(g["K"]))
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))


def test_mxfp4_exhaustive_closed_form(orc):
    """All 16 codes x 256 scale bytes against e2m1 * 2^(e-127) (255 -> 0)."""
    mag = [0, .5, 1, 1.5, 2, 3, 4, 6]
    codes = np.arange(16)
    blocks = np.zeros((256, 16), np.uint8)
    blocks[:, :8] = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    scales = np.arange(256, dtype=np.uint8)[:, None]
    rc, out = orc.dequant_mxfp4(blocks, scales, 256, 16)
    assert rc == 0
    for e in range(256):
        for c in range(16):
            v = (-1 if c & 8 else 1) * mag[c & 7]
            with np.errstate(over="ignore"):  # 6 * 2^127 overflows f32 to inf, as in C
                want = 0.0 if e == 255 else np.float32(np.ldexp(np.float64(v), e - 127))
            assert out[e, c] == np.float32(want) and (np.signbit(out[e, c]) == np.signbit(
                np.float32(want)) or want == 0), (e, c)


def test_layout_known_answers(orc):
    """reference tests/test_qweight.c:130-225, restated."""
    cfg = make_cfg(method=1, bits=4, group_size=2)
    qw = np.array([[1 | (2 << 16)], [0], [0], [0]], np.int32)
    rc, out = orc.dequant(cfg, qw, np.ones((2, 2), np.float32), 2, 4)
    assert rc == 0 and out[0, 0] == 1 and out[1, 0] == 2 and out[0, 1] == 0
    cfg = make_cfg(method=1, bits=4, group_size=2, transposed=1)
    qw = np.array([[3 << 16, 0, 0, 0]], np.int32)
    rc, out = orc.dequant(cfg, qw, np.ones((2, 2), np.float32), 2, 4)
    assert rc == 0 and out[1, 0] == 3
    cfg = make_cfg(method=2, bits=4, group_size=4, zero_point=1)
    qw = np.array([[5 << 12, np.uint32(7 << 28).view(np.int32)]], np.int32)
    qz = np.array([[8 | (8 << 4)], [8 | (8 << 4)]], np.int32)
    rc, out = orc.dequant(cfg, qw, np.full((2, 2), .5, np.float32), 2, 8, qzeros=qz)
    assert rc == 0 and out[0, 3] == -1.5 and out[1, 7] == -0.5 and out[0, 0] == -4.0
    cfg = make_cfg(method=2, bits=4, group_size=2, zero_point=1, desc_act=1)
    rc, out = orc.dequant(cfg, np.array([[2 | (2 << 4)]], np.int32),
                          np.array([[1.0], [4.0]], np.float32), 1, 8,
                          qzeros=np.zeros((2, 1), np.int32),
                          g_idx=np.array([1, 0] * 4, np.int32))
    assert rc == 0 and out[0, 0] == 8.0 and out[0, 1] == 2.0


def test_error_paths_match_reference(orc):
    g = golden("errors")
    want = dict(zip([str(n) for n in g["names"]], g["rc"]))
    qw = np.zeros((4, 1), np.int32)
    sc = np.ones((2, 2), np.float32)
    gq = np.zeros((1, 2), np.int32)
    got = {
        "awq8": orc.dequant(make_cfg(method=1, bits=8, group_size=2), qw, sc, 2, 4)[0],
        "bad_sc_cols": orc.dequant(make_cfg(method=1, bits=4, group_size=2), qw,
                                   np.ones((2, 3), np.float32), 2, 4)[0],
        "bits3": orc.dequant(make_cfg(method=2, bits=3, group_size=2), qw, sc, 2, 4)[0],
        "method0": orc.dequant(make_cfg(method=0, bits=4, group_size=2), qw, sc, 2, 4)[0],
        "gidx_range": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                  g_idx=np.array([0, 1, 2, 0, 0, 0, 0, 0], np.int32))[0],
        "gidx_neg": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                g_idx=np.array([0, -1, 0, 0, 0, 0, 0, 0], np.int32))[0],
        "gidx_short": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                  g_idx=np.zeros(4, np.int32))[0],
        "gptq_shape": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 16)[0],
        "scales_rows": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq,
                                   np.ones((1, 2), np.float32), 2, 8)[0],
        "qz_rows": orc.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                               qzeros=np.zeros((1, 1), np.int32))[0],
        "marlin_k": orc.dequant_marlin(make_cfg(method=2, bits=4, group_size=8, layout=1),
                                       np.zeros((1, 128), np.int32),
                                       np.ones((1, 64), np.float32), 64, 8)[0],
        "mx_cols": orc.dequant_mxfp4(np.zeros((2, 4), np.uint8), np.zeros((2, 1), np.uint8),
                                     2, 16)[0],
        "ct_rows": orc.dequant_ct(make_cfg(method=3, bits=4, group_size=8),
                                  np.zeros((3, 1), np.int32), np.ones((2, 1), np.float32),
                                  2, 8)[0],
    }
    assert got == want


def test_quant_i8_golden(orc):
    g = golden("quant_i8")
    s, q = orc.quant_rows_i8(g["X"])
    assert np.array_equal(q, g["q"]) and np.array_equal(s.view(np.uint32), g["s"].view(np.uint32))
    s, q = orc.quant_rows_i8(g["Xr"])
    assert np.array_equal(q, g["qr"]) and np.array_equal(s, g["sr"])
    for i in range(4):
        assert np.array_equal(orc.dequant_row_i8(q[i], s[i]), g["dq"][i])


def test_quant_i8_edge_semantics(orc):
    """Round half away from zero on exact ties, clamp at +-127, zero row -> scale 0."""
    x = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, 0.0, -127.0], np.float32)
    s, q = orc.quant_row_i8(x)
    assert s == np.float32(1.0) and list(q) == [127, 1, -1, 2, -2, 3, 0, -127]
    s, q = orc.quant_row_i8(np.zeros(5, np.float32))
    assert s == 0 and not q.any()


@pytest.mark.parametrize("name", ["w8_tail", "w8_m1", "w8_m8"])
def test_w8a16_golden(orc, name):
    g = golden(name)
    assert np.array_equal(orc.matmul_w8a16(g["A"], g["W8"], g["sw"], g["bias"]), g["C"])
    assert np.array_equal(orc.matmul_w8a16(g["A"], g["W8"], g["sw"]), g["C_nobias"])
    # fp64 brute force: the f32 accumulation stays within 1e-5 of the exact sum
    ex = (g["A"].astype(np.float64) @ g["W8"].astype(np.float64).T) * g["sw"] + g["bias"]
    assert np.abs(ex - g["C"]).max() <= 1e-5 * np.abs(ex).max()


@pytest.mark.parametrize("name", ["nt_tail", "nt_k128", "nt_k4096"])
def test_matmul_nt_golden(orc, name):
    g = golden(name)
    out = orc.matmul_nt(g["A"], g["W"], g["bias"])
    assert np.array_equal(out, g["C"])
    ex = g["A"].astype(np.float64) @ g["W"].astype(np.float64).T + g["bias"]
    assert np.abs(ex - out).max() <= 1e-5 * np.abs(ex).max()


def test_qcfg_golden():
    g = golden("qcfg")
    names = ("method", "bits", "group_size", "zero_point", "desc_act", "transposed", "v2",
             "packed_dim", "offset", "layout")
    for t, rc, cfg in zip(g["texts"], g["rc"], g["cfg"]):
        r, c = qcfg_from_json(str(t))
        assert r == rc, t
        if rc:
            assert [c[n] for n in names] == list(cfg), t


def test_moe_composition_bruteforce(orc):
    """orc_moe_ffn against a float64 composition of its parts on a tiny expert set."""
    import synth
    T, E, mi, ne, k = 5, 64, 32, 4, 2
    h = synth.normal(1, (T, E))
    wgu = [synth.normal(10 + e, (2 * mi, E), 0.05) for e in range(ne)]
    wdn = [synth.normal(20 + e, (E, mi), 0.05) for e in range(ne)]
    ids = np.array([[0, 1], [2, 3], [1, 1], [3, -1], [0, 2]], np.int32)
    wts = np.array([[.6, .4], [.5, .5], [.3, .7], [1., 0.], [.2, .8]], np.float32)
    out = orc.moe_ffn(h, wgu, wdn, ids, wts)
    ref = np.zeros((T, E))
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            if e < 0:
                continue
            gu = wgu[e].astype(np.float64) @ h[t]
            a = gu[:mi] / (1 + np.exp(-gu[:mi])) * gu[mi:]
            ref[t] += wts[t, j] * (wdn[e].astype(np.float64) @ a)
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.skipif(not have_reference(), reason="reference build oracle/_ref absent")
def test_oracle_equals_reference_fresh_inputs(orc):
    """Where the reference builds, the oracle matches it on fresh seeded inputs too."""
    import synth
    ref = Reference()
    W = synth.normal(77, (128, 384), 0.02)
    gi = synth.act_order_gidx(78, 384, 128)
    q, z, s = synth.quantize_groups(W, 128, g_idx=gi)
    qw, qz = synth.gptq_pack(q, z)
    cfg = make_cfg(method=2, bits=4, group_size=128, zero_point=1, desc_act=1)
    a = orc.dequant(cfg, qw, s, 128, 384, qzeros=qz, g_idx=gi)
    b = ref.dequant(cfg, qw, s, 128, 384, qzeros=qz, g_idx=gi)
    assert a[0] == b[0] == 0 and np.array_equal(a[1], b[1])
    A = synth.normal(79, (11, 384))
    assert np.array_equal(orc.matmul_nt(A, a[1]), ref.matmul_nt(A, b[1]))
    sw, W8 = orc.quant_rows_i8(W)
    sw2, W82 = ref.quant_rows_i8(W)
    assert np.array_equal(W8, W82) and np.array_equal(sw, sw2)
    assert np.array_equal(orc.matmul_w8a16(A, W8, sw), ref.matmul_w8a16(A, W8, sw))
    for t in [str(x) for x in golden("qcfg")["texts"]]:
        r1, c1 = qcfg_from_json(t)
        r2, c2 = ref.qcfg_from_json(t)
        assert r1 == r2 and (not r1 or c1 == c2), t
