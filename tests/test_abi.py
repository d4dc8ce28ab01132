"""C-ABI boundary checks that need no GPU: the library loads, exports every function the
public headers declare (and nothing else), and its host-only logic (config parsing,
argument validation) matches the reference's golden vectors."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT, golden

LIB = os.path.join(ROOT, "sglang.c_amd", "libsgl_qlinear.so")
HEADERS = ["qweight.h", "quant.h", "ops.h", "qlinear.h", "qload.h", "qcache.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        txt = open(os.path.join(ROOT, "include", "sgl", h)).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        txt = re.sub(r"#.*", "", txt)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", txt):
            name = m.group(1)
            if name.startswith("sgl_"):
                names.add(name)
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libsgl_qlinear.so is not built: run __graft_entry__.build()")
    return ctypes.CDLL(LIB)


def test_exports_match_headers(lib):
    want = declared_functions()
    assert len(want) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    sgl = {n for n in exported if n.startswith("sgl_")}
    assert want <= sgl, f"missing: {sorted(want - sgl)}"
    assert sgl <= want, f"exported but undeclared: {sorted(sgl - want)}"
    for n in want:
        getattr(lib, n)


def test_q_pack():
    import sgl_qlinear as q
    assert [q.q_pack(b) for b in (0, 2, 4, 8)] == [0, 16, 8, 4]


def test_qcfg_from_json_golden():
    import sgl_qlinear as q
    g = golden("qcfg")
    names = ("method", "bits", "group_size", "zero_point", "desc_act", "transposed", "v2",
             "packed_dim", "offset", "layout")
    for t, rc, cfg in zip(g["texts"], g["rc"], g["cfg"]):
        r, c = q.qcfg_from_json(str(t))
        assert r == rc, t
        assert [c[n] for n in names] == list(cfg), t


def test_validation_errors_match_reference():
    """Argument violations are caught on the host, before any device work, with the reference's
    return codes (golden errors.npz)."""
    import sgl_qlinear as q
    mk = q.make_cfg
    want = dict(zip([str(n) for n in golden("errors")["names"]], golden("errors")["rc"]))
    qw = np.zeros((4, 1), np.int32)
    sc = np.ones((2, 2), np.float32)
    gq = np.zeros((1, 2), np.int32)
    got = {
        "awq8": q.qweight_dequant(mk(method=1, bits=8, group_size=2), qw, sc, 2, 4)[0],
        "bad_sc_cols": q.qweight_dequant(mk(method=1, bits=4, group_size=2), qw,
                                         np.ones((2, 3), np.float32), 2, 4)[0],
        "bits3": q.qweight_dequant(mk(method=2, bits=3, group_size=2), qw, sc, 2, 4)[0],
        "method0": q.qweight_dequant(mk(method=0, bits=4, group_size=2), qw, sc, 2, 4)[0],
        "gidx_range": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                        g_idx=np.array([0, 1, 2, 0, 0, 0, 0, 0]))[0],
        "gidx_neg": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                      g_idx=np.array([0, -1, 0, 0, 0, 0, 0, 0]))[0],
        "gidx_short": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                        g_idx=np.zeros(4))[0],
        "gptq_shape": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq, sc, 2, 16)[0],
        "scales_rows": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq,
                                         np.ones((1, 2), np.float32), 2, 8)[0],
        "qz_rows": q.qweight_dequant(mk(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                     qzeros=np.zeros((1, 1), np.int32))[0],
        "marlin_k": q.qweight_dequant_marlin(mk(method=2, bits=4, group_size=8, layout=1),
                                             np.zeros((1, 128), np.int32),
                                             np.ones((1, 64), np.float32), 64, 8)[0],
        "mx_cols": q.qweight_dequant_mxfp4(np.zeros((2, 4), np.uint8), np.zeros((2, 1), np.uint8),
                                           2, 16)[0],
        "ct_rows": q.qweight_dequant_ct(mk(method=3, bits=4, group_size=8),
                                        np.zeros((3, 1), np.int32), np.ones((2, 1), np.float32),
                                        2, 8)[0],
    }
    assert got == want
