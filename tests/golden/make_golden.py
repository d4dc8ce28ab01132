"""Writes the golden vectors under tests/golden/ by running the REFERENCE's own compiled C
(oracle/_ref/libsglref.so, built by `make -C oracle ref` from the reference sources in place).

Run in the build container only (the reference is not present on the GPU box):
    make -C oracle ref && python tests/golden/make_golden.py

Each .npz holds inputs and the reference's outputs (data only).  marlin_unit.npz carries the
data of the reference's known-answer file tests/_marlin_unit.json (MIT licence, (c) the
sglang.c authors), converted to arrays.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "sglang.c_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
from oracle.oracle import Reference, make_cfg  # noqa: E402
import synth  # noqa: E402

REF_ROOT = os.environ.get("SGL_REF_ROOT", "/root/reference")


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


def cfg_arr(c):
    return np.array([getattr(c, n) for n, _ in c._fields_], np.int32)


def dequant_cases(ref):
    cases = {}
    W = synth.normal(0x5EED1001, (64, 256), 0.02)
    # GPTQ 4-bit, G=32, natural groups
    q, z, s = synth.quantize_groups(W, 32)
    qw, qz = synth.gptq_pack(q, z)
    cases["gptq4"] = dict(cfg=make_cfg(method=2, bits=4, group_size=32, zero_point=1),
                          qweight=qw, qzeros=qz, scales=s, N=64, K=256)
    # GPTQ act-order
    gi = synth.act_order_gidx(0x5EED1002, 256, 32)
    q, z, s = synth.quantize_groups(W, 32, g_idx=gi)
    qw, qz = synth.gptq_pack(q, z)
    cases["gptq4_act"] = dict(cfg=make_cfg(method=2, bits=4, group_size=32, zero_point=1,
                                           desc_act=1),
                              qweight=qw, qzeros=qz, scales=s, g_idx=gi, N=64, K=256)
    # GPTQ v2 (stored zeros are z-1)
    q, z, s = synth.quantize_groups(W, 64)
    qw, qz = synth.gptq_pack(q, z, v2=True)
    cases["gptq4_v2"] = dict(cfg=make_cfg(method=2, bits=4, group_size=64, zero_point=1, v2=1),
                             qweight=qw, qzeros=qz, scales=s, N=64, K=256)
    # GPTQ without qzeros
    cases["gptq4_noz"] = dict(cfg=make_cfg(method=2, bits=4, group_size=64, zero_point=1),
                              qweight=qw, scales=s, N=64, K=256)
    # GPTQ 8-bit: exercises the n>>3 zero-word indexing
    W8 = synth.normal(0x5EED1003, (16, 64), 0.02)
    q, z, s = synth.quantize_groups(W8, 32, bits=8)
    qw, qz = synth.gptq_pack(q, z, bits=8)
    cases["gptq8"] = dict(cfg=make_cfg(method=2, bits=8, group_size=32, zero_point=1),
                          qweight=qw, qzeros=qz, scales=s, N=16, K=64)
    # GPTQ with ragged K (K not a multiple of the group) and group_size -1
    W9 = synth.normal(0x5EED1004, (24, 200), 0.02)
    q, z, s = synth.quantize_groups(W9, 0)
    Kp = 200
    qpad = np.zeros((24, 208), np.uint8)
    qpad[:, :Kp] = q
    qw, qz = synth.gptq_pack(qpad, z)
    cases["gptq4_rowgroup"] = dict(cfg=make_cfg(method=2, bits=4, group_size=-1, zero_point=1),
                                   qweight=qw, qzeros=qz, scales=s, N=24, K=200)
    # AWQ gemm / gemv / no zero point
    q, z, s = synth.quantize_groups(W, 32)
    qw, qz = synth.awq_pack(q, z)
    cases["awq4"] = dict(cfg=make_cfg(method=1, bits=4, group_size=32, zero_point=1),
                         qweight=qw, qzeros=qz, scales=s, N=64, K=256)
    qwt, _ = synth.awq_pack(q, z, transposed=True)
    cases["awq4_gemv"] = dict(cfg=make_cfg(method=1, bits=4, group_size=32, zero_point=1,
                                           transposed=1),
                              qweight=qwt, qzeros=qz, scales=s, N=64, K=256)
    cases["awq4_noz"] = dict(cfg=make_cfg(method=1, bits=4, group_size=32, zero_point=0),
                             qweight=qw, scales=s, N=64, K=256)
    out = {}
    for name, c in cases.items():
        rc, dq = ref.dequant(c["cfg"], c["qweight"], c["scales"], c["N"], c["K"],
                             qzeros=c.get("qzeros"), g_idx=c.get("g_idx"))
        assert rc == 0, name
        arr = dict(cfg=cfg_arr(c["cfg"]), qweight=c["qweight"], scales=c["scales"],
                   N=np.int64(c["N"]), K=np.int64(c["K"]), expected=dq)
        for opt in ("qzeros", "g_idx"):
            if opt in c:
                arr[opt] = c[opt]
        save("dequant_" + name, **arr)
        out[name] = dq
    return out


def marlin_cases(ref):
    W = synth.normal(0x5EED2001, (128, 64), 0.02)
    for bits, withz in ((4, True), (4, False), (8, True), (8, False)):
        q, z, s = synth.quantize_groups(W, 32, bits=bits, sym=not withz)
        qw, qz, sc = synth.marlin_pack(q, z, s, bits=bits, with_zeros=withz)
        cfg = make_cfg(method=2, bits=bits, group_size=32, zero_point=1, layout=1)
        rc, dq = ref.dequant_marlin(cfg, qw, sc, 128, 64, qzeros=qz)
        assert rc == 0
        # the natural-layout twin of the same codes (GPTQ pack) must dequantize identically
        arr = dict(cfg=cfg_arr(cfg), qweight=qw, scales=sc, N=np.int64(128), K=np.int64(64),
                   expected=dq, codes=q, zeros=z, nat_scales=s)
        if qz is not None:
            arr["qzeros"] = qz
        save(f"marlin{bits}_{'asym' if withz else 'sym'}", **arr)


def marlin_unit_fixture():
    path = os.path.join(REF_ROOT, "tests", "_marlin_unit.json")
    d = json.load(open(path))
    arrs = {}
    for c in d["cases"]:
        p = c["name"] + "_"
        for k in ("K", "N", "G", "bits", "has_z", "qw_rows", "qw_cols", "qz_rows", "qz_cols",
                  "sc_rows", "sc_cols"):
            arrs[p + k] = np.int64(c[k])
        arrs[p + "qweight"] = np.array(c["qweight"], np.int64).astype(np.int32)
        arrs[p + "qzeros"] = np.array(c["qzeros"], np.int64).astype(np.int32)
        arrs[p + "scales"] = np.array(c["scales"], np.float32)
        arrs[p + "expected"] = np.array(c["expected"], np.float32)
    arrs["names"] = np.array([c["name"] for c in d["cases"]])
    save("marlin_unit", **arrs)


def ct_mxfp4_cases(ref):
    W = synth.normal(0x5EED3001, (32, 192), 0.02)
    for bits in (4, 8):
        half = 1 << (bits - 1)
        sc = (np.abs(W).reshape(32, 6, 32).max(axis=2) / (half - 1)).astype(np.float16)
        sc = sc.astype(np.float32)
        sq = np.clip(np.round(W / np.repeat(sc, 32, axis=1)), -half, half - 1).astype(np.int32)
        wp = synth.ct_pack(sq, bits)
        cfg = make_cfg(method=3, bits=bits, group_size=32, offset=half, packed_dim=1)
        rc, dq = ref.dequant_ct(cfg, wp, sc, 32, 192)
        assert rc == 0
        save(f"ct{bits}", cfg=cfg_arr(cfg), wpacked=wp, scales=sc, N=np.int64(32),
             K=np.int64(192), expected=dq)
    # MXFP4, including scale bytes 255 (-> 0), 0 (2^-127) and 254, and a ragged K
    Wm = synth.normal(0x5EED3002, (16, 160), 0.02)
    blocks, scales = synth.mxfp4_quantize(Wm)
    scales[0, 0] = 255
    scales[1, 1] = 0
    scales[2, 2] = 254
    scales[3, 3] = 1
    rc, dq = ref.dequant_mxfp4(blocks, scales, 16, 160)
    assert rc == 0
    save("mxfp4", blocks=blocks, scales=scales, N=np.int64(16), K=np.int64(160), expected=dq)
    # ragged K: 150 values per row, ceil(150/32) = 5 scale columns
    rc, dq2 = ref.dequant_mxfp4(blocks, scales[:, :5], 16, 150)
    assert rc == 0
    save("mxfp4_ragged", blocks=blocks, scales=scales[:, :5], N=np.int64(16), K=np.int64(150),
         expected=dq2)


def int8_cases(ref):
    rows = [np.zeros(37, np.float32),
            np.array([1.0, -1.0, 0.5, -0.5] * 9 + [127.0], np.float32),
            np.linspace(-3, 3, 37).astype(np.float32),
            np.full(37, 1e-40, np.float32),
            np.array([(i - 18) * (127.0 / 36.0) * 0.01 for i in range(37)], np.float32),
            synth.normal(0x5EED4001, 37, 1.0),
            synth.normal(0x5EED4002, 37, 1e30)]
    X = np.stack(rows)
    s, q = ref.quant_rows_i8(X)
    Xr = synth.normal(0x5EED4003, (16, 896), 0.02)
    sr, qr = ref.quant_rows_i8(Xr)
    dq = np.stack([ref.dequant_row_i8(qr[i], sr[i]) for i in range(4)])
    save("quant_i8", X=X, q=q, s=s, Xr=Xr, qr=qr, sr=sr, dq=dq)
    # W8A16 matmul: a ragged K (tail path) and the Qwen2.5-0.5B K with M=1 and M=8
    out = {}
    for name, (M, N, K) in {"w8_tail": (3, 40, 100), "w8_m1": (1, 64, 896),
                            "w8_m8": (8, 48, 896)}.items():
        A = synth.normal(0x5EED4100 + K + M, (M, K), 1.0)
        W = synth.normal(0x5EED4200 + K + M, (N, K), 0.02)
        sw, W8 = ref.quant_rows_i8(W)
        bias = synth.normal(0x5EED4300 + M, N, 0.1)
        Cm = ref.matmul_w8a16(A, W8, sw, bias)
        C0 = ref.matmul_w8a16(A, W8, sw, None)
        save(name, A=A, W8=W8, sw=sw, bias=bias, C=Cm, C_nobias=C0)
        out[name] = Cm
    # f32 NT matmul: M>8 (two row blocks), K with and without a tail
    for name, (M, N, K) in {"nt_tail": (9, 33, 100), "nt_k128": (3, 16, 128),
                            "nt_k4096": (1, 8, 4096)}.items():
        A = synth.normal(0x5EED4400 + K, (M, K), 1.0)
        W = synth.normal(0x5EED4500 + K, (N, K), 0.02)
        bias = synth.normal(0x5EED4600 + K, N, 0.1)
        save(name, A=A, W=W, bias=bias, C=ref.matmul_nt(A, W, bias))
    return out


def error_cases(ref):
    """Shape/config violations: the reference returns -1; record each rc."""
    qw = np.zeros((4, 1), np.int32)
    sc = np.ones((2, 2), np.float32)
    rcs = {}
    rcs["awq8"] = ref.dequant(make_cfg(method=1, bits=8, group_size=2), qw, sc, 2, 4)[0]
    rcs["bad_sc_cols"] = ref.dequant(make_cfg(method=1, bits=4, group_size=2), qw,
                                     np.ones((2, 3), np.float32), 2, 4)[0]
    rcs["bits3"] = ref.dequant(make_cfg(method=2, bits=3, group_size=2), qw, sc, 2, 4)[0]
    rcs["method0"] = ref.dequant(make_cfg(method=0, bits=4, group_size=2), qw, sc, 2, 4)[0]
    gq = np.zeros((1, 2), np.int32)
    rcs["gidx_range"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                    g_idx=np.array([0, 1, 2, 0, 0, 0, 0, 0], np.int32))[0]
    rcs["gidx_neg"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                  g_idx=np.array([0, -1, 0, 0, 0, 0, 0, 0], np.int32))[0]
    rcs["gidx_short"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                    g_idx=np.zeros(4, np.int32))[0]
    rcs["gptq_shape"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 16)[0]
    rcs["scales_rows"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq,
                                     np.ones((1, 2), np.float32), 2, 8)[0]
    rcs["qz_rows"] = ref.dequant(make_cfg(method=2, bits=4, group_size=4), gq, sc, 2, 8,
                                 qzeros=np.zeros((1, 1), np.int32))[0]
    rcs["marlin_k"] = ref.dequant_marlin(make_cfg(method=2, bits=4, group_size=8, layout=1),
                                         np.zeros((1, 128), np.int32),
                                         np.ones((1, 64), np.float32), 64, 8)[0]
    rcs["mx_cols"] = ref.dequant_mxfp4(np.zeros((2, 4), np.uint8), np.zeros((2, 1), np.uint8),
                                       2, 16)[0]
    rcs["ct_rows"] = ref.dequant_ct(make_cfg(method=3, bits=4, group_size=8),
                                    np.zeros((3, 1), np.int32), np.ones((2, 1), np.float32),
                                    2, 8)[0]
    names = sorted(rcs)
    save("errors", names=np.array(names), rc=np.array([rcs[n] for n in names], np.int64))


QCFG_TEXTS = [
    # reference tests/test_qweight.c:384-421
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"awq","version":"gemm",'
    '"zero_point":true}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"awq","version":"gemv",'
    '"zero_point":false}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"gptq","desc_act":true,'
    '"sym":true,"format":"gptq"}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"gptq","format":"gptq_v2"}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"gptq",'
    '"format":"gptq_marlin_v9"}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"gptq",'
    '"format":"gptq_marlin"}}',
    '{"quantization_config":{"bits":4,"group_size":128,"quant_method":"awq","version":"marlin",'
    '"zero_point":false}}',
    '{"hidden_size":64}',
    # further branches of reference src/qweight.c:375-482
    '{"quantization_config":{"quant_method":"gptq","bits":8,"group_size":-1,"desc_act":0}}',
    '{"quantization_config":{"quant_method":"gptq","format":"marlin","bits":4}}',
    '{"quantization_config":{"quant_method":"awq","version":"gemv_fast","bits":4.4}}',
    '{"quantization_config":{"quant_method":"compressed-tensors","format":"pack-quantized",'
    '"config_groups":{"group_0":{"weights":{"num_bits":4,"group_size":32,"symmetric":true}}}}}',
    '{"quantization_config":{"quant_method":"compressed-tensors","format":"pack-quantized",'
    '"config_groups":{"group_0":{"weights":{"num_bits":8,"group_size":-1}}},"packed_dim":0}}',
    '{"quantization_config":{"quant_method":"compressed-tensors","format":"pack-quantized",'
    '"config_groups":{"group_0":{"weights":{"num_bits":4,"symmetric":false}}}}}',
    '{"quantization_config":{"quant_method":"compressed-tensors","format":"float-quantized"}}',
    '{"quantization_config":{"quant_method":"compressed-tensors","format":"pack-quantized",'
    '"config_groups":{"g":{"weights":{"num_bits":2}}}}}',
    '{"quantization_config":{"quant_method":"compressed-tensors"}}',
    '{"quantization_config":{"quant_method":"mxfp4"}}',
    '{"quantization_config":{"quant_method":"fp8"}}',
    '{"quantization_config":[1,2]}',
    '{"quantization_config":{"quant_method":"awq","zero_point":0,"group_size":64.5}}',
    '{"quantization_config":{"quant_method":"gptq","format":null,"bits":true}}',
    'not json',
    '',
]


def qcfg_cases(ref):
    rcs, cfgs = [], []
    for t in QCFG_TEXTS:
        rc, c = ref.qcfg_from_json(t)
        rcs.append(rc)
        cfgs.append([c[n] for n in ("method", "bits", "group_size", "zero_point", "desc_act",
                                    "transposed", "v2", "packed_dim", "offset", "layout")])
    save("qcfg", texts=np.array(QCFG_TEXTS), rc=np.array(rcs, np.int64),
         cfg=np.array(cfgs, np.int64))


def main():
    ref = Reference()
    dequant_cases(ref)
    marlin_cases(ref)
    marlin_unit_fixture()
    ct_mxfp4_cases(ref)
    int8_cases(ref)
    error_cases(ref)
    qcfg_cases(ref)
    tot = sum(os.path.getsize(os.path.join(HERE, f)) for f in os.listdir(HERE)
              if f.endswith(".npz"))
    print(f"golden vectors written: {tot / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
