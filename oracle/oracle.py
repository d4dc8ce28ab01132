"""ctypes front end of the CPU checker (oracle/liboracle.so) and of the compiled reference
(oracle/_ref/libsglref.so, present only where the reference sources were available to build).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package.

The C functions restate the reference (each cites reference file:line in sgl_oracle.c);
the Python function qcfg_from_json restates reference src/qweight.c:375-482 together with the
JSON accessors of reference src/json.c:266-300.
"""
import ctypes as C
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libsglref.so")


class QCfg(C.Structure):
    """Same field order as reference include/sgl/qweight.h:45-56."""
    _fields_ = [(n, C.c_int) for n in ("method", "bits", "group_size", "zero_point", "desc_act",
                                        "transposed", "v2", "packed_dim", "offset", "layout")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


def make_cfg(**kw):
    c = QCfg()
    for k, v in kw.items():
        setattr(c, k, int(v))
    return c


_P = C.c_void_p
_I64 = C.c_int64


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class _Lib:
    """Binds one shared library whose symbols are <prefix>qweight_dequant, ... ."""

    def __init__(self, path, prefix):
        self.path = path
        self.lib = C.CDLL(path)
        self.prefix = prefix
        L, p = self.lib, prefix
        self._dq = getattr(L, p + "qweight_dequant")
        self._dq.argtypes = [C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _P, _I64, _I64, _I64, _P]
        self._dq.restype = C.c_int
        self._mar = getattr(L, p + "qweight_dequant_marlin")
        self._mar.argtypes = [C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                              _I64, _I64, _P]
        self._mar.restype = C.c_int
        self._ct = getattr(L, p + "qweight_dequant_ct")
        self._ct.argtypes = [C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P]
        self._ct.restype = C.c_int
        self._mx = getattr(L, p + "qweight_dequant_mxfp4")
        self._mx.argtypes = [_P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P]
        self._mx.restype = C.c_int
        self._qr = getattr(L, p + "quant_row_i8")
        self._qr.argtypes = [_P, _P, C.c_int]
        self._qr.restype = C.c_float
        self._qrs = getattr(L, p + "quant_rows_i8")
        self._qrs.argtypes = [_P, _P, _P, C.c_int, C.c_int]
        self._qrs.restype = None
        self._dqr = getattr(L, p + "dequant_row_i8")
        self._dqr.argtypes = [_P, C.c_float, _P, C.c_int]
        self._dqr.restype = None
        self._w8 = getattr(L, p + "matmul_w8a16")
        self._w8.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int]
        self._w8.restype = None
        self._nt = getattr(L, p + "matmul_nt")
        self._nt.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int]
        self._nt.restype = None

    # -- dequant ------------------------------------------------------------------------
    def dequant(self, cfg, qweight, scales, N, K, qzeros=None, g_idx=None, shapes=None):
        """Returns (rc, out f32 [N,K]).  shapes overrides the row/col counts passed to C."""
        qw = np.ascontiguousarray(qweight, dtype=np.int32)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        qz = None if qzeros is None else np.ascontiguousarray(qzeros, dtype=np.int32)
        gi = None if g_idx is None else np.ascontiguousarray(g_idx, dtype=np.int32)
        s = dict(qw=qw.shape, qz=(0, 0) if qz is None else qz.shape, sc=sc.shape,
                 g=0 if gi is None else gi.shape[0])
        if shapes:
            s.update(shapes)
        out = np.zeros((N, K), np.float32)
        rc = self._dq(C.byref(cfg), _ptr(qw), s["qw"][0], s["qw"][1], _ptr(qz), s["qz"][0],
                      s["qz"][1], _ptr(sc), s["sc"][0], s["sc"][1], _ptr(gi), s["g"], N, K,
                      _ptr(out))
        return rc, out

    def dequant_marlin(self, cfg, qweight, scales, N, K, qzeros=None, shapes=None):
        qw = np.ascontiguousarray(qweight, dtype=np.int32)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        qz = None if qzeros is None else np.ascontiguousarray(qzeros, dtype=np.int32)
        s = dict(qw=qw.shape, qz=(0, 0) if qz is None else qz.shape, sc=sc.shape)
        if shapes:
            s.update(shapes)
        out = np.zeros((N, K), np.float32)
        rc = self._mar(C.byref(cfg), _ptr(qw), s["qw"][0], s["qw"][1], _ptr(qz), s["qz"][0],
                       s["qz"][1], _ptr(sc), s["sc"][0], s["sc"][1], N, K, _ptr(out))
        return rc, out

    def dequant_ct(self, cfg, wpacked, scales, N, K, shapes=None):
        wp = np.ascontiguousarray(wpacked, dtype=np.int32)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        s = dict(w=wp.shape, sc=sc.shape)
        if shapes:
            s.update(shapes)
        out = np.zeros((N, K), np.float32)
        rc = self._ct(C.byref(cfg), _ptr(wp), s["w"][0], s["w"][1], _ptr(sc), s["sc"][0],
                      s["sc"][1], N, K, _ptr(out))
        return rc, out

    def dequant_mxfp4(self, blocks, scales, N, K, shapes=None):
        wp = np.ascontiguousarray(blocks, dtype=np.uint8)
        sc = np.ascontiguousarray(scales, dtype=np.uint8)
        s = dict(w=wp.shape, sc=sc.shape)
        if shapes:
            s.update(shapes)
        out = np.zeros((N, K), np.float32)
        rc = self._mx(None, _ptr(wp), s["w"][0], s["w"][1], _ptr(sc), s["sc"][0], s["sc"][1],
                      N, K, _ptr(out))
        return rc, out

    # -- int8 ---------------------------------------------------------------------------
    def quant_row_i8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.shape[0], np.int8)
        s = self._qr(_ptr(x), _ptr(q), x.shape[0])
        return np.float32(s), q

    def quant_rows_i8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.shape, np.int8)
        s = np.zeros(x.shape[0], np.float32)
        self._qrs(_ptr(x), _ptr(q), _ptr(s), x.shape[0], x.shape[1])
        return s, q

    def dequant_row_i8(self, q, scale):
        q = np.ascontiguousarray(q, dtype=np.int8)
        out = np.zeros(q.shape[0], np.float32)
        self._dqr(_ptr(q), float(scale), _ptr(out), q.shape[0])
        return out

    def matmul_w8a16(self, A, W, sw, bias=None):
        A = np.ascontiguousarray(A, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.int8)
        sw = np.ascontiguousarray(sw, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        M, K = A.shape
        N = W.shape[0]
        Cm = np.zeros((M, N), np.float32)
        self._w8(_ptr(A), _ptr(W), _ptr(sw), _ptr(b), _ptr(Cm), M, N, K)
        return Cm

    def matmul_nt(self, A, W, bias=None):
        A = np.ascontiguousarray(A, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        M, K = A.shape
        N = W.shape[0]
        Cm = np.zeros((M, N), np.float32)
        self._nt(_ptr(A), _ptr(W), _ptr(b), _ptr(Cm), M, N, K)
        return Cm


class Oracle(_Lib):
    def __init__(self, path=LIB_PATH):
        super().__init__(path, "orc_")
        self._moe = self.lib.orc_moe_ffn
        self._moe.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, C.c_int, _P]
        self._moe.restype = None
        self.lib.orc_num_threads.restype = C.c_int
        self._route = self.lib.orc_moe_route
        self._route.argtypes = [_P, C.c_int, C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_int, C.c_float, _P, _P]
        self._route.restype = None
        self._shared = self.lib.orc_moe_shared
        self._shared.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P]
        self._shared.restype = None

    def moe_route(self, logits, k, bias=None, sigmoid=True, n_group=0, topk_group=0,
                  norm=True, scale=1.0):
        """logits f32 [T, n_experts] -> (ids int32 [T, k], weights f32 [T, k])."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        T, ne = lg.shape
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        ids = np.zeros((T, k), np.int32)
        w = np.zeros((T, k), np.float32)
        self._route(_ptr(lg), T, ne, _ptr(b), int(sigmoid), n_group, topk_group, k, int(norm),
                    scale, _ptr(ids), _ptr(w))
        return ids, w

    def moe_shared(self, h, wg, wu, wd, out):
        """out += shared SwiGLU MLP of h (in place); wg/wu [sh, E], wd [E, sh]."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        T, E = h.shape
        wg, wu, wd = (np.ascontiguousarray(x, dtype=np.float32) for x in (wg, wu, wd))
        assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
        self._shared(_ptr(h), T, E, wg.shape[0], _ptr(wg), _ptr(wu), _ptr(wd), _ptr(out))
        return out

    def num_threads(self):
        return self.lib.orc_num_threads()

    def moe_ffn(self, h, w_gu, w_dn, ids, wts):
        """h f32 [T,E]; w_gu list of f32 [2*mi,E]; w_dn list of f32 [E,mi]; ids/wts [T,k]."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        T, E = h.shape
        mi = w_gu[0].shape[0] // 2
        gu = [np.ascontiguousarray(w, dtype=np.float32) for w in w_gu]
        dn = [np.ascontiguousarray(w, dtype=np.float32) for w in w_dn]
        pgu = (C.c_void_p * len(gu))(*[w.ctypes.data for w in gu])
        pdn = (C.c_void_p * len(dn))(*[w.ctypes.data for w in dn])
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        wts = np.ascontiguousarray(wts, dtype=np.float32)
        out = np.zeros((T, E), np.float32)
        self._moe(_ptr(h), T, E, mi, C.cast(pgu, C.c_void_p), C.cast(pdn, C.c_void_p),
                  _ptr(ids), _ptr(wts), ids.shape[1], _ptr(out))
        return out


class Reference(_Lib):
    """The reference's own C, compiled from its sources by oracle/Makefile (target ref)."""

    def __init__(self, path=REF_PATH):
        super().__init__(path, "sgl_")
        self._cfg = self.lib.sgl_qcfg_from_json
        self._cfg.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(QCfg)]
        self._cfg.restype = C.c_int
        # keep the reference's INFO chatter off the test output
        try:
            self.lib.sgl_log_set_level.argtypes = [C.c_int]
            self.lib.sgl_log_set_level(3)
        except AttributeError:
            pass

    def qcfg_from_json(self, text):
        b = text.encode()
        c = QCfg()
        rc = self._cfg(b, len(b), C.byref(c))
        return rc, c.as_dict()


def have_reference():
    return os.path.exists(REF_PATH)


def _jget(obj, key):
    # reference src/json.c:266-271: first matching key of an object, else None
    if not isinstance(obj, dict):
        return None
    return obj.get(key)


def _get_int(obj, key, d):
    # reference src/json.c:285-293: bools count, numbers round half away from zero
    v = _jget(obj, key) if isinstance(obj, dict) and key in obj else None
    if not (isinstance(obj, dict) and key in obj):
        return d
    if isinstance(v, bool):
        return int(v)
    if isinstance(v, (int, float)):
        return int(v + 0.5) if v >= 0 else -int(-v + 0.5)
    return d


def _get_bool(obj, key, d):
    # reference src/json.c:295-300
    if not (isinstance(obj, dict) and key in obj):
        return d
    v = obj[key]
    if isinstance(v, bool):
        return int(v)
    if isinstance(v, (int, float)):
        return int(v != 0)
    return d


def _get_str(obj, key, d):
    # reference src/json.c:273-276
    v = _jget(obj, key)
    return v if isinstance(v, str) else d


def qcfg_from_json(text):
    """Restates reference src/qweight.c:375-482.  Returns (rc, cfg dict)."""
    cfg = {n: 0 for n, _ in QCfg._fields_}
    if not text:
        return 0, cfg
    try:
        root = json.loads(text)
    except ValueError:
        return 0, cfg
    qc = _jget(root, "quantization_config")
    if not isinstance(qc, dict):
        return 0, cfg
    method = _get_str(qc, "quant_method", "")
    cfg["bits"] = _get_int(qc, "bits", 4)
    cfg["group_size"] = _get_int(qc, "group_size", 128)
    if method == "awq":
        cfg["method"] = 1
        cfg["zero_point"] = _get_bool(qc, "zero_point", 1)
        ver = _get_str(qc, "version", "gemm")
        cfg["transposed"] = int(ver == "gemv")
        if ver == "marlin":
            cfg["layout"] = 1
    elif method == "gptq":
        cfg["method"] = 2
        cfg["zero_point"] = 1
        cfg["desc_act"] = _get_bool(qc, "desc_act", 0)
        fmt = _get_str(qc, "format", "gptq")
        if fmt == "gptq_v2":
            cfg["v2"] = 1
        elif fmt in ("marlin", "gptq_marlin"):
            cfg["layout"] = 1
        elif fmt and fmt != "gptq":
            cfg["method"] = 0
            return 0, cfg
    elif method == "compressed-tensors":
        fmt = _get_str(qc, "format", "")
        groups = _jget(qc, "config_groups")
        g0 = next(iter(groups.values())) if isinstance(groups, dict) and groups else None
        wq = _jget(g0, "weights") if g0 is not None else None
        nb, gsz, sym = 4, 128, 1
        if isinstance(wq, dict):
            nb = _get_int(wq, "num_bits", 4)
            gsz = _get_int(wq, "group_size", 128)
            sym = _get_bool(wq, "symmetric", 1)
            if gsz <= 0:
                gsz = 128
            if not sym:
                return 0, cfg
        if fmt != "pack-quantized":
            return 0, cfg
        if nb not in (4, 8):
            return 0, cfg
        cfg.update(method=3, bits=nb, group_size=gsz, packed_dim=_get_int(qc, "packed_dim", 1),
                   offset=1 << (nb - 1), zero_point=0)
    elif method == "mxfp4":
        cfg.update(method=4, bits=4, group_size=32, zero_point=0)
    else:
        return 0, cfg
    return 1, cfg
