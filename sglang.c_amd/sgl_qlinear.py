"""Python binding of libsgl_qlinear.so (ctypes), the way a maintainer would bind the C ABI of
include/sgl/{qweight,quant,ops,qlinear}.h from Python.  Used by the tests and bench.py.

Two groups of entry points:
  * the reference's C API, host buffers in and out (numpy): qweight_dequant, qweight_dequant_marlin,
    qweight_dequant_ct, qweight_dequant_mxfp4, qcfg_from_json, quant_rows_i8, quant_row_i8,
    dequant_row_i8, matmul_w8a16, matmul_nt;
  * the device-resident layer: QLinear (create from host buffers, forward / dequant on torch
    device tensors) and qmoe_forward.

There is no fallback: if the shared library is missing this module raises on import.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsgl_qlinear.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built (run `make -C sglang.c_amd` or "
                      "__graft_entry__.build())")
# torch bundles its own HIP runtime with the same SONAME (libamdhip64.so.7).  Loading torch first
# makes the library's dependency resolve to that already-loaded runtime, so one process never
# holds two HIP runtimes (which leaves one of them without devices).
try:
    import torch  # noqa: F401
except ImportError:
    torch = None
_L = C.CDLL(LIB_PATH)


def _hip_runtimes():
    with open("/proc/self/maps") as f:
        return sorted({ln.split()[-1] for ln in f if "libamdhip64.so" in ln})


if len(_hip_runtimes()) > 1:
    raise ImportError(f"two HIP runtimes are mapped ({_hip_runtimes()}); import torch before "
                      "anything that loads libamdhip64")

F32, BF16, F16 = 0, 1, 2
Q_NONE, Q_AWQ, Q_GPTQ, Q_CT, Q_MXFP4 = 0, 1, 2, 3, 4
LAYOUT_NATURAL, LAYOUT_MARLIN = 0, 1


class QCfg(C.Structure):
    """sgl_qcfg (include/sgl/qweight.h)."""
    _fields_ = [(n, C.c_int) for n in ("method", "bits", "group_size", "zero_point", "desc_act",
                                        "transposed", "v2", "packed_dim", "offset", "layout")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


def make_cfg(**kw):
    c = QCfg()
    for k, v in kw.items():
        setattr(c, k, int(v))
    return c


_P, _I64, _I = C.c_void_p, C.c_int64, C.c_int


def _sig(name, res, *args):
    f = getattr(_L, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_dq = _sig("sgl_qweight_dequant", _I, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
           _I64, _P, _I64, _I64, _I64, _P)
_dq_mar = _sig("sgl_qweight_dequant_marlin", _I, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64,
               _P, _I64, _I64, _I64, _I64, _P)
_dq_ct = _sig("sgl_qweight_dequant_ct", _I, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _I64,
              _I64, _P)
_dq_mx = _sig("sgl_qweight_dequant_mxfp4", _I, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P)
_qcfg = _sig("sgl_qcfg_from_json", _I, C.c_char_p, C.c_size_t, C.POINTER(QCfg))
_qpack = _sig("sgl_q_pack", _I, _I)
_qrow = _sig("sgl_quant_row_i8", C.c_float, _P, _P, _I)
_qrows = _sig("sgl_quant_rows_i8", None, _P, _P, _P, _I, _I)
_dqrow = _sig("sgl_dequant_row_i8", None, _P, C.c_float, _P, _I)
_w8 = _sig("sgl_matmul_w8a16", None, _P, _P, _P, _P, _P, _I, _I, _I)
_nt = _sig("sgl_matmul_nt", None, _P, _P, _P, _P, _I, _I, _I)

_create = _sig("sgl_qlinear_create", _P, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64, _P,
               _I64, _I64, _P, _I64, _I64, _I64, _I)
_create_mar = _sig("sgl_qlinear_create_marlin", _P, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64,
                   _I64, _P, _I64, _I64, _I64, _I64, _I)
_create_ct = _sig("sgl_qlinear_create_ct", _P, C.POINTER(QCfg), _P, _I64, _I64, _P, _I64, _I64,
                  _I64, _I64, _I)
_create_mx = _sig("sgl_qlinear_create_mxfp4", _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I)
_create_w8 = _sig("sgl_qlinear_create_w8", _P, _P, _P, _I64, _I64, _I)
_forward = _sig("sgl_qlinear_forward", _I, _P, _P, _I, _I64, _P, _P, _P)
_dequant = _sig("sgl_qlinear_dequant", _I, _P, _P, _P)
_nout = _sig("sgl_qlinear_out_features", _I64, _P)
_nin = _sig("sgl_qlinear_in_features", _I64, _P)
_wbytes = _sig("sgl_qlinear_weight_bytes", _I64, _P)
_destroy = _sig("sgl_qlinear_destroy", None, _P)
_moe = _sig("sgl_qmoe_forward", _I, _P, _P, _I, _P, _I, _I64, _P, _P, _I, _P, _P)


class QLoadInfo(C.Structure):
    _fields_ = [("kind", C.c_int), ("N", C.c_int64), ("K", C.c_int64), ("transposed", C.c_int),
                ("layout", C.c_int)]


QLOAD_KINDS = {0: "natural", 1: "marlin", 2: "ct", 3: "mxfp4"}
_RAWFN = C.CFUNCTYPE(C.c_int, _P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(C.c_int),
                     C.POINTER(C.c_int64), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t))
_qst_open = _sig("sgl_qst_open", _P, C.c_char_p)
_qst_raw = _sig("sgl_qst_get_raw", _I, _P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(C.c_int),
                C.POINTER(C.c_int64), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t))
_qst_close = _sig("sgl_qst_close", None, _P)
_qst_raw_fn = C.cast(_qst_raw, _RAWFN)  # the reader's own lookup, passed to load / probe
_probe = _sig("sgl_qlinear_probe", _I, C.POINTER(QCfg), _RAWFN, _P, C.c_char_p,
              C.POINTER(QLoadInfo))
_load = _sig("sgl_qlinear_load", _P, C.POINTER(QCfg), _RAWFN, _P, C.c_char_p,
             C.POINTER(C.c_int64), C.POINTER(C.c_int64), _I)


def _np(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _shape2(a):
    return (0, 0) if a is None else (a.shape[0], a.shape[1] if a.ndim > 1 else 1)


# ---- reference C API (host buffers) -----------------------------------------------------
def q_pack(bits):
    return _qpack(bits)


def qweight_dequant(cfg, qweight, scales, N, K, qzeros=None, g_idx=None, shapes=None):
    qw, sc, qz, gi = (_np(qweight, np.int32), _np(scales, np.float32), _np(qzeros, np.int32),
                      _np(g_idx, np.int32))
    s = dict(qw=_shape2(qw), qz=_shape2(qz), sc=_shape2(sc), g=0 if gi is None else gi.shape[0])
    s.update(shapes or {})
    out = np.zeros((N, K), np.float32)
    rc = _dq(C.byref(cfg), _ptr(qw), *s["qw"], _ptr(qz), *s["qz"], _ptr(sc), *s["sc"], _ptr(gi),
             s["g"], N, K, _ptr(out))
    return rc, out


def qweight_dequant_marlin(cfg, qweight, scales, N, K, qzeros=None, shapes=None):
    qw, sc, qz = _np(qweight, np.int32), _np(scales, np.float32), _np(qzeros, np.int32)
    s = dict(qw=_shape2(qw), qz=_shape2(qz), sc=_shape2(sc))
    s.update(shapes or {})
    out = np.zeros((N, K), np.float32)
    rc = _dq_mar(C.byref(cfg), _ptr(qw), *s["qw"], _ptr(qz), *s["qz"], _ptr(sc), *s["sc"], N, K,
                 _ptr(out))
    return rc, out


def qweight_dequant_ct(cfg, wpacked, scales, N, K, shapes=None):
    wp, sc = _np(wpacked, np.int32), _np(scales, np.float32)
    s = dict(w=_shape2(wp), sc=_shape2(sc))
    s.update(shapes or {})
    out = np.zeros((N, K), np.float32)
    rc = _dq_ct(C.byref(cfg), _ptr(wp), *s["w"], _ptr(sc), *s["sc"], N, K, _ptr(out))
    return rc, out


def qweight_dequant_mxfp4(blocks, scales, N, K, shapes=None):
    wp, sc = _np(blocks, np.uint8), _np(scales, np.uint8)
    s = dict(w=_shape2(wp), sc=_shape2(sc))
    s.update(shapes or {})
    out = np.zeros((N, K), np.float32)
    rc = _dq_mx(None, _ptr(wp), *s["w"], _ptr(sc), *s["sc"], N, K, _ptr(out))
    return rc, out


def qcfg_from_json(text):
    b = text.encode()
    c = QCfg()
    rc = _qcfg(b, len(b), C.byref(c))
    return rc, c.as_dict()


def quant_row_i8(x):
    x = _np(x, np.float32)
    q = np.zeros(x.shape[0], np.int8)
    s = _qrow(_ptr(x), _ptr(q), x.shape[0])
    return np.float32(s), q


def quant_rows_i8(x):
    x = _np(x, np.float32)
    q = np.zeros(x.shape, np.int8)
    s = np.zeros(x.shape[0], np.float32)
    _qrows(_ptr(x), _ptr(q), _ptr(s), x.shape[0], x.shape[1])
    return s, q


def dequant_row_i8(q, scale):
    q = _np(q, np.int8)
    out = np.zeros(q.shape[0], np.float32)
    _dqrow(_ptr(q), float(scale), _ptr(out), q.shape[0])
    return out


def matmul_w8a16(A, W, sw, bias=None):
    A, W, sw, b = _np(A, np.float32), _np(W, np.int8), _np(sw, np.float32), _np(bias, np.float32)
    out = np.zeros((A.shape[0], W.shape[0]), np.float32)
    _w8(_ptr(A), _ptr(W), _ptr(sw), _ptr(b), _ptr(out), A.shape[0], W.shape[0], A.shape[1])
    return out


def matmul_nt(A, W, bias=None):
    A, W, b = _np(A, np.float32), _np(W, np.float32), _np(bias, np.float32)
    out = np.zeros((A.shape[0], W.shape[0]), np.float32)
    _nt(_ptr(A), _ptr(W), _ptr(b), _ptr(out), A.shape[0], W.shape[0], A.shape[1])
    return out


# ---- device-resident layer ----------------------------------------------------------------
def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


_TORCH_DT = {}


def _dtype_code(t):
    import torch
    m = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
    if t.dtype not in m:
        raise TypeError(f"unsupported activation dtype {t.dtype}")
    return m[t.dtype]


class SafeTensors:
    """A single safetensors file opened by the library's reader (sgl_qst_*)."""

    def __init__(self, path):
        self.h = C.c_void_p(_qst_open(str(path).encode()))
        if not self.h:
            raise RuntimeError(f"sgl_qst_open({path}) failed (see the log line above)")

    def get_raw(self, name):
        """(dtype, dims, bytes) of a tensor, or None when the file has none by that name."""
        dt, nd, dims = C.c_char_p(), C.c_int(), (C.c_int64 * 4)()
        ptr, nb = C.c_void_p(), C.c_size_t()
        if not _qst_raw(self.h, name.encode(), C.byref(dt), C.byref(nd), dims, C.byref(ptr),
                        C.byref(nb)):
            return None
        data = C.string_at(ptr.value, nb.value) if nb.value else b""
        return (dt.value.decode("utf-8", "replace"), tuple(dims[i] for i in range(nd.value)),
                data)

    def probe(self, cfg, base):
        """(rc, info): rc 1 = loadable, 0 = no quantized tensors, -1 = error."""
        info = QLoadInfo()
        rc = _probe(C.byref(cfg), _qst_raw_fn, self.h, base.encode(), C.byref(info))
        return rc, {"kind": QLOAD_KINDS.get(info.kind), "N": info.N, "K": info.K,
                    "transposed": info.transposed, "layout": info.layout}

    def close(self):
        if self.h:
            _qst_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QLinear:
    """A quantized weight resident on the GPU (sgl_qlinear)."""

    def __init__(self, handle):
        if not handle:
            raise RuntimeError("sgl_qlinear_create failed (see the log line above)")
        self.h = C.c_void_p(handle)
        self.N = _nout(self.h)
        self.K = _nin(self.h)

    @classmethod
    def from_awq_gptq(cls, cfg, qweight, scales, N, K, qzeros=None, g_idx=None, dev=0):
        qw, sc, qz, gi = (_np(qweight, np.int32), _np(scales, np.float32), _np(qzeros, np.int32),
                          _np(g_idx, np.int32))
        return cls(_create(C.byref(cfg), _ptr(qw), *_shape2(qw), _ptr(qz), *_shape2(qz), _ptr(sc),
                           *_shape2(sc), _ptr(gi), 0 if gi is None else gi.shape[0], N, K, dev))

    @classmethod
    def from_marlin(cls, cfg, qweight, scales, N, K, qzeros=None, dev=0):
        qw, sc, qz = _np(qweight, np.int32), _np(scales, np.float32), _np(qzeros, np.int32)
        return cls(_create_mar(C.byref(cfg), _ptr(qw), *_shape2(qw), _ptr(qz), *_shape2(qz),
                               _ptr(sc), *_shape2(sc), N, K, dev))

    @classmethod
    def from_ct(cls, cfg, wpacked, scales, N, K, dev=0):
        wp, sc = _np(wpacked, np.int32), _np(scales, np.float32)
        return cls(_create_ct(C.byref(cfg), _ptr(wp), *_shape2(wp), _ptr(sc), *_shape2(sc), N, K,
                              dev))

    @classmethod
    def from_mxfp4(cls, blocks, scales, N, K, dev=0):
        wp, sc = _np(blocks, np.uint8), _np(scales, np.uint8)
        return cls(_create_mx(_ptr(wp), *_shape2(wp), _ptr(sc), *_shape2(sc), N, K, dev))

    @classmethod
    def load(cls, cfg, st, base, dev=0):
        """sgl_qlinear_load from a SafeTensors reader: the tensors under `base` as the
        reference's quant_get finds them.  cfg.transposed may be set (AWQ gemv layout)."""
        return cls(_load(C.byref(cfg), _qst_raw_fn, st.h, base.encode(), None, None, dev))

    @classmethod
    def from_w8(cls, W8, sw, dev=0):
        W, s = _np(W8, np.int8), _np(sw, np.float32)
        return cls(_create_w8(_ptr(W), _ptr(s), W.shape[0], W.shape[1], dev))

    @property
    def weight_bytes(self):
        return _wbytes(self.h)

    def forward(self, A, bias=None, out=None):
        """A: torch tensor [M, K] on the GPU (f32/bf16/f16). Returns f32 [M, N]."""
        import torch
        A = A.contiguous()
        M = A.shape[0]
        if out is None:
            out = torch.empty((M, self.N), dtype=torch.float32, device=A.device)
        rc = _forward(self.h, C.c_void_p(A.data_ptr()), _dtype_code(A), M,
                      None if bias is None else C.c_void_p(bias.data_ptr()),
                      C.c_void_p(out.data_ptr()), _stream())
        if rc != 0:
            raise RuntimeError("sgl_qlinear_forward failed")
        return out

    def dequant(self):
        import torch
        out = torch.empty((self.N, self.K), dtype=torch.float32, device="cuda")
        if _dequant(self.h, C.c_void_p(out.data_ptr()), _stream()) != 0:
            raise RuntimeError("sgl_qlinear_dequant failed")
        return out

    def close(self):
        if self.h:
            _destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def qmoe_forward(gate_up, down, h, topk_ids, topk_w, out=None):
    """gate_up/down: lists of QLinear; h [T,E] device tensor; topk_ids int32 / topk_w f32 [T,k]."""
    import torch
    n = len(gate_up)
    gu = (C.c_void_p * n)(*[q.h.value for q in gate_up])
    dn = (C.c_void_p * n)(*[q.h.value for q in down])
    h = h.contiguous()
    T = h.shape[0]
    E = down[0].N
    if out is None:
        out = torch.empty((T, E), dtype=torch.float32, device=h.device)
    ids = topk_ids.contiguous()
    wts = topk_w.contiguous()
    rc = _moe(C.cast(gu, C.c_void_p), C.cast(dn, C.c_void_p), n, C.c_void_p(h.data_ptr()),
              _dtype_code(h), T, C.c_void_p(ids.data_ptr()), C.c_void_p(wts.data_ptr()),
              ids.shape[1], C.c_void_p(out.data_ptr()), _stream())
    if rc != 0:
        raise RuntimeError("sgl_qmoe_forward failed")
    return out


class QMoERouting(C.Structure):
    _fields_ = [("sigmoid", C.c_int), ("n_group", C.c_int), ("topk_group", C.c_int),
                ("k", C.c_int), ("norm_topk", C.c_int), ("routed_scale", C.c_float)]


_router = _sig("sgl_qmoe_router_logits", _I, _P, _I, _P, _I, _I64, _I64, _P, _P)
_route = _sig("sgl_qmoe_route", _I, C.POINTER(QMoERouting), _P, _P, _I, _I64, _P, _P, _P)
_shared = _sig("sgl_qmoe_shared", _I, _P, _P, _P, _I, _I64, _P, _P)


def qmoe_router_logits(router_w, h, out=None):
    """router_w f32 [n_experts, E], h [T, E] device tensors -> logits f32 [T, n_experts]."""
    import torch
    w, h = router_w.contiguous(), h.contiguous()
    T, E = h.shape
    if out is None:
        out = torch.empty((T, w.shape[0]), dtype=torch.float32, device=h.device)
    if _router(C.c_void_p(w.data_ptr()), w.shape[0], C.c_void_p(h.data_ptr()), _dtype_code(h),
               T, E, C.c_void_p(out.data_ptr()), _stream()) != 0:
        raise RuntimeError("sgl_qmoe_router_logits failed")
    return out


def qmoe_route(logits, k, bias=None, sigmoid=True, n_group=0, topk_group=0, norm=True,
               scale=1.0):
    """logits f32 [T, n_experts] device tensor -> (topk_ids int32 [T, k], topk_w f32 [T, k])."""
    import torch
    lg = logits.contiguous()
    T, ne = lg.shape
    r = QMoERouting(int(sigmoid), n_group, topk_group, k, int(norm), scale)
    ids = torch.empty((T, k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, k), dtype=torch.float32, device=lg.device)
    b = None if bias is None else bias.contiguous()
    if _route(C.byref(r), C.c_void_p(lg.data_ptr()), None if b is None else C.c_void_p(b.data_ptr()),
              ne, T, C.c_void_p(ids.data_ptr()), C.c_void_p(w.data_ptr()), _stream()) != 0:
        raise RuntimeError("sgl_qmoe_route failed")
    return ids, w


def qmoe_shared(gate_up, down, h, out):
    """out [T, E] f32 device tensor += the shared experts' SwiGLU MLP of h (in place)."""
    h = h.contiguous()
    if _shared(gate_up.h, down.h, C.c_void_p(h.data_ptr()), _dtype_code(h), h.shape[0],
               C.c_void_p(out.data_ptr()), _stream()) != 0:
        raise RuntimeError("sgl_qmoe_shared failed")
    return out


_mlp = _sig("sgl_qmlp_forward", _I, _P, _P, _P, _P, _I, _I64, _P, _P)
_qrows_dev = _sig("sgl_quant_rows_i8_dev", _I, _P, _P, _P, _I64, _I64, _P)
_dqrows_dev = _sig("sgl_dequant_rows_i8_dev", _I, _P, _P, _P, _I64, _I64, _P)


def qmlp_forward(gate, up, down, h, out=None):
    """Dense SwiGLU MLP of h [T, E] (device): up None means gate is the fused [2I, E] weight."""
    import torch
    h = h.contiguous()
    if out is None:
        out = torch.empty((h.shape[0], down.N), dtype=torch.float32, device=h.device)
    if _mlp(gate.h, None if up is None else up.h, down.h, C.c_void_p(h.data_ptr()),
            _dtype_code(h), h.shape[0], C.c_void_p(out.data_ptr()), _stream()) != 0:
        raise RuntimeError("sgl_qmlp_forward failed")
    return out


def quant_rows_i8_dev(x):
    """x f32 [rows, dim] device tensor -> (int8 [rows, dim], f32 scales [rows]) on the device."""
    import torch
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    if _qrows_dev(C.c_void_p(x.data_ptr()), C.c_void_p(q.data_ptr()), C.c_void_p(s.data_ptr()),
                  x.shape[0], x.shape[1], _stream()) != 0:
        raise RuntimeError("sgl_quant_rows_i8_dev failed")
    return q, s


def dequant_rows_i8_dev(q, scales):
    import torch
    q, scales = q.contiguous(), scales.contiguous()
    o = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    if _dqrows_dev(C.c_void_p(q.data_ptr()), C.c_void_p(scales.data_ptr()),
                   C.c_void_p(o.data_ptr()), q.shape[0], q.shape[1], _stream()) != 0:
        raise RuntimeError("sgl_dequant_rows_i8_dev failed")
    return o
