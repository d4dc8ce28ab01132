"""Load path on the host: the safetensors reader (sgl_qst_*) and sgl_qlinear_probe, which
makes the decisions of the reference loader's quant_get (reference src/safetensors.c:271-471)
without a device: tensor names, dtype checks, N/K, Marlin fallback, AWQ orientation."""
import numpy as np
import pytest
from safetensors.numpy import save_file

import sgl_qlinear as q
from qload_cases import write_weight

BASE = "model.layers.0.mlp.up_proj"


def _probe(path, cfg, base=BASE):
    st = q.SafeTensors(path)
    try:
        return st.probe(q.make_cfg(**cfg), base)
    finally:
        st.close()


def test_reader_views(tmp_path):
    t = {"a": np.arange(12, dtype=np.int32).reshape(3, 4), "b": np.ones((2, 3, 4, 5), np.float16),
         "c": np.array([7], np.int64), "s": np.array(3.0, np.float32)}
    save_file(t, str(tmp_path / "x.safetensors"))
    st = q.SafeTensors(tmp_path / "x.safetensors")
    dt, dims, data = st.get_raw("a")
    assert (dt, dims) == ("I32", (3, 4)) and data == t["a"].tobytes()
    dt, dims, data = st.get_raw("b")
    assert (dt, dims) == ("F16", (2, 3, 4, 5)) and data == t["b"].tobytes()
    assert st.get_raw("c")[:2] == ("I64", (1,))
    assert st.get_raw("s") is None  # 0-d tensors are not found, as the reference's shard_raw
    assert st.get_raw("missing") is None
    st.close()


def test_reader_rejects_bad_files(tmp_path):
    (tmp_path / "short").write_bytes(b"abc")
    with pytest.raises(RuntimeError):
        q.SafeTensors(tmp_path / "short")
    (tmp_path / "over").write_bytes((1000).to_bytes(8, "little") + b"{}")
    with pytest.raises(RuntimeError):
        q.SafeTensors(tmp_path / "over")
    (tmp_path / "arr").write_bytes((2).to_bytes(8, "little") + b"[]")
    with pytest.raises(RuntimeError):
        q.SafeTensors(tmp_path / "arr")


@pytest.mark.parametrize("fmt,N,K,kind,tr", [
    ("gptq4", 96, 256, "natural", 0), ("gptq4_act", 96, 256, "natural", 0),
    ("gptq8", 96, 256, "natural", 0), ("awq4", 96, 256, "natural", 0),
    ("awq4_gemv", 96, 256, "natural", 1), ("marlin4_asym", 128, 256, "marlin", 0),
    ("marlin8_sym", 128, 256, "marlin", 0), ("ct4", 96, 256, "ct", 0), ("ct8", 96, 200, "ct", 0),
    ("mxfp4", 96, 256, "mxfp4", 0)])
def test_probe_formats(tmp_path, fmt, N, K, kind, tr):
    p = tmp_path / "w.safetensors"
    _, _, cfg = write_weight(p, fmt, N, K)
    rc, info = _probe(p, cfg)
    assert rc == 1 and info["kind"] == kind and (info["N"], info["K"]) == (N, K), info
    assert info["transposed"] == tr


def test_awq_orientation_from_shapes(tmp_path):
    """A gemv-layout AWQ weight under a config that says gemm is read as gemv; a square weight
    follows the config (reference src/safetensors.c:400-418)."""
    p = tmp_path / "w.safetensors"
    _, _, cfg = write_weight(p, "awq4_gemv", 96, 256)
    cfg["transposed"] = 0
    rc, info = _probe(p, cfg)
    assert rc == 1 and info["transposed"] == 1 and (info["N"], info["K"]) == (96, 256)
    _, _, cfg = write_weight(p, "awq4", 128, 128)
    rc, info = _probe(p, cfg)
    assert rc == 1 and info["transposed"] == 0


def test_marlin_shape_mismatch_falls_back(tmp_path):
    """A config that says Marlin over natural-layout tensors is read in the natural layout."""
    p = tmp_path / "w.safetensors"
    _, _, cfg = write_weight(p, "gptq4", 128, 256)
    cfg["layout"] = 1
    rc, info = _probe(p, cfg)
    assert rc == 1 and info["kind"] == "natural" and info["layout"] == 0


def test_ct_without_weight_shape(tmp_path):
    """Without weight_shape, K = packed columns x codes per word."""
    p = tmp_path / "w.safetensors"
    _, a, cfg = write_weight(p, "ct4", 96, 256)
    save_file({BASE + ".weight_packed": np.asarray(a["wpacked"], np.int32),
               BASE + ".weight_scale": np.asarray(a["scales"], np.float32)}, str(p))
    rc, info = _probe(p, cfg)
    assert rc == 1 and (info["N"], info["K"]) == (96, 256)


def test_probe_errors(tmp_path):
    p = tmp_path / "w.safetensors"
    _, a, cfg = write_weight(p, "gptq4", 96, 256)
    qw, qz, sc = a["qweight"], a["qzeros"], a["scales"].astype(np.float16)
    assert _probe(p, cfg, base="model.other")[0] == 0          # nothing under that name
    save_file({BASE + ".qweight": qw, BASE + ".qzeros": qz}, str(p))
    assert _probe(p, cfg)[0] == -1                              # no scales
    save_file({BASE + ".qweight": qw.astype(np.float32), BASE + ".qzeros": qz,
               BASE + ".scales": sc}, str(p))
    assert _probe(p, cfg)[0] == -1                              # qweight not I32
    save_file({BASE + ".qweight": qw, BASE + ".scales": sc}, str(p))
    assert _probe(p, cfg)[0] == -1                              # zero_point without qzeros
    save_file({BASE + ".qweight": qw, BASE + ".qzeros": qz, BASE + ".scales": sc[:1]}, str(p))
    assert _probe(p, cfg)[0] == -1                              # scale rows != K / G
    save_file({BASE + ".qweight": qw, BASE + ".qzeros": qz,
               BASE + ".scales": sc.astype(np.int32)}, str(p))
    assert _probe(p, cfg)[0] == -1                              # scales dtype
    _, a, cfg = write_weight(p, "awq4", 96, 256)
    save_file({BASE + ".qweight": np.zeros((256, 7), np.int32), BASE + ".qzeros": a["qzeros"],
               BASE + ".scales": a["scales"].astype(np.float16)}, str(p))
    assert _probe(p, cfg)[0] == -1                              # AWQ shapes fit neither layout
