"""Load path on the GPU: sgl_qlinear_load from a safetensors file gives the weight that the
reference loader's quant_get + sgl_qweight_dequant* would (bit for bit), and the same device
bits as creating it from the buffers directly; its forward meets the matmul tolerance."""
import numpy as np
import pytest

import synth
import sgl_qlinear as q
from linear_cases import oracle_forward, oracle_weight, product, rel_err
from qload_cases import write_weight

pytestmark = pytest.mark.gpu
TOL = 1e-3
BASE = "model.layers.3.self_attn.o_proj"


def _load(path, cfg):
    st = q.SafeTensors(path)
    c = q.make_cfg(**cfg)
    ql = q.QLinear.load(c, st, BASE)
    st.close()  # the handle keeps its own device copy
    return ql, c


@pytest.mark.parametrize("fmt,N,K", [
    ("gptq4", 200, 512), ("gptq4_act", 200, 512), ("gptq8", 200, 512), ("gptq4_v2", 200, 512),
    ("awq4", 200, 512), ("awq4_gemv", 200, 512), ("marlin4_asym", 256, 512),
    ("marlin8_sym", 256, 512), ("ct4", 200, 512), ("ct8", 200, 384), ("mxfp4", 200, 512)])
def test_load_matches_reference(orc, tmp_path, fmt, N, K):
    import torch
    p = tmp_path / "w.safetensors"
    kind, a, cfg = write_weight(p, fmt, N, K, base=BASE, seed=17)
    print(f"[gpu] load {fmt} N={N} K={K}", flush=True)
    ql, c = _load(p, cfg)
    assert (ql.N, ql.K) == (N, K)
    W = oracle_weight(orc, kind, a, N, K)
    got = ql.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), W.view(np.uint32)), fmt
    direct = product(kind, a, N, K)
    assert torch.equal(direct.dequant(), ql.dequant())
    A = synth.normal(18, (5, K))
    y = ql.forward(torch.from_numpy(A).cuda()).cpu().numpy()
    assert rel_err(y, oracle_forward(orc, kind, a, W, A)) <= TOL


@pytest.mark.parametrize("sdt", ["BF16", "F32"])
def test_load_scale_dtypes(orc, tmp_path, sdt):
    p = tmp_path / "w.safetensors"
    kind, a, cfg = write_weight(p, "gptq4", 128, 512, base=BASE, seed=19, scale_dtype=sdt)
    print(f"[gpu] load gptq4 scales {sdt}", flush=True)
    ql, _ = _load(p, cfg)
    W = oracle_weight(orc, kind, a, 128, 512)
    assert np.array_equal(ql.dequant().cpu().numpy().view(np.uint32), W.view(np.uint32))


def test_load_marlin_fallback_and_awq_orientation(orc, tmp_path):
    """Config says Marlin but the tensors are natural: read natural; config says AWQ gemm but
    the tensors are gemv: read gemv and report it in cfg.transposed."""
    p = tmp_path / "w.safetensors"
    kind, a, cfg = write_weight(p, "gptq4", 128, 512, base=BASE, seed=23)
    cfg["layout"] = 1
    ql, _ = _load(p, cfg)
    W = oracle_weight(orc, kind, a, 128, 512)
    assert np.array_equal(ql.dequant().cpu().numpy().view(np.uint32), W.view(np.uint32))
    kind, a, cfg = write_weight(p, "awq4_gemv", 128, 512, base=BASE, seed=29)
    cfg["transposed"] = 0
    ql, c = _load(p, cfg)
    assert c.transposed == 1
    W = oracle_weight(orc, kind, a, 128, 512)
    assert np.array_equal(ql.dequant().cpu().numpy().view(np.uint32), W.view(np.uint32))


def test_load_missing_tensors_returns_none(tmp_path):
    p = tmp_path / "w.safetensors"
    _, _, cfg = write_weight(p, "gptq4", 128, 512, base=BASE)
    st = q.SafeTensors(p)
    with pytest.raises(RuntimeError):
        q.QLinear.load(q.make_cfg(**cfg), st, "model.layers.9.mlp.gate_proj")
    st.close()
