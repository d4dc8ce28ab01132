"""The steps either side of the quantized linear, on the GPU: the dense SwiGLU MLP block
(reference src/llama.c:1162-1176, against the oracle's sgl_matmul_nt composition) with fused
or separate gate/up weights, and the int8 KV-row quantization on device pointers (bit for bit
against the oracle's sgl_quant_rows_i8)."""
import numpy as np
import pytest

import synth
from linear_cases import rel_err
from oracle.oracle import make_cfg as ocfg

pytestmark = pytest.mark.gpu
CFG = dict(method=2, bits=4, group_size=128, zero_point=1)


def _gptq(orc, seed, N, K):
    c, z, s = synth.quantize_groups(synth.normal(seed, (N, K), 0.02), 128)
    qw, qz = synth.gptq_pack(c, z)
    rc, W = orc.dequant(ocfg(**CFG), qw, s, N, K, qzeros=qz)
    assert rc == 0
    return (qw, qz, s), W


def _ql(parts, N, K):
    import sgl_qlinear as q
    qw, qz, s = parts
    return q.QLinear.from_awq_gptq(q.make_cfg(**CFG), qw, s, N, K, qzeros=qz)


@pytest.mark.parametrize("T", [3, 40])
def test_qmlp_fused_and_separate(orc, T):
    import torch
    import sgl_qlinear as q
    E, I = 512, 384
    pg, wg = _gptq(orc, 1, I, E)
    pu, wu = _gptq(orc, 2, I, E)
    pd, wd = _gptq(orc, 3, E, I)
    # the fused gate/up weight: the same codes, gate columns then up columns
    pf = tuple(np.concatenate([a, b], axis=1) for a, b in zip(pg, pu))
    gate, up, down, fused = _ql(pg, I, E), _ql(pu, I, E), _ql(pd, E, I), _ql(pf, 2 * I, E)
    h = synth.normal(4, (T, E))
    th = torch.from_numpy(h).cuda()
    ref = orc.moe_shared(h, wg, wu, wd, np.zeros((T, E), np.float32))
    print(f"[gpu] qmlp T={T}", flush=True)
    assert rel_err(q.qmlp_forward(gate, up, down, th).cpu().numpy(), ref) <= 1e-3
    assert rel_err(q.qmlp_forward(fused, None, down, th).cpu().numpy(), ref) <= 1e-3
    hb = synth.bf16_bits_to_f32(synth.to_bf16_bits(h))
    refb = orc.moe_shared(hb, wg, wu, wd, np.zeros((T, E), np.float32))
    y = q.qmlp_forward(fused, None, down, torch.from_numpy(hb).cuda().to(torch.bfloat16))
    assert rel_err(y.cpu().numpy(), refb) <= 1e-3


def test_kv_quant_dev_bit_exact(orc):
    import torch
    import sgl_qlinear as q
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((64, 576)) * 3).astype(np.float32)
    x[5] = 0                                        # zero row: scale 0, codes 0
    x[6] = np.float32(1e-40) * rng.standard_normal(576).astype(np.float32)  # denormals
    x[7, :4] = [127.0, 63.5, -63.5, 0.5]            # exact .5 ties after scaling
    s_ref, q_ref = orc.quant_rows_i8(x)
    qd, sd = q.quant_rows_i8_dev(torch.from_numpy(x).cuda())
    assert np.array_equal(qd.cpu().numpy(), q_ref)
    assert np.array_equal(sd.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    back = q.dequant_rows_i8_dev(qd, sd).cpu().numpy()
    assert np.array_equal(back, q_ref.astype(np.float32) * s_ref[:, None])


def test_empty_batches():
    """Zero rows through every device entry point returns at once, with the empty tensors'
    NULL data pointers: forward, MoE forward, router logits, routing, shared experts, dense
    MLP and the int8 row quant/dequant."""
    import torch
    import sgl_qlinear as q
    import synth
    E, I = 256, 128
    c, z, s = synth.quantize_groups(synth.normal(3, (2 * I, E), 0.02), 128)
    qw, qz = synth.gptq_pack(c, z)
    cfg = q.make_cfg(method=2, bits=4, group_size=128, zero_point=1)
    gu = q.QLinear.from_awq_gptq(cfg, qw, s, 2 * I, E, qzeros=qz)
    c, z, s = synth.quantize_groups(synth.normal(4, (E, I), 0.02), 128)
    qw, qz = synth.gptq_pack(c, z)
    dn = q.QLinear.from_awq_gptq(cfg, qw, s, E, I, qzeros=qz)
    h = torch.empty((0, E), device="cuda")
    print("[gpu] empty batches", flush=True)
    assert gu.forward(h).shape == (0, 2 * I)
    ids = torch.empty((0, 2), dtype=torch.int32, device="cuda")
    wts = torch.empty((0, 2), dtype=torch.float32, device="cuda")
    assert q.qmoe_forward([gu], [dn], h, ids, wts).shape == (0, E)
    w = torch.randn(4, E, device="cuda")
    lg = q.qmoe_router_logits(w, h)
    assert lg.shape == (0, 4)
    i2, w2 = q.qmoe_route(lg, 2)
    assert i2.shape == (0, 2) and w2.shape == (0, 2)
    out = torch.empty((0, E), device="cuda")
    q.qmoe_shared(gu, dn, h, out)
    assert q.qmlp_forward(gu, None, dn, h).shape == (0, E)
    qq, sc = q.quant_rows_i8_dev(torch.empty((0, E), device="cuda"))
    assert q.dequant_rows_i8_dev(qq, sc).shape == (0, E)
    torch.cuda.synchronize()
