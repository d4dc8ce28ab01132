"""A HIP graph captured from a small call keeps working after a larger eager call on the same
handle has outgrown its workspace: the outgrown buffer stays allocated until the handle is
destroyed.  Replays are compared with the eager result of the same call, bit for bit."""
import numpy as np
import pytest

import synth
from linear_cases import build, product

pytestmark = pytest.mark.gpu


def _capture(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # sizes the workspace for this call
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_linear_graph_after_larger_eager_call():
    import torch
    kind, a = build("gptq4", 1024, 2048, seed=41)
    ql = product(kind, a, 1024, 2048)
    A = torch.from_numpy(synth.normal(42, (64, 2048))).cuda().to(torch.bfloat16)
    out = torch.empty((64, 1024), device="cuda")
    ref = ql.forward(A).clone()
    g = _capture(torch, lambda: ql.forward(A, out=out))
    big = torch.from_numpy(synth.normal(43, (2048, 2048))).cuda().to(torch.bfloat16)
    for i in range(3):
        ql.forward(big)  # grows the handle's workspace
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i


def test_moe_graph_after_larger_eager_call():
    import torch
    import sgl_qlinear as q
    n_exp, E, mi, k = 8, 256, 128, 2
    gu, dn = [], []
    for e in range(n_exp):
        kind, a = build("gptq4", 2 * mi, E, seed=50 + 2 * e)
        gu.append(product(kind, a, 2 * mi, E))
        kind, a = build("gptq4", E, mi, seed=51 + 2 * e)
        dn.append(product(kind, a, E, mi))
    ids, wts = synth.moe_routing(60, 1, n_exp, k)
    tid, tw = torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda()
    h = torch.from_numpy(synth.normal(61, (1, E))).cuda().to(torch.bfloat16)
    out = torch.empty((1, E), device="cuda")
    ref = q.qmoe_forward(gu, dn, h, tid, tw).clone()
    g = _capture(torch, lambda: q.qmoe_forward(gu, dn, h, tid, tw, out=out))
    ids2, wts2 = synth.moe_routing(62, 512, n_exp, k)
    h2 = torch.from_numpy(synth.normal(63, (512, E))).cuda().to(torch.bfloat16)
    for i in range(3):
        q.qmoe_forward(gu, dn, h2, torch.from_numpy(ids2).cuda(), torch.from_numpy(wts2).cuda())
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
