"""Pinning of the oracle's MoE routing (orc_moe_route, reference src/deepseek.c:593-633) and
shared-expert add (orc_moe_shared, :679-687) by independent formulations: numpy sorts and
masks instead of greedy scans, float64 brute force, and hand-built ties / masked groups."""
import numpy as np
import pytest


def np_route(lg, k, bias=None, sigmoid=True, n_group=0, topk_group=0, norm=True, scale=1.0):
    lg = lg.astype(np.float32)
    T, ne = lg.shape
    if sigmoid:
        s = (1.0 / (1.0 + np.exp(-lg.astype(np.float64)))).astype(np.float32)
    else:
        e = np.exp((lg - lg.max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float32)
        s = e * (1.0 / e.astype(np.float64).sum(axis=1, keepdims=True)).astype(np.float32)
    ch = s + (0 if bias is None else bias.astype(np.float32))
    if n_group > 1:
        epg = ne // n_group
        g = ch.reshape(T, n_group, epg)
        top = -np.sort(-g, axis=2)
        gs = top[:, :, 0] + (top[:, :, 1] if epg > 1 else 0)
        keep = np.argsort(-gs, axis=1, kind="stable")[:, :topk_group]
        mask = np.ones((T, n_group), bool)
        np.put_along_axis(mask, keep, False, axis=1)
        ch = np.where(np.repeat(mask, epg, axis=1), np.float32(-1e30), ch)
    order = np.argsort(-ch, axis=1, kind="stable")[:, :k]
    ids = np.where(np.take_along_axis(ch, order, 1) > np.float32(-1e30), order, -1)
    w = np.where(ids >= 0, np.take_along_axis(s, np.maximum(ids, 0), 1), 0).astype(np.float32)
    if norm and k > 1:
        w = (w / (w.astype(np.float64).sum(axis=1, keepdims=True) + 1e-20)).astype(np.float32)
    return ids.astype(np.int32), (w * np.float32(scale)).astype(np.float32)


@pytest.mark.parametrize("ne,k,sig,ng,tg,bias,norm", [
    (64, 6, True, 8, 3, True, True), (64, 6, False, 0, 0, False, True),
    (256, 8, True, 8, 4, True, True), (16, 1, True, 0, 0, False, True),
    (32, 4, False, 4, 2, False, False), (8, 2, True, 8, 3, True, True)])
def test_route_matches_numpy(orc, ne, k, sig, ng, tg, bias, norm):
    rng = np.random.default_rng(ne * 100 + k)
    lg = rng.standard_normal((40, ne)).astype(np.float32) * 2
    b = rng.standard_normal(ne).astype(np.float32) * 0.1 if bias else None
    ids, w = orc.moe_route(lg, k, b, sig, ng, tg, norm, 2.5)
    ids2, w2 = np_route(lg, k, b, sig, ng, tg, norm, 2.5)
    assert np.array_equal(ids, ids2)
    np.testing.assert_allclose(w, w2, rtol=2e-6, atol=0)


def test_route_ties_go_to_lower_index(orc):
    lg = np.array([[0.5, 1.0, 1.0, 0.2, 1.0, 1.0]], np.float32)
    ids, _ = orc.moe_route(lg, 3, sigmoid=True)
    assert ids.tolist() == [[1, 2, 4]]
    # group scores tie (groups 0 and 2): the lower group wins
    lg = np.array([[1.0, 1.0, 0.0, 0.0, 1.0, 1.0, 0.5, 0.5]], np.float32)
    ids, _ = orc.moe_route(lg, 2, sigmoid=True, n_group=4, topk_group=1)
    assert ids.tolist() == [[0, 1]]


def test_route_masked_groups_leave_slots_empty(orc):
    """Fewer unmasked experts than k: the rest are -1 with weight 0."""
    lg = np.arange(16, dtype=np.float32)[None, :]
    ids, w = orc.moe_route(lg, 6, sigmoid=True, n_group=4, topk_group=1, norm=True)
    assert ids.tolist() == [[15, 14, 13, 12, -1, -1]]
    assert w[0, 4] == 0 and w[0, 5] == 0
    np.testing.assert_allclose(w[0, :4].sum(), 1.0, rtol=1e-6)


def test_route_weights_use_uncorrected_scores(orc):
    """The correction bias changes the choice, the weight is the plain score; k = 1 is not
    normalised; the scale multiplies."""
    lg = np.array([[2.0, 0.0]], np.float32)
    ids, w = orc.moe_route(lg, 1, bias=np.array([0, 10], np.float32), sigmoid=True, norm=True,
                           scale=3.0)
    assert ids.tolist() == [[1]]
    assert w[0, 0] == np.float32(np.float32(0.5) * np.float32(3.0))


def test_route_single_expert_groups(orc):
    """Groups of one expert: the group score is that expert's (no second term)."""
    lg = np.array([[0.1, 3.0, 2.0, -1.0]], np.float32)
    ids, _ = orc.moe_route(lg, 2, sigmoid=True, n_group=4, topk_group=2)
    assert ids.tolist() == [[1, 2]]


def test_shared_matches_float64(orc):
    rng = np.random.default_rng(5)
    T, E, sh = 3, 48, 20
    h = rng.standard_normal((T, E)).astype(np.float32)
    wg, wu = (rng.standard_normal((sh, E)).astype(np.float32) * 0.1 for _ in range(2))
    wd = rng.standard_normal((E, sh)).astype(np.float32) * 0.1
    base = rng.standard_normal((T, E)).astype(np.float32)
    out = orc.moe_shared(h, wg, wu, wd, base.copy())
    g = h.astype(np.float64) @ wg.T.astype(np.float64)
    u = h.astype(np.float64) @ wu.T.astype(np.float64)
    ref = base + ((g / (1 + np.exp(-g))) * u) @ wd.T.astype(np.float64)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
