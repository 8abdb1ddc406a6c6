"""Pins the oracle's MoE routing, grouping and combine against brute force and closed forms."""
import math

import numpy as np
import pytest

from oracle import aq_oracle as orc


def _brute_route(row, k):
    """Sort by (-logit, index); weights = softmax over the k winners (moek.mojo:156-197)."""
    order = sorted(range(len(row)), key=lambda i: (-float(row[i]), i))[:k]
    top = [float(row[i]) for i in order]
    ex = [math.exp(v - top[0]) for v in top]
    return order, [v / sum(ex) for v in ex]


def test_route_brute_force_and_ties():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((20, 128)).astype(np.float32)
    logits[3, :] = 0.0
    logits[4, [9, 2, 70]] = 5.0
    ids, w = orc.route_top8(logits)
    for t in range(20):
        o, ww = _brute_route(logits[t], 8)
        assert ids[t].tolist() == o
        np.testing.assert_allclose(w[t], ww, rtol=1e-12)
    assert ids[3].tolist() == list(range(8))
    assert ids[4, :3].tolist() == [2, 9, 70]


def test_route_equals_softmax_topk_renormalise():
    """w_k = exp(l_k - l_max) / sum_top exp(.) equals softmax over all experts, top-k, renormalised (the
    transformers Qwen3-MoE router with norm_topk_prob)."""
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((16, 128))
    ids, w = orc.route_top8(logits.astype(np.float32))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for t in range(16):
        sel = p[t, ids[t]]
        np.testing.assert_allclose(w[t], sel / sel.sum(), rtol=1e-6)
        assert np.all(np.diff(logits[t, ids[t]]) <= 0)


def test_expert_lists_items_brute_force():
    rng = np.random.default_rng(2)
    t, e, k = 30, 16, 4
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)])
    lists, counts = orc.expert_lists(ids, e, t)
    flat = ids.ravel()
    for ex in range(e):
        want = [i for i in range(t * k) if flat[i] == ex]  # ascending i (moek.mojo:438-441)
        assert counts[ex] == len(want)
        assert lists[ex, :len(want)].tolist() == want
        assert np.all(lists[ex, len(want):] == -1)
    items = orc.expert_items(counts, 8)
    want_items = [(ex, c) for ex in range(e) for c in range(0, counts[ex], 8)]
    assert [tuple(r) for r in items.tolist()] == want_items


@pytest.mark.parametrize("tm", [1, 8, 32])
def test_p_group_brute_force(tm):
    rng = np.random.default_rng(3)
    t, e, k = 25, 8, 3
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)])
    g = orc.p_group(ids, e, tm)
    flat = ids.ravel()
    off = 0
    tiles = []
    for ex in range(e):
        members = [i for i in range(t * k) if flat[i] == ex]
        assert g["cnt"][ex] == len(members)
        assert g["offs"][ex] == off
        for r, i in enumerate(members):
            assert g["slot"][i] == off + r
            assert g["src"][off + r] == i // k
        padded = -(-len(members) // tm) * tm
        assert np.all(g["src"][off + len(members):off + padded] == -1)
        tiles += [(ex, off + c) for c in range(0, len(members), tm)]
        off += padded
    assert g["rows_total"] == off
    assert [tuple(r) for r in g["tiles"].tolist()] == tiles


def test_gather_combine_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 6))
    src = np.array([2, -1, 0, 4, -1])
    xg = orc.p_gather(x, src)
    assert np.all(xg[1] == 0) and np.all(xg[4] == 0) and np.all(xg[0] == x[2])
    yd = rng.standard_normal((7, 6))
    slot = np.array([3, 0, 6, 1])
    w = np.array([[0.25, 0.75], [0.5, 0.5]])
    y = orc.p_combine(yd, slot, w)
    np.testing.assert_allclose(y[0], 0.25 * yd[3] + 0.75 * yd[0])
    np.testing.assert_allclose(y[1], 0.5 * yd[6] + 0.5 * yd[1])


def test_moe_layer_per_token_brute_force():
    """The grouped oracle equals a per-token dense evaluation of the selected experts."""
    rng = np.random.default_rng(5)
    t, e, d, f, g = 6, 4, 64, 32, 32
    gu_q = rng.integers(0, 2 ** 32, (e * 2 * f, d // 8), dtype=np.uint32)
    gu_s = (rng.random((e * 2 * f, d // g)) * 0.05 + 0.01).astype(np.float16)
    dn_q = rng.integers(0, 2 ** 32, (e * d, f // 8), dtype=np.uint32)
    dn_s = (rng.random((e * d, f // g)) * 0.05 + 0.01).astype(np.float16)
    x = rng.standard_normal((t, d)).astype(np.float32)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    y, ids, w = orc.moe_layer(x, logits, gu_q, gu_s, dn_q, dn_s, g, f, topk=2)
    gu = orc.q4w_dequant(gu_q, gu_s, g).astype(np.float64)
    dn = orc.q4w_dequant(dn_q, dn_s, g).astype(np.float64)
    for tt in range(t):
        acc = np.zeros(d)
        for kk in range(2):
            ex = ids[tt, kk]
            h = gu[ex * 2 * f:(ex + 1) * 2 * f] @ x[tt].astype(np.float64)
            a = h[:f] / (1 + np.exp(-h[:f])) * h[f:]
            acc += w[tt, kk] * (dn[ex * d:(ex + 1) * d] @ a)
        np.testing.assert_allclose(y[tt], acc, rtol=1e-10, atol=1e-12)


def test_cpu_baseline_restatements_match_the_oracle():
    """bench.py's CPU baseline computes what the oracle computes: its transformers-style MoE block (softmax, top-k,
    renormalise, per-expert loop with index_add_) and its ternary dequantisation (the float64 oracle, to fp32
    rounding), so the time it reports is for the same work."""
    from aq import synth
    from oracle import cpu_baseline as cb
    d = synth.c3(tokens=24, experts=8, hidden=64, ffn=32)
    got = cb.moe_forward(d, topk=2)().numpy()
    ref, _, _ = orc.moe_layer(d["x"], d["logits"], d["gu_q"], d["gu_s"], d["dn_q"], d["dn_s"], 32, 32, topk=2)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5 * np.abs(ref).max())
    rng = np.random.default_rng(5)
    w, s = synth.ternary_matrix(rng, 48, 256)
    np.testing.assert_array_equal(cb.dequant_t2(w, s).numpy(), orc.t2w_dequant(w, s).astype(np.float32))
