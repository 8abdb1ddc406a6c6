"""MoE path on the GPU vs the oracle: routing, grouping, lists/items, grouped GEMM, combine, decode experts, router
GEMV, and the whole C3 block (qwen3moe/kernels/moek.mojo, lfm2moe/kernels/mk.mojo)."""
import numpy as np
import pytest

from _util import exact_int4_product, kat_int4, rel_inf, to_dev, to_np
from oracle import aq_oracle as orc

pytestmark = pytest.mark.gpu


def _i32(a, dev):
    return to_dev(np.asarray(a, np.int32), dev)


@pytest.mark.parametrize("t,e,k", [(404, 128, 8), (1, 128, 8), (37, 32, 4), (5, 256, 8), (3, 64, 2)])
def test_route_bit_exact_ids(dev, t, e, k):
    import torch
    rng = np.random.default_rng(t + e)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    ids = torch.empty((t, k), dtype=torch.int32, device=dev)
    w = torch.empty((t, k), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_route(to_dev(logits, dev), ids, w, k)
    rid, rw = orc.route_top8(logits, k)
    np.testing.assert_array_equal(to_np(ids), rid)
    np.testing.assert_allclose(to_np(w), rw, rtol=2e-6, atol=1e-7)


def test_route_ties_lowest_index(dev):
    """Forced ties: equal logits are taken in ascending expert order (moek.mojo:178)."""
    import torch
    logits = np.zeros((3, 128), np.float32)
    logits[1, [5, 77, 3, 100]] = 1.0          # four tied winners, then ties among the zeros
    logits[2] = np.repeat(np.arange(64, dtype=np.float32), 2)[::-1]  # pairs of equal values
    ids = torch.empty((3, 8), dtype=torch.int32, device=dev)
    w = torch.empty((3, 8), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_route(to_dev(logits, dev), ids, w, 8)
    got = to_np(ids)
    np.testing.assert_array_equal(got[0], np.arange(8))
    np.testing.assert_array_equal(got[1], [3, 5, 77, 100, 0, 1, 2, 4])
    np.testing.assert_array_equal(got, orc.route_top8(logits)[0])


@pytest.mark.parametrize("t,e,k,d", [(404, 128, 8, 2048), (5, 256, 8, 64), (3, 64, 2, 8), (9, 33, 3, 24)])
def test_route_pack(dev, t, e, k, d):
    """The fused routing + fp16 rounding of x: ids and weights bit-equal to moe_route's, xq = fp16(x) (RNE)."""
    import torch
    rng = np.random.default_rng(t * 7 + d)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    x = (rng.standard_normal((t, d)) * 3).astype(np.float32)
    x[0, :4] = [1e-8, 65504.0, -70000.0, 2.0 ** -24 * 1.5]  # fp16 subnormal, max, overflow, a rounding tie
    ids = torch.empty((t, k), dtype=torch.int32, device=dev)
    w = torch.empty((t, k), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_route(to_dev(logits, dev), ids, w, k)
    ids2 = torch.empty_like(ids)
    w2 = torch.empty_like(w)
    xq = torch.empty((t, d // 2), dtype=torch.int32, device=dev)
    torch.ops.aq.moe_route_pack(to_dev(logits, dev), ids2, w2, k, to_dev(x, dev), xq)
    np.testing.assert_array_equal(to_np(ids2), to_np(ids))
    np.testing.assert_array_equal(to_np(w2).view(np.uint32), to_np(w).view(np.uint32))
    with np.errstate(over="ignore"):  # -70000 rounds to -inf in fp16, as intended
        want = x.astype(np.float16)
    np.testing.assert_array_equal(to_np(xq).view(np.uint16).reshape(t, d), want.view(np.uint16))


def test_route_minus_infinity_logits(dev):
    """-inf logits are ranked by index after the finite ones, none taken twice; their weights are 0."""
    import torch
    logits = np.full((2, 128), -np.inf, np.float32)
    logits[0, [90, 7, 30]] = [0.5, 0.5, -1.0]
    logits[1, :] = np.arange(128, dtype=np.float32)
    logits[1, [1, 2]] = -np.inf
    ids = torch.empty((2, 8), dtype=torch.int32, device=dev)
    w = torch.empty((2, 8), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_route(to_dev(logits, dev), ids, w, 8)
    rid, rw = orc.route_top8(logits, 8)
    np.testing.assert_array_equal(to_np(ids), rid)
    np.testing.assert_array_equal(to_np(ids)[0], [7, 90, 30, 0, 1, 2, 3, 4])
    np.testing.assert_allclose(to_np(w), rw, rtol=2e-6, atol=1e-7)
    assert (to_np(w)[0, 3:] == 0).all()


@pytest.mark.parametrize("t,e,k,tm", [(404, 128, 8, 32), (404, 128, 8, 16), (50, 8, 2, 48), (1, 128, 8, 32),
                                      (1000, 128, 8, 64), (7, 3, 3, 16)])
def test_group_bit_exact(dev, t, e, k, tm):
    import torch
    from aq import _lib
    rng = np.random.default_rng(t * 3 + e + tm)
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    ref = orc.p_group(ids, e, tm)
    max_rows = _lib.lib().aq_moe_group_max_rows(t, k, e, tm)
    max_tiles = _lib.lib().aq_moe_group_max_tiles(t, k, e, tm)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, offs, slot = torch.empty(e, **i32), torch.empty(e + 1, **i32), torch.empty(t * k, **i32)
    src, tiles, nt = torch.empty(max_rows, **i32), torch.empty(2 * max_tiles, **i32), torch.empty(1, **i32)
    torch.ops.aq.moe_group(_i32(ids, dev), e, tm, counts, offs, slot, src, tiles, nt)
    np.testing.assert_array_equal(to_np(counts), ref["cnt"])
    np.testing.assert_array_equal(to_np(offs)[:e], ref["offs"])
    assert int(to_np(offs)[e]) == ref["rows_total"]
    np.testing.assert_array_equal(to_np(slot), ref["slot"])
    got_src = to_np(src)
    np.testing.assert_array_equal(got_src[:ref["rows_total"]], ref["src"])
    assert np.all(got_src[ref["rows_total"]:] == -1)
    n_t = int(to_np(nt)[0])
    assert n_t == len(ref["tiles"])
    np.testing.assert_array_equal(to_np(tiles)[:2 * n_t].reshape(-1, 2), ref["tiles"])


def test_expert_lists_and_items(dev):
    """qwen3moe's p_expert_lists / p_expert_items order."""
    import torch
    rng = np.random.default_rng(4)
    t, e, k = 200, 128, 8
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    lists_ref, counts_ref = orc.expert_lists(ids, e, t)
    items_ref = orc.expert_items(counts_ref, 8)
    i32 = dict(dtype=torch.int32, device=dev)
    lists, counts = torch.full((e, t), -1, **i32), torch.empty(e, **i32)
    items, nitems = torch.empty(2 * (t * k // 8 + e), **i32), torch.empty(1, **i32)
    scratch = torch.empty(e + 1 + 4 * t * k + 1, **i32)
    torch.ops.aq.moe_expert_lists(_i32(ids, dev), e, lists, counts, 8, items, nitems, scratch)
    np.testing.assert_array_equal(to_np(counts), counts_ref)
    got = to_np(lists)
    for ex in range(e):
        np.testing.assert_array_equal(got[ex, :counts_ref[ex]], lists_ref[ex, :counts_ref[ex]])
    n_i = int(to_np(nitems)[0])
    np.testing.assert_array_equal(to_np(items)[:2 * n_i].reshape(-1, 2), items_ref)


def _small_moe(rng, e, d, f, g, kat=False):
    if kat:
        gu_v, gu_s, _ = kat_int4(rng, e * 2 * f, d, g)
        dn_v, dn_s, _ = kat_int4(rng, e * d, f, g)
        return orc.q4w_pack(gu_v), gu_s, orc.q4w_pack(dn_v), dn_s, gu_v, dn_v
    from aq import synth
    gu_q, gu_s = synth.int4_matrix(rng, e * 2 * f, d, g)
    dn_q, dn_s = synth.int4_matrix(rng, e * d, f, g)
    return gu_q, gu_s, dn_q, dn_s, None, None


@pytest.mark.parametrize("d,n,g", [(256, 96, 32), (768, 64, 128), (2048, 32, 128), (512, 48, 64)])
def test_grouped_gemm_kat_exact(dev, d, n, g):
    """Grouped GEMM without the SwiGLU epilogue on integer-exact inputs: each grouped row equals its token's exact
    product with its expert's matrix; padding rows are zero. G = 128 is qwen3moe's expert group
    (qwen3moe/kernels/moek.mojo:26, qwen3moe/export.py:39); K = 768 is its down projection (6 groups a row)."""
    import torch
    rng = np.random.default_rng(8 + d + g)
    t, e, k, tm = 60, 6, 2, 32
    vals, ws, _ = kat_int4(rng, e * n, d, g)
    x = rng.integers(-3, 4, size=(t, d)).astype(np.float16)
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    ref = orc.p_group(ids, e, tm)
    from aq import _lib
    max_rows = _lib.lib().aq_moe_group_max_rows(t, k, e, tm)
    max_tiles = _lib.lib().aq_moe_group_max_tiles(t, k, e, tm)
    src = np.full(max_rows, -1, np.int32)
    src[:ref["rows_total"]] = ref["src"]
    tiles = np.zeros((max_tiles, 2), np.int32)
    tiles[:len(ref["tiles"])] = ref["tiles"]
    out = torch.zeros((max_rows, n), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_gemm_q4(to_dev(x, dev), _i32(src, dev), to_dev(orc.q4w_pack(vals), dev), to_dev(ws, dev), e, g,
                             _i32(tiles.ravel(), dev), _i32([len(ref["tiles"])], dev), tm, False, out)
    got = to_np(out)
    for row in range(ref["rows_total"]):
        tok = ref["src"][row]
        if tok < 0:
            assert np.all(got[row] == 0)
            continue
        ex = int(np.searchsorted(ref["offs"], row, side="right") - 1)
        exact = exact_int4_product(vals[ex * n:(ex + 1) * n], ws[ex * n:(ex + 1) * n], x[tok:tok + 1].astype(np.float32),
                                   g)
        np.testing.assert_array_equal(got[row], exact[0].astype(np.float32))


@pytest.mark.parametrize("t,tm", [(404, 32), (404, 48), (404, 64), (64, 16)])
def test_c3_moe_block(dev, t, tm):
    """C3: Qwen3-30B-A3B-shaped block (128 experts, D 2048, F 768, G 32, top 8), fp32 x, vs the oracle."""
    import torch
    from aq import moe, synth
    d = synth.c3(tokens=t)
    to = lambda a: to_dev(a, dev)  # noqa: E731
    blk = moe.MoeBlock(to(d["gu_q"]), to(d["gu_s"]), to(d["dn_q"]), to(d["dn_s"]), 128, 2048, 768, 32, 8,
                       max_tokens=512, tm=tm)
    out = torch.empty((t, 2048), dtype=torch.float32, device=dev)
    blk.forward(to(d["x"]), to(d["logits"]), out)
    ref, rids, _ = orc.moe_layer(d["x"], d["logits"], d["gu_q"], d["gu_s"], d["dn_q"], d["dn_s"], 32, 768)
    np.testing.assert_array_equal(to_np(blk.ids[:t]), rids)
    assert rel_inf(to_np(out), ref) < 1e-2
    # the residual form adds onto out
    res = np.random.default_rng(1).standard_normal((t, 2048)).astype(np.float32)
    out2 = to(res)
    blk.forward(to(d["x"]), to(d["logits"]), out2, add=True)
    assert rel_inf(to_np(out2), ref + res) < 1e-2


def test_c3_moe_block_group128(dev):
    """The C3 block at qwen3moe's own expert group, G = 128 (qwen3moe/kernels/moek.mojo:26, qwen3moe/export.py:39):
    grouped gate|up over K = 2048 (16 groups a row) and grouped down over K = 768 (6 groups a row)."""
    import torch
    from aq import moe, synth
    t = 404
    d = synth.c3(tokens=t, group=128)
    to = lambda a: to_dev(a, dev)  # noqa: E731
    blk = moe.MoeBlock(to(d["gu_q"]), to(d["gu_s"]), to(d["dn_q"]), to(d["dn_s"]), 128, 2048, 768, 128, 8,
                       max_tokens=512, tm=48)
    out = torch.empty((t, 2048), dtype=torch.float32, device=dev)
    blk.forward(to(d["x"]), to(d["logits"]), out)
    ref, rids, _ = orc.moe_layer(d["x"], d["logits"], d["gu_q"], d["gu_s"], d["dn_q"], d["dn_s"], 128, 768)
    np.testing.assert_array_equal(to_np(blk.ids[:t]), rids)
    assert rel_inf(to_np(out), ref) < 1e-2


@pytest.mark.parametrize("g", [32, 128])
def test_c3_decode_one_token(dev, g):
    """One token through the decode experts (route, gate|up over the 8 chosen experts, weighted down), at C0's group
    and at qwen3moe's G = 128."""
    import torch
    from aq import moe, synth
    d = synth.c3(tokens=1, group=g)
    to = lambda a: to_dev(a, dev)  # noqa: E731
    blk = moe.MoeBlock(to(d["gu_q"]), to(d["gu_s"]), to(d["dn_q"]), to(d["dn_s"]), 128, 2048, 768, g, 8,
                       max_tokens=1)
    out = torch.empty(2048, dtype=torch.float32, device=dev)
    blk.decode(to(d["x"][0]), to(d["logits"][0]), out)
    ref, _, _ = orc.moe_layer(d["x"], d["logits"], d["gu_q"], d["gu_s"], d["dn_q"], d["dn_s"], g, 768)
    assert rel_inf(to_np(out), ref[0]) < 1e-3


@pytest.mark.parametrize("hidden,ffn,g", [(8192, 256, 32), (8192, 256, 128), (4096, 512, 64)])
def test_moe_decode_deep_pipeline(dev, hidden, ffn, g):
    """Decode experts at widths where the gate|up launch streams several chunks per lane through its register sets
    (K = 8192: four chunks a row per lane, so four sets in flight; K = 4096: two), vs the oracle."""
    import torch
    from aq import moe, synth
    d = synth.c3(seed=9, tokens=1, experts=16, hidden=hidden, ffn=ffn, group=g)
    to = lambda a: to_dev(a, dev)  # noqa: E731
    blk = moe.MoeBlock(to(d["gu_q"]), to(d["gu_s"]), to(d["dn_q"]), to(d["dn_s"]), 16, hidden, ffn, g, 8,
                       max_tokens=1)
    out = torch.empty(hidden, dtype=torch.float32, device=dev)
    blk.decode(to(d["x"][0]), to(d["logits"][0]), out)
    ref, _, _ = orc.moe_layer(d["x"], d["logits"], d["gu_q"], d["gu_s"], d["dn_q"], d["dn_s"], g, ffn)
    assert rel_inf(to_np(out), ref[0]) < 1e-3


@pytest.mark.parametrize("t,e,k,tm", [(50, 8, 4, 16), (404, 128, 8, 48), (3000, 64, 2, 32)])
def test_group_repeated_ids(dev, t, e, k, tm):
    """A token that names one expert more than once: every entry is counted and one expert's entries keep ascending
    i, as p_group's ordered scan gives them (lfm2moe/kernels/mk.mojo:123-161); the lists follow p_expert_lists."""
    import torch
    from aq import _lib
    rng = np.random.default_rng(t + e + k)
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    rep = rng.choice(t, size=max(1, t // 10), replace=False)
    ids[rep, k - 1] = ids[rep, 0]            # the first and last choice of these tokens coincide
    ids[0, :] = ids[0, 0]                    # one token names a single expert k times
    ref = orc.p_group(ids, e, tm)
    max_rows = _lib.lib().aq_moe_group_max_rows(t, k, e, tm)
    max_tiles = _lib.lib().aq_moe_group_max_tiles(t, k, e, tm)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, offs, slot = torch.empty(e, **i32), torch.empty(e + 1, **i32), torch.empty(t * k, **i32)
    src, tiles, nt = torch.empty(max_rows, **i32), torch.empty(2 * max_tiles, **i32), torch.empty(1, **i32)
    torch.ops.aq.moe_group(_i32(ids, dev), e, tm, counts, offs, slot, src, tiles, nt)
    np.testing.assert_array_equal(to_np(counts), ref["cnt"])
    assert to_np(counts).sum() == t * k
    np.testing.assert_array_equal(to_np(offs)[:e], ref["offs"])
    np.testing.assert_array_equal(to_np(slot), ref["slot"])
    np.testing.assert_array_equal(to_np(src)[:ref["rows_total"]], ref["src"])
    n_t = int(to_np(nt)[0])
    np.testing.assert_array_equal(to_np(tiles)[:2 * n_t].reshape(-1, 2), ref["tiles"])
    lists_ref, counts_ref = orc.expert_lists(ids, e, t * k)
    lists, counts2 = torch.full((e, t * k), -1, **i32), torch.empty(e, **i32)
    scratch = torch.empty(e + 1 + 4 * t * k + 1, **i32)
    torch.ops.aq.moe_expert_lists(_i32(ids, dev), e, lists, counts2, 8, torch.empty(0, **i32),
                                  torch.empty(0, **i32), scratch)
    np.testing.assert_array_equal(to_np(counts2), counts_ref)
    got = to_np(lists)
    for ex in range(e):
        np.testing.assert_array_equal(got[ex, :counts_ref[ex]], lists_ref[ex, :counts_ref[ex]])


def test_moe_sum_identity_slots(dev):
    """p_moe_sum: part rows indexed by entry t*topk + k, added onto x."""
    import torch
    rng = np.random.default_rng(6)
    t, k, dd = 9, 8, 64
    part = rng.standard_normal((t * k, dd)).astype(np.float32)
    w = rng.random((t, k)).astype(np.float32)
    x0 = rng.standard_normal((t, dd)).astype(np.float32)
    y = to_dev(x0, dev)
    torch.ops.aq.moe_combine(to_dev(part, dev), torch.empty(0, dtype=torch.int32, device=dev), to_dev(w, dev), y, True)
    ref = x0 + orc.p_combine(part, np.arange(t * k), w)
    np.testing.assert_allclose(to_np(y), ref, rtol=1e-5, atol=1e-5)


def test_invalid_ids_are_inert(dev):
    """Ids outside [0, E) select nothing: no out-of-range weight rows are read and they add zero."""
    import torch
    rng = np.random.default_rng(7)
    e, d, f, g = 4, 256, 64, 32
    gu_q, gu_s, dn_q, dn_s, _, _ = _small_moe(rng, e, d, f, g)
    x = rng.standard_normal(d).astype(np.float32)
    ids = np.array([1, -3, 7, 2], np.int32)
    wts = np.array([0.5, 0.2, 0.2, 0.1], np.float32)
    a = torch.empty((4, f), dtype=torch.float32, device=dev)
    torch.ops.aq.moe_gate_up_q4(to_dev(gu_q, dev), to_dev(gu_s, dev), e, _i32(ids, dev), to_dev(x, dev), a, g)
    an = to_np(a)
    assert np.all(an[1] == 0) and np.all(an[2] == 0)
    y = torch.empty(d, dtype=torch.float32, device=dev)
    torch.ops.aq.moe_down_q4(to_dev(dn_q, dev), to_dev(dn_s, dev), e, _i32(ids, dev), to_dev(wts, dev), a, y, g, False)
    ref = np.zeros(d)
    for j in (0, 3):
        ex = ids[j]
        h = orc.gemv_q4(gu_q[ex * 2 * f:(ex + 1) * 2 * f], gu_s[ex * 2 * f:(ex + 1) * 2 * f], x, g)
        act = orc.silu(h[:f]) * h[f:]
        assert rel_inf(an[j], act) < 1e-4
        ref += wts[j] * orc.gemv_q4(dn_q[ex * d:(ex + 1) * d], dn_s[ex * d:(ex + 1) * d], an[j], g)
    assert rel_inf(to_np(y), ref) < 1e-4


def test_router_gemv_f32(dev):
    import torch
    rng = np.random.default_rng(2)
    w = rng.standard_normal((128, 2048)).astype(np.float32)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    y = torch.empty((3, 128), dtype=torch.float32, device=dev)
    torch.ops.aq.gemv_f32(to_dev(w, dev), to_dev(x, dev), y)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(to_np(y), ref, rtol=1e-4, atol=1e-4)
