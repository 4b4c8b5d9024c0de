"""Pins the CPU oracle before it is trusted to check the GPU (CPU only, no GPU).

Every oracle function is checked against something that does not share its code: a
library routine (torch sort / SDPA / bf16 conversion / normalize), exact fp64 or rational
arithmetic, or a brute-force statement of the reference's rule on tiny inputs. Each check
is chosen so that a plausible slip (a dropped term, a flipped tie rule, an off-by-one in
the window, a transposed operand) fails it. The reference ships no golden vectors for this
path (its tests regenerate seeded tensors through the absent upstream package), so the
fixtures under tests/golden/ are written from this oracle and pinned here by these checks.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

RNG = np.random.default_rng(20261201)


# ----------------------------------------------------------------------------- keys


def brute_order(scores, length):
    """Best-first columns by the packed-key contract: score descending, a tie to the lower
    column (reference select_fused.py:71-77 key layout), columns < length only."""
    cols = [c for c in range(length)]
    return sorted(cols, key=lambda c: (-float(scores[c]), c))


def test_ordered_bits_is_the_float_order():
    vals = np.array([-np.inf, -3e38, -1.0, -1e-30, -1e-45, -0.0, 0.0, 1e-45, 1e-30, 1.0, 3e38, np.inf],
                    dtype=np.float32)
    bits = oracle.ordered_bits(vals)
    assert (np.diff(bits.astype(np.int64)) > 0).all()  # strictly increasing, -0.0 just below +0.0
    x = RNG.standard_normal(10_000).astype(np.float32) * 10.0 ** RNG.integers(-30, 30, 10_000)
    order_bits = np.argsort(oracle.ordered_bits(x), kind="stable")
    assert np.array_equal(np.sort(x, kind="stable"), x[order_bits])


@pytest.mark.parametrize("rows,cols,top_p", [(3, 17, 5), (4, 64, 64), (2, 40, 100), (5, 128, 33)])
def test_select_topk_scores_equals_brute_force(rows, cols, top_p):
    scores = RNG.integers(-4, 5, (rows, cols)).astype(np.float32)  # many ties
    lengths = RNG.integers(0, cols + 1, rows)
    got = oracle.select_topk_scores(scores, lengths, top_p)
    keep = min(top_p, cols)
    assert got.shape == (rows, oracle.next_pow2(keep))
    ids = oracle.unpack_ids(got)
    for r in range(rows):
        want = brute_order(scores[r], int(lengths[r]))[:keep]
        assert ids[r, : len(want)].tolist() == want
        assert (got[r, len(want):] == oracle.EMPTY).all()


def test_select_topk_scores_sampled_path_width():
    """Rows wider than 4 * top_p take the reference's fallback (select_fused.py:97-117):
    torch.topk(k=min(top_p, N)) over the length-masked packed keys, so the width is
    min(top_p, N), not its next power of two."""
    scores = RNG.standard_normal((8, 512)).astype(np.float32)
    lengths = np.array([512, 300, 100, 99, 7, 1, 0, 512])
    got = oracle.select_topk_scores(scores, lengths, 100)
    assert got.shape == (8, 100)
    keys = torch.from_numpy(oracle.pack_keys(scores, lengths))
    want = torch.topk(keys, k=100, dim=1, sorted=True).values.numpy()
    assert np.array_equal(got, want)


def test_all_tied_scores_pick_ids_in_ascending_order():
    got = oracle.unpack_ids(oracle.select_topk_scores(np.zeros((2, 300), np.float32), np.array([300, 7]), 64))
    assert got[0].tolist() == list(range(64))
    assert got[1, :7].tolist() == list(range(7)) and (got[1, 7:] == -1).all()


def test_best_first_keys_is_sort_slice_and_masks_unlisted():
    keys = oracle.pack_keys(RNG.standard_normal((4, 50)).astype(np.float32), np.array([50, 20, 0, 50]))
    want = torch.sort(torch.from_numpy(keys), dim=1, descending=True).values[:, :16].numpy()
    assert np.array_equal(oracle.best_first_keys(keys, 16), want)
    poisoned = keys.copy()
    poisoned[:, 30:] = np.int64((1 << 63) - 1)  # unlisted slots hold garbage larger than any key
    got = oracle.best_first_keys(poisoned, 16, counts=np.array([30, 30, 30, 30]))
    masked = keys.copy()
    masked[:, 30:] = oracle.EMPTY
    want = torch.sort(torch.from_numpy(masked), dim=1, descending=True).values[:, :16].numpy()
    assert np.array_equal(got, want)


def test_unpack_round_trip():
    scores = RNG.standard_normal((3, 33)).astype(np.float32)
    keys = oracle.pack_keys(scores, np.array([33, 10, 0]))
    ids = oracle.unpack_ids(keys)
    assert np.array_equal(ids[0], np.arange(33))
    assert np.array_equal(ids[1, :10], np.arange(10)) and (ids[1, 10:] == -1).all()
    assert (ids[2] == -1).all()


# ----------------------------------------------------------------------------- expansion


def literal_expand(picks, members, position, window, sink, top_k):
    """The reference's walk (select_fused.py:172-214) as a literal loop: picks in rank order,
    slots in table order, keep sink <= id < window_start up to top_k; then the window, then
    the sinks that are not in it."""
    window_start = max(0, position + 1 - window)
    kept = []
    for b in picks:
        if b < 0 or b >= len(members):
            continue
        for m in members[b]:
            if m >= sink and m < window_start and len(kept) < top_k:
                kept.append(int(m))
    tail = list(range(window_start, position + 1)) + list(range(0, min(sink, window_start)))
    row = kept + tail
    return row + [-1] * (top_k + window + sink - len(row)), len(row)


@pytest.mark.parametrize("window,sink,top_k", [(8, 2, 20), (0, 0, 50), (16, 4, 3), (100, 4, 64)])
def test_expand_matches_literal_walk(window, sink, top_k):
    members = RNG.integers(-1, 120, (12, 6)).astype(np.int32)
    picks = RNG.integers(-1, 14, (5, 7)).astype(np.int32)  # includes -1 and out-of-range picks
    positions = np.array([0, 3, 40, 90, 119])
    lists, lengths = oracle.expand_in_order(picks, members, positions, window, sink, top_k)
    for r in range(5):
        want, n = literal_expand(picks[r].tolist(), members.tolist(), int(positions[r]), window, sink, top_k)
        assert lists[r].tolist() == want and int(lengths[r]) == n


def test_expand_invariants_causal_and_counts():
    members = RNG.integers(0, 1000, (64, 16)).astype(np.int32)
    picks = RNG.permutation(64)[None, :32].astype(np.int32)
    for pos in (0, 5, 511, 999):
        lst, n = oracle.expand_in_order(picks, members, np.array([pos]), 512, 4, 4096)
        sel = lst[0, : n[0]]
        assert (sel <= pos).all() and (lst[0, n[0]:] == -1).all()
        window_start = max(0, pos + 1 - 512)
        assert sorted(sel[sel >= window_start].tolist())[-(pos + 1 - window_start):] == list(range(window_start, pos + 1))


def test_visible_counts_rule():
    pos = np.array([-1, 0, 511, 512, 1023, 1024, 100000])
    assert oracle.visible_counts(pos, 64, 512, 8).tolist() == [-8, 0, 0, 8, 8, 16, 64]
    ends = np.array([10, 20, 20, 35, 64])
    assert oracle.visible_counts(np.array([8, 9, 19, 34, 63, 500]), 5, 1, 1, ends).tolist() == [0, 1, 3, 4, 5, 5]


# ----------------------------------------------------------------------------- numbers


def test_bf16_round_matches_torch():
    x = np.concatenate([RNG.standard_normal(5000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 65504.0, 3.4e38, 1e-40], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oracle.bf16_round(x).view(np.uint32), want.view(np.uint32))


def test_canonical_scores_exact_on_integers_and_close_to_fp64():
    q = RNG.integers(-8, 9, (3, 64)).astype(np.float32)
    c = RNG.integers(-8, 9, (10, 64)).astype(np.float32)
    assert np.array_equal(oracle.canonical_scores(q, c, "fp32"), (q.astype(np.int64) @ c.astype(np.int64).T))
    q = RNG.standard_normal((4, 128)).astype(np.float32)
    c = RNG.standard_normal((50, 128)).astype(np.float32)
    for mode in ("fp32", "bf16"):
        qq, cc = (q, c) if mode == "fp32" else (oracle.bf16_round(q), oracle.bf16_round(c))
        exact = qq.astype(np.float64) @ cc.astype(np.float64).T
        got = oracle.canonical_scores(q, c, mode).astype(np.float64)
        assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -23 + 1e-30)


def test_canonical_scores_follow_the_documented_order():
    """fp32 rounding happens once, after the fp64 tree: a rational computation of the same
    value rounds to the same float."""
    q = RNG.standard_normal((2, 32)).astype(np.float32)
    c = RNG.standard_normal((3, 32)).astype(np.float32)
    got = oracle.canonical_scores(q, c, "fp32")
    for i in range(2):
        for j in range(3):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(q[i], c[j]))
            assert abs(float(got[i, j]) - float(exact)) <= abs(float(exact)) * 2.0 ** -24 + 1e-38


def test_index_queries_is_group_mean():
    q = RNG.standard_normal((2, 128, 8, 16)).astype(np.float32)
    got = oracle.index_queries(q, 2, chunk=4)
    want = torch.from_numpy(q).double().view(2, 32, 4, 2, 4, 16).mean(dim=(2, 4)).numpy()
    assert got.shape == (2, 32, 2, 16)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    exact = np.full((1, 8, 4, 4), 0.5, np.float32)  # exactly representable sums and quotient
    assert np.array_equal(oracle.index_queries(exact, 2, 2), np.full((1, 4, 2, 4), 0.5, np.float32))


def test_bucket_centroids_mean_and_normalized():
    keys = RNG.standard_normal((40, 8)).astype(np.float32)
    members = np.array([[0, 1, 2, -1], [5, -1, 7, 9], [-1, -1, -1, -1]], np.int32)
    mean = oracle.bucket_centroids(keys, members, "mean")
    assert np.allclose(mean[0], keys[[0, 1, 2]].mean(0), atol=1e-6)
    assert np.allclose(mean[1], keys[[5, 7, 9]].mean(0), atol=1e-6)
    assert (mean[2] == 0).all()
    norm = oracle.bucket_centroids(keys, members, "normalized")
    want = F.normalize(torch.from_numpy(keys[[5, 7, 9]]).sum(0, keepdim=True).double(), dim=-1).numpy()[0]
    assert np.allclose(norm[1], want, atol=1e-6)


# ----------------------------------------------------------------------------- reading


def test_sparse_read_full_causal_equals_torch_sdpa():
    T, Hq, Hkv, D = 24, 4, 2, 16
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, T, h, D, generator=g) for h in (Hq, Hkv, Hkv))
    ids = np.tile(np.arange(T, dtype=np.int32), (T, 1))
    ids = np.where(ids <= np.arange(T)[:, None], ids, -1)[None]
    lengths = (np.arange(T) + 1)[None]
    got = oracle.sparse_read(q.numpy(), k.numpy(), v.numpy(), ids, lengths)
    kk = k.repeat_interleave(2, dim=2).permute(0, 2, 1, 3).double()
    vv = v.repeat_interleave(2, dim=2).permute(0, 2, 1, 3).double()
    want = F.scaled_dot_product_attention(q.permute(0, 2, 1, 3).double(), kk, vv, is_causal=True)
    assert np.allclose(got, want.permute(0, 2, 1, 3).numpy(), atol=1e-6)


def test_sparse_read_edge_semantics():
    q = RNG.standard_normal((1, 2, 2, 8)).astype(np.float32)
    k = RNG.standard_normal((1, 10, 1, 8)).astype(np.float32)
    v = RNG.standard_normal((1, 10, 1, 8)).astype(np.float32)
    dup = np.array([[[4, 4, -1], [-1, -1, -1]]], np.int32)
    lengths = np.array([[3, 0]])
    out = oracle.sparse_read(q, k, v, dup, lengths)
    assert np.allclose(out[0, 0, 0], v[0, 4, 0]) and np.allclose(out[0, 0, 1], v[0, 4, 0])  # duplicate -> V row
    assert (out[0, 1] == 0).all()
    assert np.isnan(oracle.sparse_read(q, k, v, dup, lengths, empty="nan")[0, 1]).all()
    # duplicates count per occurrence: ids [1, 1, 2] weight row 1 twice
    ids = np.array([[[1, 1, 2], [1, 2, -1]]], np.int32)
    out = oracle.sparse_read(q, k, v, ids, np.array([[3, 2]]))
    s = (k[0, [1, 1, 2], 0] @ q[0, 0, 0]) / np.sqrt(8.0)
    p = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    assert np.allclose(out[0, 0, 0], p @ v[0, [1, 1, 2], 0], atol=1e-6)


def test_chunked_read_is_shared_list_plus_causal_block():
    q = RNG.standard_normal((1, 8, 2, 8)).astype(np.float32)
    k = RNG.standard_normal((1, 8, 1, 8)).astype(np.float32)
    v = RNG.standard_normal((1, 8, 1, 8)).astype(np.float32)
    chunk_ids = np.array([[[[-1, -1]], [[0, 2]]]], np.int32)  # [B, C=2, Hkv, W]
    chunk_len = np.array([[[0], [2]]])
    got = oracle.sparse_read_chunked(q, k, v, chunk_ids, chunk_len, chunk=4)
    row = 6  # chunk 1: list {0, 2} + its causal block {4, 5, 6}
    ids = np.array([[[[0, 2, 4, 5, 6]]]], np.int32)
    want = oracle.sparse_read(q[:, [row]], k, v, ids, np.array([[[5]]]))
    assert np.allclose(got[:, row], want[:, 0])


def _paged_case():
    """Logical lists of a small flat select, a row-shuffled pool and its slot table."""
    T, Hkv, D = 96, 2, 16
    k = RNG.standard_normal((1, T, Hkv, D)).astype(np.float32)
    v = RNG.standard_normal((1, T, Hkv, D)).astype(np.float32)
    q = RNG.standard_normal((1, 2, 4, D)).astype(np.float32)
    cents = RNG.standard_normal((12, D)).astype(np.float32)
    members = np.arange(96, dtype=np.int32).reshape(12, 8)
    lists, lengths = oracle.flat_select(RNG.standard_normal((2, D)).astype(np.float32), np.array([95, 60]), cents,
                                        members, cluster_block_size=8, block_buckets=1, top_p=4, top_k=16,
                                        window=8, sink=2, mode="fp32")
    perm = RNG.permutation(T).astype(np.int32)  # logical t lives in pool row perm[t] (rows >= T unused)
    pool_k = np.zeros((1, T + 20, Hkv, D), np.float32)
    pool_v = np.zeros_like(pool_k)
    pool_k[0, perm], pool_v[0, perm] = k[0], v[0]
    return q, k, v, lists, lengths, perm, pool_k, pool_v


def test_map_slots_identity_inverse_and_bounds():
    q, k, v, lists, lengths, perm, pool_k, pool_v = _paged_case()
    ident = np.arange(96, dtype=np.int32)[None]
    assert np.array_equal(oracle.map_slots(lists, lengths, ident, np.zeros(2)), lists)
    mapped = oracle.map_slots(lists, lengths, perm[None], np.zeros(2))
    inv = np.full(perm.max() + 1, -1)
    inv[perm] = np.arange(perm.size)
    for r in range(2):
        n = int(lengths[r])
        assert np.array_equal(inv[mapped[r, :n]], lists[r, :n])  # the permutation's inverse recovers them
        assert (mapped[r, n:] == -1).all()  # padding stays -1
    # two table rows: query row r reads its own row
    two = np.stack([perm, perm[::-1]])
    m2 = oracle.map_slots(lists, lengths, two, np.array([1, 0]))
    assert np.array_equal(m2[1, : lengths[1]], perm[lists[1, : lengths[1]]])
    assert np.array_equal(m2[0, : lengths[0]], perm[::-1][lists[0, : lengths[0]]])
    # ids at or past the width, and a row outside the table, map to -1
    short = perm[None, :50]
    ms = oracle.map_slots(lists, lengths, short, np.zeros(2))
    n0 = int(lengths[0])
    assert np.array_equal(ms[0, :n0], np.where(lists[0, :n0] < 50, perm[np.minimum(lists[0, :n0], 49)], -1))
    assert (oracle.map_slots(lists, lengths, perm[None], np.array([3, -1]))[:, :n0] == -1).all()


def test_read_over_a_shuffled_pool_equals_the_unpaged_read():
    q, k, v, lists, lengths, perm, pool_k, pool_v = _paged_case()
    mapped = oracle.map_slots(lists, lengths, perm[None], np.zeros(2))
    want = oracle.sparse_read(q, k, v, lists[None], lengths[None])
    got = oracle.sparse_read(q, pool_k, pool_v, mapped[None], lengths[None])
    assert np.array_equal(got, want)
    # the transposed map (the inverse permutation) reads other rows: its read must differ
    wrong = oracle.map_slots(lists, lengths, np.argsort(perm).astype(np.int32)[None], np.zeros(2))
    assert not np.allclose(oracle.sparse_read(q, pool_k, pool_v, wrong[None], lengths[None]), want, atol=1e-3)


# ----------------------------------------------------------------------------- selection end to end


def test_flat_select_equals_brute_force():
    q = RNG.standard_normal((3, 32)).astype(np.float32)
    cents = RNG.standard_normal((20, 32)).astype(np.float32)
    members = RNG.permutation(400).astype(np.int32).reshape(20, 20)
    positions = np.array([399, 250, 100])
    ends = np.arange(20, 401, 20)
    lists, lengths = oracle.flat_select(q, positions, cents, members, cluster_block_size=1, block_buckets=1,
                                        top_p=5, top_k=60, window=16, sink=2, mode="fp32", ends=ends)
    exact = q.astype(np.float64) @ cents.astype(np.float64).T
    for r in range(3):
        visible = int(np.sum(ends <= positions[r] + 1))
        order = sorted(range(visible), key=lambda c: (-exact[r, c], c))[:5]
        want, n = literal_expand(order, members.tolist(), int(positions[r]), 16, 2, 60)
        assert lists[r].tolist() == want and int(lengths[r]) == n


def _growth_replay_literal(visible, page_buckets, node_block, size):
    """The reference's growth replay (_tree.py:100-142) for a one-level tree, stepped
    page end by page end exactly as written there, up to the page whose end is the
    row's visible count; returns (covered, made[0])."""
    covered, made = 0, 0
    for end in range(page_buckets, visible + 1, page_buckets):
        blocks = (end - covered) // node_block
        if blocks < max(1, page_buckets // node_block):
            continue
        covered += blocks * node_block
        made += blocks * node_block // size
    return covered, made


@pytest.mark.parametrize("page_buckets,node_block,size", [(8, 64, 4), (64, 64, 4), (128, 64, 16), (16, 16, 16)])
def test_tree_growth_is_the_reference_replay(page_buckets, node_block, size):
    n_nodes = 10_000
    for pages in range(0, 70):
        visible = pages * page_buckets
        assert oracle.tree_growth(visible, node_block, n_nodes, size) == \
            _growth_replay_literal(visible, page_buckets, node_block, size), (pages,)
    # the table's nodes cap the growth; negative counts see nothing
    assert oracle.tree_growth(640, 64, 3, 16) == (48, 3)
    assert oracle.tree_growth(-5, 64, 3, 16) == (0, 0)


def _tree_brute(q, ncent, children, bcent, visible, node_block, beam, top_p):
    """The one-level beam by plain sorting: made nodes of whole node_block blocks, the best
    `beam` of them (ties -> lower node), their visible children plus the fresh buckets,
    each once, the best top_p (ties -> lower bucket)."""
    size = children.shape[1]
    covered = min(visible // node_block * node_block, ncent.shape[0] * size)
    made = covered // size
    ns = ncent.astype(np.float64) @ q.astype(np.float64)
    kept = sorted(range(made), key=lambda j: (-ns[j], j))[:beam]
    cand = {int(c) for j in kept for c in children[j] if 0 <= c < visible}
    cand |= set(range(covered, visible))
    bs = bcent.astype(np.float64) @ q.astype(np.float64)
    return sorted(cand, key=lambda c: (-bs[c], c))[:top_p]


def test_tree_select_row_equals_brute_force():
    D, n_nodes, size = 16, 6, 4
    q = RNG.standard_normal(D).astype(np.float32)
    bcent = RNG.standard_normal((n_nodes * size + 5, D)).astype(np.float32)
    children = np.arange(n_nodes * size, dtype=np.int32).reshape(n_nodes, size)
    ncent = bcent[: n_nodes * size].reshape(n_nodes, size, D).mean(1)
    members = np.arange(bcent.shape[0] * 3, dtype=np.int32).reshape(bcent.shape[0], 3)
    # every visible count, incl. partial node blocks and buckets past the nodes' reach
    for visible in range(0, bcent.shape[0] + 1):
        for node_block in (4, 8):
            lst, n, picks = oracle.tree_select_row(q, ncent, children, bcent, members, position=10_000,
                                                   visible=visible, node_block=node_block, beam_width=2,
                                                   top_p=5, top_k=100, window=0, sink=0, mode="fp32")
            want = _tree_brute(q, ncent, children, bcent, visible, node_block, 2, 5)
            assert picks[: len(want)].tolist() == want and (picks[len(want):] == -1).all(), (visible, node_block)
            assert lst[:n].tolist() == [int(m) for b in want for m in members[b]]


def _beam_growth_literal(visible, page_buckets, node_size, node_block, top_level):
    """_tree.py:100-142 ``_growth_replay`` for one page, stepped page end by page end as
    written there (top_level levels), up to the page whose end is the row's visible count;
    returns (covered, made, closed)."""
    covered, made, closed = 0, [0] * top_level, [0] * top_level
    for end in range(page_buckets, visible + 1, page_buckets):
        blocks = (end - covered) // node_block
        if blocks < max(1, page_buckets // node_block):
            continue
        covered += blocks * node_block
        made[0] += blocks * node_block // node_size
        for level in range(1, top_level):
            taken = (made[level - 1] - closed[level - 1]) // node_block * node_block
            if not taken:
                break
            closed[level - 1] += taken
            made[level] += taken // node_size
    return covered, made, closed


@pytest.mark.parametrize("page_buckets,node_size,node_block,top_level",
                         [(64, 4, 64, 3), (16, 4, 64, 3), (128, 4, 64, 3), (64, 2, 16, 4), (8, 4, 16, 3)])
def test_beam_growth_is_the_reference_replay(page_buckets, node_size, node_block, top_level):
    for pages in range(0, 200):
        visible = pages * page_buckets
        assert oracle.beam_growth(visible, top_level, node_size, node_block, top_level) == \
            _beam_growth_literal(visible, page_buckets, node_size, node_block, top_level), pages


def _tiny_tree(rng, rows, size, block, levels_wanted, D=16):
    """A tree of contiguous node groups over `rows` bucket centroids: level l+1 groups whole
    blocks of `block` level-l rows into nodes of `size` consecutive rows."""
    bcent = rng.standard_normal((rows, D)).astype(np.float32)
    levels, below = [], bcent
    while len(levels) < levels_wanted:
        count = below.shape[0] // block * block
        if not count:
            break
        children = np.arange(count, dtype=np.int32).reshape(-1, size)
        cent = below[:count].reshape(-1, size, D).mean(1).astype(np.float32)
        levels.append((cent, children))
        below = cent
    return bcent, levels


def _beam_brute(q, bcent, levels, visible, size, block, top_level, beam, top_p):
    """The beam by plain sorting: growth by the literal replay at page size `block`, every
    level's candidates as a set, ranked by (-float64 score, id)."""
    covered, made, closed = _beam_growth_literal(visible, block, size, block, top_level)
    made = [min(m, lv[0].shape[0]) for m, lv in zip(made, levels)] + [0] * (top_level - len(levels))
    start = max([l + 1 for l in range(len(levels)) if made[l]], default=0)
    carried = set()
    for lv in range(start, 0, -1):
        first = 0 if lv == start else closed[lv - 1]
        cand = carried | set(range(first, made[lv - 1]))
        cent, children = levels[lv - 1]
        sc = cent.astype(np.float64) @ q.astype(np.float64)
        kept = sorted(cand, key=lambda j: (-sc[j], j))[:beam]
        carried = {int(c) for j in kept for c in children[j]}
    cand = {c for c in carried if c < visible} | set(range(covered, visible))
    sc = bcent.astype(np.float64) @ q.astype(np.float64)
    return sorted(cand, key=lambda j: (-sc[j], j))[:top_p]


def test_beam_select_row_equals_brute_force():
    rng = np.random.default_rng(17)
    size, block, top_level = 2, 8, 3
    bcent, levels = _tiny_tree(rng, 160, size, block, 3)
    assert len(levels) == 3
    members = np.arange(160 * 3, dtype=np.int32).reshape(160, 3)
    for trial in range(40):
        q = rng.standard_normal(16).astype(np.float32)
        visible = int(rng.integers(0, 161))
        for beam, top_p in ((2, 5), (3, 12), (8, 40)):
            lst, n, picks = oracle.beam_select_row(q, levels, bcent, members, position=10_000, visible=visible,
                                                   node_size=size, node_block=block, top_level=top_level,
                                                   beam_width=beam, top_p=top_p, top_k=1000, window=0, sink=0,
                                                   mode="fp32")
            want = _beam_brute(q, bcent, levels, visible, size, block, top_level, beam, top_p)
            assert picks[: len(want)].tolist() == want and (picks[len(want):] == -1).all(), (trial, visible, beam)
            assert lst[:n].tolist() == [int(m) for b in want for m in members[b]]


def test_beam_with_one_level_is_the_tree_select():
    """A one-level tree through the beam equals tree_select_row's two-level walk."""
    rng = np.random.default_rng(18)
    bcent, levels = _tiny_tree(rng, 96, 4, 16, 1)
    members = np.arange(96 * 2, dtype=np.int32).reshape(96, 2)
    for visible in range(0, 97, 5):
        q = rng.standard_normal(16).astype(np.float32)
        a = oracle.beam_select_row(q, levels, bcent, members, 500, visible, 4, 16, 1, 3, 10, 100, 0, 0)
        b = oracle.tree_select_row(q, levels[0][0], levels[0][1], bcent, members, 500, visible, 16, 3, 10, 100, 0, 0)
        assert np.array_equal(a[0], b[0]) and a[1] == b[1] and np.array_equal(a[2], b[2])


@pytest.mark.parametrize("rows,size,block,top_level,want", [
    (4096, 4, 64, 3, [1024, 256, 64]),   # the reference defaults at 32k keys (8 keys a bucket)
    (1000, 4, 64, 3, [240, 48]),          # 960 of 1000 rows in whole blocks; 48 nodes close no block
    (4096, 4, 64, 2, [1024, 256]),        # top_level stops the loop
    (63, 4, 64, 3, []),                   # no full block, no level
    (1024, 2, 8, 4, [512, 256, 128, 64]),
])
def test_build_hierarchy_levels_sums_and_norms(rows, size, block, top_level, want):
    """Level counts follow the reference loop's stop rule (pipeline.py:166-170: stop when
    the level below holds no full block or top_level levels exist), worked by hand; every
    level's sums add up (fp64) to the covered buckets' sums; centroids have unit norm and
    point along their sums."""
    rng = np.random.default_rng(rows + size)
    sums = rng.standard_normal((rows, 16)).astype(np.float32)
    levels = oracle.build_hierarchy(sums, size, block, top_level)
    assert [lv[0].shape[0] for lv in levels] == want
    reach = sums.shape[0]
    for lvl, (cent, children, node_sums) in enumerate(levels):
        assert children.shape == (want[lvl], size) and (children.reshape(-1) == np.arange(want[lvl] * size)).all()
        covered = want[lvl] * size
        for _ in range(lvl):
            covered *= size
        total = sums[:covered].astype(np.float64).sum(0)
        np.testing.assert_allclose(node_sums.astype(np.float64).sum(0), total, rtol=1e-4, atol=1e-3)
        np.testing.assert_allclose(np.linalg.norm(cent.astype(np.float64), axis=1), 1.0, rtol=1e-6)
        cos = (cent.astype(np.float64) * node_sums).sum(1) / np.linalg.norm(node_sums.astype(np.float64), axis=1)
        np.testing.assert_allclose(cos, 1.0, rtol=1e-6)
        assert covered <= reach


# --------------------------------------------------------------------------- segment build


def test_ward_pair_cost_exact_rationals_and_fsum():
    """The canonical-order fp64 cost agrees with the exact rational value on dyadic sums
    (every operation exact), and with an fsum of exact squares to 1e-14 on random sums."""
    rng = np.random.default_rng(3)
    sa = rng.integers(-64, 64, 128).astype(np.float64)
    sb = rng.integers(-64, 64, 128).astype(np.float64)
    na, nb = 4, 8  # power-of-two sizes: the means are exact
    got = oracle.ward_pair_cost(sa, sb, na, nb, 64)
    want = Fraction(na * nb, na + nb) * sum((Fraction(int(a), na) - Fraction(int(b), nb)) ** 2 for a, b in zip(sa, sb))
    assert got == float(want)
    import math
    sa, sb = rng.standard_normal(96) * 10, rng.standard_normal(96) * 10
    got = oracle.ward_pair_cost(sa, sb, 17, 23, 64)
    want = 17 * 23 / 40 * math.fsum((a / 17 - b / 23) ** 2 for a, b in zip(sa, sb))
    assert abs(got - want) <= 1e-14 * want
    assert oracle.ward_pair_cost(sa, sb, 40, 30, 64) == float("inf")
    assert oracle.ward_pair_cost(sa, sa, 5, 5, 64) == 0.0


def _ward_brute(keys, pool, target, max_size):
    """Greedy adjacent merge with no links: every step recomputes every adjacent cost from
    the current segment list and merges the first minimum."""
    sums, sizes = oracle.ward_pool_sums(keys, pool)
    segs = [(i * pool, int(sizes[i]), sums[i].copy()) for i in range(len(sizes))]
    while len(segs) > target:
        costs = [oracle.ward_pair_cost(segs[k][2], segs[k + 1][2], segs[k][1], segs[k + 1][1], max_size)
                 for k in range(len(segs) - 1)]
        k = int(np.argmin(costs))
        assert costs[k] < np.inf
        a, b = segs[k], segs[k + 1]
        segs[k:k + 2] = [(a[0], a[1] + b[1], a[2] + b[2])]
    return np.array([s[0] for s in segs] + [keys.shape[0]])


@pytest.mark.parametrize("T,D,pool,target,max_size", [(200, 8, 8, 6, 64), (333, 16, 4, 20, 48), (512, 64, 16, 5, 512)])
def test_ward_segments_equal_brute_force(T, D, pool, target, max_size):
    rng = np.random.default_rng(T + D)
    centers = rng.standard_normal((6, D)).astype(np.float32)
    labels = np.repeat(rng.integers(0, 6, T // 10 + 1), 10)[:T]
    keys = centers[labels] + 0.3 * rng.standard_normal((T, D)).astype(np.float32)
    got = oracle.ward_segments_keys(keys, pool, target, max_size)
    assert np.array_equal(got, _ward_brute(keys, pool, target, max_size))
    sizes = np.diff(got)
    assert got[0] == 0 and got[-1] == T and len(got) == target + 1
    assert (sizes > 0).all() and (sizes <= max(max_size, pool)).all()
    assert (got[:-1] % pool == 0).all()


def test_ward_segments_two_clusters_split_at_the_boundary():
    """Two well-separated halves merge into exactly the two halves; ties (identical keys)
    merge leftmost first."""
    rng = np.random.default_rng(5)
    keys = np.concatenate([np.full((1024, 32), 3.0), np.full((1024, 32), -3.0)]).astype(np.float32)
    keys += 0.01 * rng.standard_normal(keys.shape).astype(np.float32)
    assert oracle.ward_segments_keys(keys, 16, 2, 4096).tolist() == [0, 1024, 2048]
    same = np.ones((64, 8), dtype=np.float32)
    # every cost ties at 0: the leftmost pair merges each step, so the first segment grows
    assert oracle.ward_segments_keys(same, 8, 3, 64).tolist() == [0, 48, 56, 64]
    with pytest.raises(ValueError, match="max_size"):
        oracle.ward_segments_keys(same, 8, 3, 8)
