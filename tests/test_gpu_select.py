"""Selection on the GPU vs the CPU oracle: bit-exact keys, lists and lengths.

Cases follow the reference's own selection tests (test_select_topk.py,
test_select_fusion.py, test_select_wide_adversarial.py): production widths, ragged
and zero-visibility rows, tied / signed-zero / denormal / NaN / inf scores, EMPTY
tails, k == width and k > width, window/sink boundaries, bucket-cap variants, both
scoring dtypes, every LSA_SELECT_IMPL, determinism.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import keys as keys_mod
from lsa_rocm_lab.port import pipeline, select_fused
from lsa_rocm_lab.port.pipeline import Buckets, PortConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
TIME = 20261108


def _np(t):
    return t.detach().cpu().numpy()


def _lengths(kind, rows, width, gen):
    if kind == "full":
        return torch.full((rows,), width, dtype=torch.int32)
    if kind == "ragged":
        return torch.randint(1, width + 1, (rows,), generator=gen, dtype=torch.int32)
    if kind == "zeros":
        return torch.zeros(rows, dtype=torch.int32)
    return torch.randint(0, width + 1, (rows,), generator=gen, dtype=torch.int32)


@pytest.mark.parametrize("rows,width,top_p,kind", [
    (64, 4096, 1024, "full"),
    (8, 4096, 1024, "ragged"),
    (64, 1024, 1024, "full"),
    (7, 300, 128, "ragged"),
    (5, 192, 1024, "full"),
    (3, 64, 64, "zeros"),
    (16, 2048, 512, "mix0"),
    (8, 512, 32, "full"),
])
def test_select_topk_scores_matches_oracle(rows, width, top_p, kind):
    print(f"case rows={rows} width={width} top_p={top_p} {kind}", flush=True)
    g = torch.Generator().manual_seed(TIME + width + rows)
    scores = torch.randn(rows, width, generator=g)
    lengths = _lengths(kind, rows, width, g)
    got = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), top_p)
    want = oracle.select_topk_scores(scores.numpy(), lengths.numpy(), top_p)
    assert np.array_equal(_np(got), want)


def test_tied_scores_break_to_lower_column():
    scores = torch.zeros(4, 512, device=DEV)
    lengths = torch.full((4,), 512, device=DEV, dtype=torch.int32)
    got = select_fused.select_topk_scores(scores, lengths, 128)
    ids = keys_mod.unpack_ids(got[:, :128])
    assert torch.equal(ids.cpu(), torch.arange(128, dtype=torch.int32).expand(4, 128))


@pytest.mark.parametrize("case", ["signed", "nonfinite"])
def test_special_scores_match_oracle(case):
    g = torch.Generator().manual_seed(TIME + 2)
    if case == "signed":
        scale = torch.tensor([-1e30, -1e-30, 0.0, 1e-30, 1e30, -0.0, 1.0, -1.0])[:, None]
        scores = torch.randn(8, 1024, generator=g) * scale
    else:
        scores = torch.randn(4, 512, generator=g)
        scores[0, ::7] = float("nan")
        scores[1] = float("nan")
        scores[2, :3] = -0.0
        scores[3, ::5] = float("inf")
    lengths = torch.full((scores.shape[0],), scores.shape[1], dtype=torch.int32)
    got = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), 256)
    want = oracle.select_topk_scores(scores.numpy(), lengths.numpy(), 256)
    assert np.array_equal(_np(got), want)


@pytest.mark.parametrize("rows,width,top_p", [(64, 4096, 1024), (64, 1024, 1024), (7, 300, 128), (6, 8192, 1024)])
def test_best_first_keys_equals_sort_slice(rows, width, top_p):
    g = torch.Generator().manual_seed(TIME + width)
    scores = torch.randn(rows, width, generator=g).to(DEV)
    keys, _ = keys_mod.listed(scores, torch.full((rows,), width, dtype=torch.int32, device=DEV))
    got = pipeline.best_first_keys(keys, top_p)
    want = torch.sort(keys, dim=1, descending=True).values[:, : min(top_p, width)]
    assert torch.equal(got, want)


def test_best_first_keys_masks_unlisted_poison():
    g = torch.Generator().manual_seed(TIME + 4)
    rows, width = 6, 2048
    scores = torch.randn(rows, width, generator=g)
    counts = torch.tensor([width, 1000, 64, 1, 0, width], dtype=torch.int32)
    keys = torch.from_numpy(oracle.pack_keys(scores.numpy(), counts.numpy()))
    unlisted = torch.arange(width)[None, :] >= counts[:, None].long()
    keys = torch.where(unlisted, torch.full_like(keys, (1 << 63) - 2), keys)
    got = pipeline.best_first_keys(keys.to(DEV), 1024, counts=counts.to(DEV))
    want = oracle.best_first_keys(keys.numpy(), 1024, counts.numpy())
    assert np.array_equal(_np(got), want)
    assert bool((got[4] == keys_mod.EMPTY).all())


def test_wide_rows_warn_and_stay_length_respecting():
    g = torch.Generator().manual_seed(TIME)
    scores = torch.randn(8, 8192, generator=g)
    lengths = torch.tensor([8192, 8192, 4096, 1000, 64, 8, 1, 0], dtype=torch.int32)
    with pytest.warns(UserWarning, match="sampled listing"):
        got = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), 1024)
    want = oracle.select_topk_scores(scores.numpy(), lengths.numpy(), 1024)
    assert np.array_equal(_np(got), want)


def test_sampled_listing_width_is_top_p():
    """Rows wider than 4 * top_p: the reference returns torch.topk(k=min(top_p, N))
    (select_fused.py:117), so a non-power-of-two top_p gives that width."""
    g = torch.Generator().manual_seed(TIME + 1)
    scores = torch.randn(8, 512, generator=g)
    lengths = torch.tensor([512, 300, 100, 99, 7, 1, 0, 512], dtype=torch.int32)
    with pytest.warns(UserWarning, match="sampled listing"):
        got = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), 100)
    assert tuple(got.shape) == (8, 100)
    assert np.array_equal(_np(got), oracle.select_topk_scores(scores.numpy(), lengths.numpy(), 100))


def _members(rows, cap, seed=TIME + 3, holes=0.15, top=997):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(rows * cap, generator=g) * top).long().reshape(rows, cap)
    empty = torch.rand(rows, cap, generator=g) < holes
    return torch.where(empty, torch.tensor(-1), m).to(torch.int32)


@pytest.mark.parametrize("rows,width,window,sink,top_k,kind", [
    (1, 1024, 512, 4, 4096, "last"),
    (32, 1024, 512, 4, 4096, "ragged"),
    (8, 256, 512, 4, 4096, "early"),
    (4, 256, 512, 4, 4096, "boundary"),
    (4, 128, 512, 4, 64, "last"),
    (4, 128, 8, 2, 4096, "last"),
    (2, 4096, 512, 4, 4096, "last"),
    (3, 512, 0, 0, 8192, "last"),
])
def test_expand_from_keys_matches_oracle(rows, width, window, sink, top_k, kind):
    print(f"case rows={rows} width={width} window={window} sink={sink} top_k={top_k} {kind}", flush=True)
    g = torch.Generator().manual_seed(TIME + width + top_k)
    scores = torch.randn(rows, width, generator=g)
    lengths = torch.full((rows,), width, dtype=torch.int32)
    ordered = oracle.select_topk_scores(scores.numpy(), lengths.numpy(), min(1024, width))
    members = _members(width, 16)
    if kind == "last":
        positions = torch.full((rows,), 4096, dtype=torch.int32)
    elif kind == "ragged":
        positions = torch.tensor([1, 511, 512, 513, 1023, 1024, 2047, 4095] * 4, dtype=torch.int32)[:rows]
    elif kind == "early":
        positions = torch.arange(rows, dtype=torch.int32)
    else:
        positions = torch.tensor([511, 512, 513, 1024], dtype=torch.int32)[:rows]
    got_l, got_n = select_fused.expand_in_order_from_keys(
        torch.from_numpy(ordered).to(DEV), members.to(DEV), positions.to(DEV), window, sink, top_k)
    want_l, want_n = oracle.expand_in_order(oracle.unpack_ids(ordered), members.numpy(), positions.numpy(),
                                            window, sink, top_k)
    assert np.array_equal(_np(got_l), want_l)
    assert np.array_equal(_np(got_n), want_n)
    # and the int32-pick expansion (the reference chain's walk) agrees
    picks = keys_mod.unpack_ids(torch.from_numpy(ordered).to(DEV))
    l2, n2 = select_fused.expand_in_order(picks, members.to(DEV), positions.to(DEV), window, sink, top_k)
    assert torch.equal(l2, got_l) and torch.equal(n2, got_n)


def test_expand_empty_picks_contribute_nothing():
    g = torch.Generator().manual_seed(TIME + 4)
    scores = torch.randn(2, 64, generator=g)
    lengths = torch.tensor([3, 0], dtype=torch.int32)
    keys = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), 64)
    members = _members(64, 16)
    positions = torch.tensor([500, 500], dtype=torch.int32)
    got_l, got_n = select_fused.expand_in_order_from_keys(keys, members.to(DEV), positions.to(DEV), 64, 4, 128)
    want_l, want_n = oracle.expand_in_order(oracle.unpack_ids(_np(keys)), members.numpy(), positions.numpy(),
                                            64, 4, 128)
    assert np.array_equal(_np(got_l), want_l) and np.array_equal(_np(got_n), want_n)


@pytest.mark.parametrize("cap", [8, 32, 64])
def test_expand_bucket_cap_variants(cap):
    g = torch.Generator().manual_seed(TIME + 7 + cap)
    rows, width = 8, 512
    scores = torch.randn(rows, width, generator=g)
    ordered = oracle.select_topk_scores(scores.numpy(), np.full(rows, width, np.int32), 512)
    members = _members(width, cap, seed=TIME + 6)
    positions = torch.tensor([4095, 511, 512, 513, 1024, 1, 0, 2047], dtype=torch.int32)
    got_l, got_n = select_fused.expand_in_order_from_keys(
        torch.from_numpy(ordered).to(DEV), members.to(DEV), positions.to(DEV), 512, 4, 4096)
    want_l, want_n = oracle.expand_in_order(oracle.unpack_ids(ordered), members.numpy(), positions.numpy(),
                                            512, 4, 4096)
    assert np.array_equal(_np(got_l), want_l) and np.array_equal(_np(got_n), want_n)


def test_non_pow2_bucket_cap_fails_loudly():
    ordered = torch.full((4, 64), keys_mod.EMPTY, device=DEV, dtype=torch.int64)
    members = _members(64, 24).to(DEV)
    positions = torch.full((4,), 64, device=DEV, dtype=torch.int32)
    with pytest.raises(ValueError, match="power-of-two"):
        select_fused.expand_in_order_from_keys(ordered, members, positions, 64, 4, 128)


# ---------------------------------------------------------------- composition through the switch


def _index_space(T, d, seed):
    """Reference-layout workspace: one shared table over a [T, d] index space."""
    g = torch.Generator().manual_seed(seed)
    idx_q = torch.randn(T, d, generator=g) * 0.2
    idx_k = torch.randn(T, d, generator=g) * 0.2
    return idx_q, idx_k


def _oracle_flat(idx_q, positions, buckets, config, score_dtype, top_k=None):
    top_k = config.top_k if top_k is None else top_k
    cent = (buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float()).cpu().numpy()
    ve = pipeline.visible_ends(buckets)
    ends = None if ve is None else ve.cpu().numpy()
    return oracle.flat_select(_np(idx_q.float()), _np(positions), cent, _np(buckets.members),
                              cluster_block_size=config.cluster_block_size,
                              block_buckets=config.block_bucket_count, top_p=config.top_p, top_k=top_k,
                              window=config.window_size, sink=config.sink_size, mode=score_dtype, ends=ends)


def _switched(impl, *args, **kw):
    os.environ["LSA_SELECT_IMPL"] = impl
    try:
        return pipeline.flat_select(*args, **kw)
    finally:
        os.environ.pop("LSA_SELECT_IMPL", None)


@pytest.mark.parametrize("context", [512, 1536, 2048, 8192])
@pytest.mark.parametrize("score_dtype", ["bf16", "fp32"])
def test_switched_flat_select_matches_oracle(context, score_dtype):
    print(f"case context={context} {score_dtype}", flush=True)
    config = PortConfig(cluster_block_size=512, bucket_size=8, bucket_cap=16, top_p=64, top_k=256,
                        window_size=128, sink_size=4)
    idx_q, idx_k = _index_space(context, 128, TIME + context)
    buckets = pipeline.position_buckets(idx_k.to(DEV), config)
    positions = torch.arange(context)[:: max(1, context // 64)]
    rows = idx_q[positions]
    want_l, want_n = _oracle_flat(rows, positions, buckets, config, score_dtype)
    for impl in ("reference", "fused", "fused_unpack"):
        got_l, got_n = _switched(impl, rows.to(DEV), positions.to(DEV), buckets, config, score_dtype=score_dtype)
        assert np.array_equal(_np(got_l), want_l), f"{impl} lists diverged"
        assert np.array_equal(_np(got_n), want_n), f"{impl} lengths diverged"


def test_switch_production_geometry_decode_and_ragged():
    """Reference PortConfig defaults (top_p 1024, top_k 4096, window 512, sink 4) at 32k."""
    config = PortConfig()
    context = 32768
    idx_q, idx_k = _index_space(context, 128, TIME)
    buckets = pipeline.position_buckets(idx_k.to(DEV), config)
    for positions in (torch.tensor([context - 1]), torch.tensor([0]),
                      torch.tensor([0, 1, 511, 512, 513, 1024, 1536, 2045, 2047, 30000, 32767])):
        rows = idx_q[positions]
        want_l, want_n = _oracle_flat(rows, positions, buckets, config, "bf16")
        for impl in ("reference", "fused", "fused_unpack"):
            got_l, got_n = _switched(impl, rows.to(DEV), positions.to(DEV), buckets, config)
            assert np.array_equal(_np(got_l), want_l), f"{impl} {positions.tolist()[:3]}"
            assert np.array_equal(_np(got_n), want_n)


def test_fused_deterministic_across_runs():
    config = PortConfig(cluster_block_size=512, bucket_size=8, bucket_cap=16, top_p=64, top_k=256,
                        window_size=128, sink_size=4)
    idx_q, idx_k = _index_space(2048, 128, TIME)
    buckets = pipeline.position_buckets(idx_k.to(DEV), config)
    positions = torch.arange(2048, device=DEV)[::8]
    rows = idx_q.to(DEV)[positions]
    first = _switched("fused", rows, positions, buckets, config)
    for _ in range(3):
        again = _switched("fused", rows, positions, buckets, config)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])


def test_visible_counts_and_scores_match_oracle():
    config = PortConfig(cluster_block_size=512, bucket_size=8, bucket_cap=16)
    idx_q, idx_k = _index_space(4096, 64, TIME + 9)
    buckets = pipeline.position_buckets(idx_k.to(DEV), config)
    positions = torch.tensor([-1, 0, 511, 512, 1023, 4095, 9000])
    got = pipeline.visible_counts(positions.to(DEV), buckets, config)
    want = oracle.visible_counts(positions.numpy(), buckets.rows, 512, 64)
    assert np.array_equal(_np(got), want)
    for mode in ("bf16", "fp32"):
        scores, _ = pipeline._production_scores(idx_q[:7].to(DEV), positions.to(DEV), buckets, config, mode)
        cent = (buckets.centroids_f32 if mode == "fp32" else buckets.centroids.float()).cpu().numpy()
        assert np.array_equal(_np(scores), oracle.canonical_scores(idx_q[:7].numpy(), cent, mode))


def test_centroids_and_position_buckets_match_oracle():
    idx_q, idx_k = _index_space(2048, 64, TIME + 10)
    config = PortConfig(cluster_block_size=512, bucket_size=8, bucket_cap=16)
    for centroid in ("normalized", "mean"):
        b = pipeline.position_buckets(idx_k.to(DEV), config, centroid=centroid)
        members = oracle.position_members(4, 512, 8, 16)
        assert np.array_equal(_np(b.members), members)
        want = oracle.bucket_centroids(idx_k.numpy(), members, centroid)
        assert np.array_equal(_np(b.centroids_f32), want)
        assert np.array_equal(_np(b.centroids.float()), oracle.bf16_round(want))


# ---------------------------------------------------------------- per-kv-head tables (benchmark geometry)


def test_per_kv_head_flat_select_clustered():
    T, Hq, Hkv, D = 4096, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=64, seed=3, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    config = workloads.FLAT_32K
    idx = pipeline.index_queries(data.q[:, -4:], Hkv)[0]  # [4, Hkv, D]
    positions = torch.tensor([T - 1, T - 100, 2000, 63], dtype=torch.int32)
    q_np = data.q[:, -4:].float().cpu().numpy()
    assert np.array_equal(_np(idx), oracle.index_queries(q_np, Hkv)[0])
    results = {impl: _switched(impl, idx, positions.to(DEV), buckets, config) for impl in
               ("reference", "fused", "fused_unpack")}
    for g in range(Hkv):
        cent = buckets.centroids[g].float().cpu().numpy()
        want_l, want_n = oracle.flat_select(_np(idx[:, g]), positions.numpy(), cent, _np(buckets.members[g]),
                                            cluster_block_size=64, block_buckets=1, top_p=32, top_k=8192,
                                            window=0, sink=0, mode="bf16", ends=_np(buckets.ends[g]))
        for impl, (l, n) in results.items():
            assert np.array_equal(_np(l[:, g]), want_l), f"{impl} kv-head {g}"
            assert np.array_equal(_np(n[:, g]), want_n), f"{impl} kv-head {g}"


@pytest.mark.parametrize("splits", ["1", "2", "3", "16", "64"])
def test_fused_split_counts_and_repeat_launches(splits, monkeypatch):
    """Every split count of the fused select gives the oracle's lists, on two launches in a
    row with different queries (the split keys and arrival counters are reused)."""
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=4, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    config = workloads.FLAT_32K
    monkeypatch.setenv("LSA_SELECT_SPLITS", splits)
    for rows in (slice(-1, None), slice(-3, -1)):
        idx = pipeline.index_queries(data.q[:, rows], Hkv)[0]
        positions = torch.full((idx.shape[0],), T - 1, dtype=torch.int32)
        got_l, got_n = _switched("fused", idx, positions.to(DEV), buckets, config)
        for g in range(Hkv):
            cent = buckets.centroids[g].float().cpu().numpy()
            want_l, want_n = oracle.flat_select(_np(idx[:, g]), positions.numpy(), cent, _np(buckets.members[g]),
                                                cluster_block_size=64, block_buckets=1, top_p=32, top_k=8192,
                                                window=0, sink=0, mode="bf16", ends=_np(buckets.ends[g]))
            assert np.array_equal(_np(got_l[:, g]), want_l), (splits, g)
            assert np.array_equal(_np(got_n[:, g]), want_n), (splits, g)


@pytest.mark.parametrize("rows_visible", [512, 20])
def test_fused_all_tied_scores_break_to_lower_bucket(rows_visible):
    """A zero index query ties every score: the picks are the lowest visible bucket ids, in
    ascending order (the packed key's column term), and EMPTY past the visible ones."""
    T, Hkv, D = 32768, 2, 128
    cap = 64
    members = torch.arange(512 * cap, dtype=torch.int32).view(512, cap).expand(Hkv, 512, cap).contiguous()
    cent = torch.randn(Hkv, 512, D, generator=torch.Generator().manual_seed(9)).bfloat16()
    buckets = Buckets(cent.to(DEV), members.to(DEV), torch.full((Hkv, 512), cap, dtype=torch.int32).to(DEV))
    config = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=64, top_p=32, top_k=4096,
                        window_size=0, sink_size=0)
    pos = torch.tensor([rows_visible * 64 - 1], dtype=torch.int32)
    idx = torch.zeros(1, Hkv, D, device=DEV)
    got_l, got_n = _switched("fused", idx, pos.to(DEV), buckets, config)
    for g in range(Hkv):
        want_l, want_n = oracle.flat_select(np.zeros((1, D), np.float32), pos.numpy(), cent[g].float().numpy(),
                                            members[g].numpy(), cluster_block_size=64, block_buckets=1, top_p=32,
                                            top_k=4096, window=0, sink=0, mode="bf16")
        assert np.array_equal(_np(got_l[:, g]), want_l) and np.array_equal(_np(got_n[:, g]), want_n)
        first = min(32, rows_visible - 1)  # a position sees the closed blocks before its own
        assert np.array_equal(want_l[0][: first * cap], np.arange(first * cap))


@pytest.mark.parametrize("window,sink,top_k", [(0, 0, 8192), (100, 4, 8192), (300, 16, 700)])
def test_fused_select_span_tables_match_member_rows(window, sink, top_k):
    """Span tables (contiguous segments) expanded from their ends (no member-row loads)
    give the lists the member rows give, and both equal the oracle's; the window and sink
    clip picks at both ends, and top_k cuts a pick short."""
    import dataclasses

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=17, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    assert buckets.spans
    config = dataclasses.replace(workloads.FLAT_32K, window_size=window, sink_size=sink, top_k=top_k)
    idx = pipeline.index_queries(data.q[:, -3:], Hkv)[0]  # [3, Hkv, D]
    positions = torch.tensor([T - 1, 5000, 700], dtype=torch.int32, device=DEV)
    got = _switched("fused", idx, positions, buckets, config)
    ref = _switched("fused", idx, positions, dataclasses.replace(buckets, spans=False), config)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    for g in range(Hkv):
        cent = buckets.centroids[g].float().cpu().numpy()
        want_l, want_n = oracle.flat_select(_np(idx[:, g]), _np(positions), cent, _np(buckets.members[g]),
                                            cluster_block_size=64, block_buckets=1, top_p=32, top_k=top_k,
                                            window=window, sink=sink, mode="bf16", ends=_np(buckets.ends[g]))
        assert np.array_equal(_np(got[0][:, g]), want_l) and np.array_equal(_np(got[1][:, g]), want_n)


@pytest.mark.parametrize("spans", [True, False])
def test_tree_select_fresh_buckets_and_shared_children(spans):
    """Nodes covering only the first 48 of 64 buckets (the rest join as fresh candidates
    once visible), a row early in the cache (growth has made 2 of the 3 nodes; its other
    visible buckets are fresh) and two nodes sharing children (each bucket must be a
    candidate once): lists equal the oracle's two-level beam, with span tables expanded
    from their ends or the member rows walked."""
    import dataclasses

    from lsa_rocm_lab.port.pipeline import Hierarchy, NodeLevel

    T, Hq, Hkv, D = 4096, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=32, seed=23, device=DEV)
    buckets = dataclasses.replace(workloads.cluster_buckets(data, target=64), spans=spans)
    children = torch.arange(48, dtype=torch.int32).view(3, 16).clone()
    children[2, :8] = children[1, :8]  # node 2 shares half its children with node 1
    children = children.expand(Hkv, 3, 16).contiguous().to(DEV)
    ncent = buckets.centroids_f32[:, children[0].long()].mean(dim=2).contiguous()  # [Hkv, 3, D]
    tree = Hierarchy(levels=[NodeLevel(ncent, children, centroids_bf16=ncent.to(torch.bfloat16))])
    config = dataclasses.replace(workloads.TREE_131K, beam_width=2, top_p=24, window_size=64, sink_size=4,
                                 node_cluster_block_size=16)
    idx = pipeline.index_queries(data.q[:, -2:], Hkv)[0]  # [2, Hkv, D]
    pos = torch.tensor([T - 1, 2500], dtype=torch.int32, device=DEV)
    for score_dtype in ("fp32", "bf16"):
        lists, lengths = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype=score_dtype)
        ends = _np(buckets.ends)
        for r in range(2):
            for g in range(Hkv):
                nc = (ncent if score_dtype == "fp32" else tree.levels[0].centroids_bf16.float())[g]
                bc = (buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float())[g]
                visible = int((ends[g] <= int(pos[r]) + 1).sum())
                want_l, want_n, _ = oracle.tree_select_row(
                    _np(idx[r, g]), _np(nc), _np(children[g]), _np(bc), _np(buckets.members[g]), int(pos[r]),
                    visible=visible, node_block=16, beam_width=2, top_p=24, top_k=config.top_k, window=64, sink=4,
                    mode=score_dtype)
                assert np.array_equal(_np(lists[r, g]), want_l), (score_dtype, r, g)
                assert int(lengths[r, g]) == want_n
