"""The multi-level beam select on the GPU vs the CPU oracle: bit-exact lists and lengths.

The hierarchy comes from ``build_hierarchy_gpu`` (checked against the oracle's builder);
the walk (``lsa_select_beam``) is held to ``oracle.beam_select_row`` row by row: growth
replay per row, start level, carried children, open nodes, first-occurrence dedup, ties
to the lower row, then the rank-order expansion. Cases: the reference's default knobs
(3 levels of 1024/256/64 nodes over 4096 buckets, beam 64, top_p 1024, window 512,
sink 4) in both scoring types; per-kv-head tables with four levels and a narrow beam; a
tree built before the cache grew (node counts cap the growth, buckets past the nodes'
reach are fresh) with top_level below the tree's depth; ragged span tables.
"""

import dataclasses

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.pipeline import PortConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _levels(hierarchy, table, score_dtype):
    """The oracle's [(centroids, children)] of one table, in the scoring type's values."""
    out = []
    for level in hierarchy.levels:
        cent = level.centroids if score_dtype == "fp32" else level.centroids_bf16
        out.append((_np(cent[table].float() if table is not None else cent.float()),
                    _np(level.children[table] if table is not None else level.children)))
    return out


def _check(lists, lengths, idx, positions, buckets, hierarchy, config, score_dtype, tables):
    """Every (row, group) of the GPU's lists against the oracle walk. tables: None (one
    shared table) or the kv-head count (one table per kv-head)."""
    bc = buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float()
    ve = pipeline.visible_ends(buckets)
    ends = None if ve is None else _np(ve)
    groups = 1 if tables is None else tables
    for g in range(groups):
        t = None if tables is None else g
        levels = _levels(hierarchy, t, score_dtype)
        cent = _np(bc if t is None else bc[t])
        members = _np(buckets.members if t is None else buckets.members[t])
        vis = oracle.visible_counts(_np(positions), members.shape[0], config.cluster_block_size,
                                    config.block_bucket_count, None if ends is None else (ends if t is None else ends[t]))
        for r in range(positions.shape[0]):
            q = _np(idx[r] if t is None else idx[r, g])
            want_l, want_n, _ = oracle.beam_select_row(
                q, levels, cent, members, int(positions[r]), int(vis[r]), config.node_bucket_size,
                config.node_cluster_block_size, config.top_level, config.beam_width, config.top_p, config.top_k,
                config.window_size, config.sink_size, mode=score_dtype)
            got_l = _np(lists[r] if t is None else lists[r, g])
            got_n = int(lengths[r] if t is None else lengths[r, g])
            assert np.array_equal(got_l, want_l), (score_dtype, r, g, int(positions[r]), int(vis[r]))
            assert got_n == want_n, (score_dtype, r, g)


def test_beam_reference_defaults_both_scoring_types():
    """32768 keys at the reference's defaults: 4096 buckets of 8 keys (cap 16), a 3-level
    hierarchy (1024, 256, 64 nodes), beam 64, top_p 1024, top_k 4096, window 512, sink 4.
    Rows before the first block, at block edges, mid-growth (start level 1 or 2) and at
    the end, in fp32 and bf16 scoring."""
    T, D = 32768, 128
    config = PortConfig()
    gen = torch.Generator().manual_seed(41)
    keys = torch.randn(T, D, generator=gen).to(DEV)
    buckets = pipeline.position_buckets(keys, config)
    tree = pipeline.build_hierarchy_gpu(keys, buckets, config)
    assert [lv.centroids.shape[0] for lv in tree.levels] == [1024, 256, 64]
    positions = torch.tensor([0, 511, 512, 1023, 4096, 4607, 16383, 16384, 20000, 32767, 30000, 8191, 8192,
                              24575, 2048, 100, 12000, 28000, 32000, 5000, 7000, 9000, 11000, 13000],
                             dtype=torch.int32, device=DEV)
    idx = torch.randn(positions.shape[0], D, generator=gen).to(DEV)
    for score_dtype in ("fp32", "bf16"):
        lists, lengths = pipeline.tree_select(idx, positions, buckets, tree, config, score_dtype=score_dtype)
        _check(lists, lengths, idx, positions, buckets, tree, config, score_dtype, None)


def test_build_hierarchy_matches_the_oracle_builder():
    """The GPU builder's bucket key sums, node sums and centroids equal the oracle's
    (same child order, fp32 sums in slot order): sums within 1e-6 relative, centroids
    within 1e-6."""
    T, D = 16384, 64
    config = PortConfig()
    gen = torch.Generator().manual_seed(43)
    keys = torch.randn(T, D, generator=gen)
    buckets = pipeline.position_buckets(keys.to(DEV), config)
    tree = pipeline.build_hierarchy_gpu(keys.to(DEV), buckets, config)
    sums = oracle.bucket_centroids(keys.numpy(), _np(buckets.members), "sum")
    np.testing.assert_allclose(_np(tree.bucket_key_sums), sums, rtol=1e-6, atol=1e-5)
    want = oracle.build_hierarchy(sums, config.node_bucket_size, config.node_cluster_block_size, config.top_level)
    assert len(tree.levels) == len(want) == 3  # 2048 buckets: 512 nodes, then 128, then 32
    for level, (cent, children, node_sums) in zip(tree.levels, want):
        assert np.array_equal(_np(level.children), children)
        np.testing.assert_allclose(_np(level.key_sums), node_sums, rtol=1e-5, atol=1e-4)
        np.testing.assert_allclose(_np(level.centroids), cent, rtol=1e-5, atol=1e-6)
        assert torch.equal(level.centroids_bf16, level.centroids.to(torch.bfloat16))


def test_beam_per_kv_head_four_levels_narrow_beam():
    """One table per kv-head (keys [1, T, Hkv, D]), 1024 buckets of 16 keys, node size 2
    in blocks of 8 (levels of 512, 256, 128, 64 nodes), beam 4, top_p 24, bf16 and fp32:
    the beam prunes at every level."""
    T, Hkv, D = 16384, 2, 64
    config = PortConfig(cluster_block_size=256, bucket_size=16, bucket_cap=16, top_p=24, top_k=300,
                        window_size=64, sink_size=4, node_bucket_size=2, node_cluster_block_size=8, top_level=4,
                        beam_width=4)
    gen = torch.Generator().manual_seed(44)
    keys = torch.randn(1, T, Hkv, D, generator=gen).to(DEV)
    buckets = pipeline.position_buckets(keys, config)
    tree = pipeline.build_hierarchy_gpu(keys, buckets, config)
    assert [lv.centroids.shape[-2] for lv in tree.levels] == [512, 256, 128, 64]
    R = 40
    positions = torch.linspace(0, T - 1, R).round().to(torch.int32).to(DEV)
    idx = torch.randn(R, Hkv, D, generator=gen).to(DEV)
    for score_dtype in ("bf16", "fp32"):
        lists, lengths = pipeline.tree_select(idx, positions, buckets, tree, config, score_dtype=score_dtype)
        _check(lists, lengths, idx, positions, buckets, tree, config, score_dtype, Hkv)


def test_beam_tree_older_than_the_cache_and_top_level_cut():
    """A hierarchy built over the first 8192 keys serves a 16384-key cache: the node
    counts cap the growth, so the buckets past the nodes' reach are all fresh; top_level
    2 walks only the lowest two of the tree's three levels."""
    T, D = 16384, 64
    config = PortConfig(cluster_block_size=128, bucket_size=8, bucket_cap=8, top_p=32, top_k=2000,
                        window_size=32, sink_size=4, node_bucket_size=2, node_cluster_block_size=16, top_level=3,
                        beam_width=3)
    gen = torch.Generator().manual_seed(45)
    keys = torch.randn(T, D, generator=gen).to(DEV)
    old = pipeline.position_buckets(keys[: T // 2], config)
    tree = pipeline.build_hierarchy_gpu(keys[: T // 2], old, config)
    assert [lv.centroids.shape[0] for lv in tree.levels] == [512, 256, 128]
    buckets = pipeline.position_buckets(keys, config)
    assert buckets.rows == 2048
    positions = torch.tensor([0, 127, 128, 2047, 4096, 8191, 8192, 9000, 12000, 16383], dtype=torch.int32,
                             device=DEV)
    idx = torch.randn(positions.shape[0], D, generator=gen).to(DEV)
    for top_level in (3, 2):
        cfg = dataclasses.replace(config, top_level=top_level)
        for score_dtype in ("fp32", "bf16"):
            lists, lengths = pipeline.tree_select(idx, positions, buckets, tree, cfg, score_dtype=score_dtype)
            _check(lists, lengths, idx, positions, buckets, tree, cfg, score_dtype, None)


@pytest.mark.parametrize("spans", [True, False])
def test_beam_ragged_span_tables(spans):
    """Ragged clustered tables (128 bucket spans of varying length, visibility from the
    span ends) under a two-level hierarchy (32 nodes, then 8): the span expansion and the member walk both give
    the oracle's lists."""
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=29, device=DEV)
    buckets = dataclasses.replace(workloads.cluster_buckets(data, target=T // 64), spans=spans)
    config = PortConfig(cluster_block_size=64, bucket_size=32, bucket_cap=256, top_p=16, top_k=1500,
                        window_size=64, sink_size=4, node_bucket_size=4, node_cluster_block_size=16, top_level=3,
                        beam_width=4)
    tree = pipeline.build_hierarchy_gpu(data.k, buckets, config)
    assert len(tree.levels) >= 2
    idx = pipeline.index_queries(data.q[:, -6:], Hkv)[0]  # [6, Hkv, D]
    positions = torch.tensor([T - 1, 6000, 3000, 1500, 400, 40], dtype=torch.int32, device=DEV)
    for score_dtype in ("bf16", "fp32"):
        lists, lengths = pipeline.tree_select(idx, positions, buckets, tree, config, score_dtype=score_dtype)
        _check(lists, lengths, idx, positions, buckets, tree, config, score_dtype, Hkv)


def test_beam_edges_no_growth_top_level_one_and_bf16_queries():
    """Rows that see no bucket or fewer than one node block (no node is made: the fresh
    buckets alone, or nothing and the tail only); top_level 1 over a 3-level hierarchy
    walks only level 1 and equals the one-level tree kernel; bf16 index queries."""
    T, D = 16384, 64
    config = PortConfig(cluster_block_size=128, bucket_size=8, bucket_cap=8, top_p=32, top_k=2000,
                        window_size=32, sink_size=4, node_bucket_size=2, node_cluster_block_size=16, top_level=3,
                        beam_width=3)
    gen = torch.Generator().manual_seed(46)
    keys = torch.randn(T, D, generator=gen).to(DEV)
    buckets = pipeline.position_buckets(keys, config)
    tree = pipeline.build_hierarchy_gpu(keys, buckets, config)
    assert len(tree.levels) == 3
    positions = torch.tensor([0, 5, 127, 128, 200, 2047, 2048, 16383], dtype=torch.int32, device=DEV)
    idx = torch.randn(positions.shape[0], D, generator=gen).to(DEV)
    for q in (idx, idx.to(torch.bfloat16)):
        lists, lengths = pipeline.tree_select(q, positions, buckets, tree, config, score_dtype="bf16")
        _check(lists, lengths, q.float(), positions, buckets, tree, config, "bf16", None)
    one = dataclasses.replace(config, top_level=1)
    a = pipeline.tree_select(idx, positions, buckets, tree, one)
    b = pipeline.tree_select(idx, positions, buckets, dataclasses.replace(tree, levels=tree.levels[:1]), one)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    _check(a[0], a[1], idx, positions, buckets, tree, one, "fp32", None)
