"""The one-launch decode with one selection a batch row shared by every kv-head
(``flat_decode_shared``, the reference's own decode layout: port/bench.py:147-153, one
index-space table, [B, W] lists shared by the heads).

Lists and lengths must be byte-identical to the fused select's on the same index queries
and table (and through it to the oracle's); outputs within max-abs 2e-2 / mean-abs 2e-3
of the fp64 oracle read of those lists, and bit-identical to the two-launch path
(select, then the split-K read) where the read's split matches, or across repeated
launches and a paged copy of the cache.
"""

import dataclasses
import os

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import _abi, workloads
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.pipeline import PortConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy() if t.is_floating_point() else t.detach().cpu().numpy()


def fused(*args, **kw):
    os.environ["LSA_SELECT_IMPL"] = "fused"
    try:
        return pipeline.flat_select(*args, **kw)
    finally:
        os.environ.pop("LSA_SELECT_IMPL", None)


def check_read(out, want, max_abs=2e-2, mean_abs=2e-3):
    err = np.abs(_np(out) - want)
    assert np.isfinite(err).all()
    assert err.max() <= max_abs and err.mean() <= mean_abs, (err.max(), err.mean())


@pytest.fixture(scope="module")
def space():
    return workloads.index_space(32768)


@pytest.mark.parametrize("positions", [[32767], [32764, 32765, 32766, 32767], [0, 5, 511, 512, 4095, 20000]])
def test_refcfg_shared_decode_equals_select_then_read(space, positions):
    """The reference's decode arm at its own knobs (PortConfig defaults: 4096 buckets,
    top_p 1024, top_k 4096, window 512, sink 4; 32k, Hq 32 / Hkv 8, D 128 bf16): the
    shared decode's lists equal the fused select's byte for byte (and the oracle's), its
    output is the read of those lists (bf16 bar against the fp64 oracle, each row against
    its own position), and a second launch repeats it bit for bit (the counters and the
    published keys were left zero). Rows at different positions share one cache."""
    cfg = PortConfig()
    D = 128
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    B = len(positions)
    print(f"case refcfg shared decode positions={positions}", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()  # [B, 1, Hq, D]
    idx = space.idx_q[pos.long()].contiguous()
    out, lists, lengths = pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg)
    want_l, want_n = fused(idx, pos, space.buckets, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lengths, want_n)
    assert torch.equal(lists, want_l)
    ol, on = oracle.flat_select(_np(idx), np.array(positions), _np(space.buckets.centroids.float()),
                                _np(space.buckets.members), cluster_block_size=cfg.cluster_block_size,
                                block_buckets=cfg.block_bucket_count, top_p=cfg.top_p, top_k=cfg.top_k,
                                window=cfg.window_size, sink=cfg.sink_size, mode="bf16")
    assert np.array_equal(_np(lists), ol) and np.array_equal(_np(lengths), on)
    k, v = _np(space.k), _np(space.v)
    for b in range(B):
        want = oracle.sparse_read(_np(q[b:b + 1]), k, v, _np(lists[b:b + 1])[None], _np(lengths[b:b + 1])[None],
                                  D ** -0.5)
        check_read(out[b:b + 1], want)
    again = pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg)
    torch.cuda.synchronize()
    for a, b_ in zip((out, lists, lengths), again):
        assert torch.equal(a, b_)


@pytest.mark.parametrize("splits,readers", [(1, 1), (3, 5), (64, 64), (17, 24)])
def test_shared_decode_any_launch_shape(space, splits, readers):
    """The select split and reader counts change only who does the work: lists are the
    same bytes at every shape, outputs within the bf16 bar of the oracle."""
    cfg = PortConfig()
    positions = [32767, 9000]
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    print(f"case shared decode splits={splits} readers={readers}", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    out, lists, lengths = pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg,
                                                      splits=splits, readers=readers)
    want_l, want_n = fused(idx, pos, space.buckets, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lists, want_l) and torch.equal(lengths, want_n)
    want = oracle.sparse_read(_np(q[:1]), _np(space.k), _np(space.v), _np(lists[:1])[None], _np(lengths[:1])[None],
                              128 ** -0.5)
    check_read(out[:1], want)


def test_shared_decode_paged_cache_is_the_same_read(space):
    """A paged copy of the cache (pages of 16 tokens in shuffled order in one pool, a slot
    table a batch row): the lists hold pool rows - the slot table applied to the unpaged
    lists - and the output is bit-identical to the unpaged launch's (the same rows read in
    the same order)."""
    cfg = PortConfig()
    positions = [32767, 17000]
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    print("case shared decode paged page=16", flush=True)
    B = len(positions)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    cache = workloads.paged(space.k.expand(B, -1, -1, -1).contiguous(), space.v.expand(B, -1, -1, -1).contiguous(),
                            page=16, seed=3, spare_pages=5)
    flat = pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg)
    paged = pipeline.flat_decode_shared(q, cache.k, cache.v, idx, pos, space.buckets, cfg, slot_table=cache.slot_table)
    torch.cuda.synchronize()
    assert torch.equal(paged[2], flat[2])
    want = oracle.map_slots(_np(flat[1]), _np(flat[2]), _np(cache.slot_table), np.arange(B))
    assert np.array_equal(_np(paged[1]), want)
    assert torch.equal(paged[0], flat[0])


def test_shared_decode_small_tables_fp16_d64_per_row_fp32_scores():
    """Reduced knobs and the other types: fp16 K/V, head dim 64, 4 query heads a kv-head,
    fp32 scores, one table a batch row (each row's own index space), a window and sinks
    wider than some rows' context, top_k clipping a pick. Lists equal the fused select's
    on each row's own table; outputs within the bar of the oracle."""
    T, Hq, Hkv, D = 4096, 16, 4, 64
    cfg = PortConfig(cluster_block_size=256, bucket_size=8, bucket_cap=16, top_p=40,
                     top_k=300, window_size=100, sink_size=4)
    spaces = [workloads.index_space(T, Hq, Hkv, D, seed=s, config=cfg, dtype=torch.float16) for s in (5, 6, 7)]
    positions = [4095, 1000, 60]
    B = len(positions)
    print("case shared decode per-row tables fp16 d64 fp32 scores", flush=True)
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    q = torch.stack([s.q[0, p] for s, p in zip(spaces, positions)])[:, None].contiguous()
    k = torch.cat([s.k for s in spaces]).contiguous()
    v = torch.cat([s.v for s in spaces]).contiguous()
    idx = torch.stack([s.idx_q[p] for s, p in zip(spaces, positions)]).contiguous()
    bs = [s.buckets for s in spaces]
    stacked = dataclasses.replace(bs[0], centroids=torch.stack([b.centroids for b in bs]),
                                  members=torch.stack([b.members for b in bs]),
                                  sizes=torch.stack([b.sizes for b in bs]),
                                  centroids_f32=torch.stack([b.centroids_f32 for b in bs]),
                                  ends=torch.stack([b.ends for b in bs]))
    out, lists, lengths = pipeline.flat_decode_shared(q, k, v, idx, pos, stacked, cfg, score_dtype="fp32")
    torch.cuda.synchronize()
    for b in range(B):
        wl, wn = fused(idx[b:b + 1], pos[b:b + 1], bs[b], cfg, score_dtype="fp32")
        assert torch.equal(lists[b:b + 1], wl) and torch.equal(lengths[b:b + 1], wn), b
        want = oracle.sparse_read(_np(q[b:b + 1]), _np(k[b:b + 1]), _np(v[b:b + 1]), _np(lists[b:b + 1])[None],
                                  _np(lengths[b:b + 1])[None], D ** -0.5)
        check_read(out[b:b + 1], want)
    assert int(lengths.min()) < cfg.top_k + cfg.window_size + cfg.sink_size


def test_shared_decode_gives_up_and_recovers(space):
    """The select workgroups withheld (a host test hook) with a tiny spin limit: every
    reader gives up, sets the status word and still arrives; the next call raises and
    zeroes the counters, and the call after it is bit-identical to one before."""
    cfg = PortConfig()
    pos = torch.tensor([32767], device=DEV, dtype=torch.int32)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    run = lambda: pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg)
    good = run()
    torch.cuda.synchronize()
    word = _abi.StatusWord.get(torch.device(DEV))
    assert int(word[0]) == 0
    lib = _abi.load()
    print("case shared decode give-up: skip_publish=1 spin_limit=64", flush=True)
    lib.lsa_debug_decode(1, 64)
    try:
        run()
        torch.cuda.synchronize()
    finally:
        lib.lsa_debug_decode(0, 0)
    assert int(word[0]) == 1
    with pytest.raises(_abi.LsaError, match="gave up"):
        run()
    assert int(word[0]) == 0
    again = run()
    torch.cuda.synchronize()
    for a, b in zip(good, again):
        assert torch.equal(a, b)


def test_shared_decode_rejects_what_it_cannot_hold(space):
    """More than 1024 picks or a table without span ends is refused before any launch."""
    cfg = dataclasses.replace(PortConfig(), top_p=2048)
    pos = torch.tensor([32767], device=DEV, dtype=torch.int32)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    with pytest.raises(ValueError, match="picks exceed"):
        pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, space.buckets, cfg)
    with pytest.raises(ValueError, match="span ends"):
        pipeline.flat_decode_shared(q, space.k, space.v, idx, pos, dataclasses.replace(space.buckets, spans=False),
                                    PortConfig())


# ---------------------------------------------------------------- the tree arm


@pytest.fixture(scope="module")
def tree(space):
    return pipeline.build_hierarchy_gpu(space.idx_k, space.buckets, PortConfig())


@pytest.mark.parametrize("score_dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("positions", [[32767], [32764, 32765, 32766, 32767], [0, 5, 511, 512, 4095, 4096, 20000]])
def test_refcfg_tree_shared_decode_equals_beam_then_read(space, tree, positions, score_dtype):
    """The reference's tree arm at its own knobs (node size 4, node blocks of 64, levels of
    1024/256/64 nodes, beam 64, top_p 1024 over 4096 buckets; 32k, Hq 32 / Hkv 8, D 128
    bf16): the shared tree decode's lists equal the beam select's byte for byte (rows whose
    growth starts the walk at levels 0..3), its output is the read of those lists (bf16 bar
    against the fp64 oracle), and a second launch repeats it bit for bit."""
    cfg = PortConfig()
    D = 128
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    B = len(positions)
    print(f"case refcfg tree shared decode positions={positions} scores={score_dtype}", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    out, lists, lengths = pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg,
                                                      score_dtype=score_dtype)
    want_l, want_n = pipeline.tree_select(idx, pos, space.buckets, tree, cfg, score_dtype=score_dtype)
    torch.cuda.synchronize()
    assert torch.equal(lengths, want_n)
    assert torch.equal(lists, want_l)
    k, v = _np(space.k), _np(space.v)
    for b in range(B):
        want = oracle.sparse_read(_np(q[b:b + 1]), k, v, _np(lists[b:b + 1])[None], _np(lengths[b:b + 1])[None],
                                  D ** -0.5)
        check_read(out[b:b + 1], want)
    again = pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg,
                                        score_dtype=score_dtype)
    torch.cuda.synchronize()
    for a, b_ in zip((out, lists, lengths), again):
        assert torch.equal(a, b_)


def test_refcfg_tree_shared_decode_matches_the_oracle_beam(space, tree):
    """The last row's list against the numpy beam walk itself (fp32 scores), not only
    against the GPU beam select."""
    cfg = PortConfig()
    T = 32768
    pos = torch.tensor([T - 1], device=DEV, dtype=torch.int32)
    print("case refcfg tree shared decode vs oracle beam", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    _, lists, lengths = pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg)
    torch.cuda.synchronize()
    levels = [(_np(lv.centroids), _np(lv.children)) for lv in tree.levels]
    vis = oracle.visible_counts(np.array([T - 1]), space.buckets.rows, cfg.cluster_block_size,
                                cfg.block_bucket_count)
    wl, wn, _ = oracle.beam_select_row(_np(idx[0]), levels, _np(space.buckets.centroids_f32),
                                       _np(space.buckets.members), T - 1, int(vis[0]), cfg.node_bucket_size,
                                       cfg.node_cluster_block_size, cfg.top_level, cfg.beam_width, cfg.top_p,
                                       cfg.top_k, cfg.window_size, cfg.sink_size, mode="fp32")
    assert int(lengths[0]) == wn
    assert np.array_equal(_np(lists[0]), wl)


@pytest.mark.parametrize("splits,readers", [(1, 1), (7, 9), (256, 64)])
def test_tree_shared_decode_any_launch_shape(space, tree, splits, readers):
    """Select splits (one workgroup scoring all 5440 columns, or 256 of them) and reader
    counts change only who does the work."""
    cfg = PortConfig()
    pos = torch.tensor([32767, 6000], device=DEV, dtype=torch.int32)
    print(f"case tree shared decode splits={splits} readers={readers}", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    out, lists, lengths = pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg,
                                                      splits=splits, readers=readers)
    want_l, want_n = pipeline.tree_select(idx, pos, space.buckets, tree, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lists, want_l) and torch.equal(lengths, want_n)
    want = oracle.sparse_read(_np(q[:1]), _np(space.k), _np(space.v), _np(lists[:1])[None], _np(lengths[:1])[None],
                              128 ** -0.5)
    check_read(out[:1], want)


def test_tree_shared_decode_paged_cache_is_the_same_read(space, tree):
    """A paged cache: the lists hold pool rows (the slot table applied to the unpaged
    lists) and the output is bit-identical to the unpaged launch's."""
    cfg = PortConfig()
    positions = [32767, 17000]
    B = len(positions)
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    print("case tree shared decode paged page=16", flush=True)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    cache = workloads.paged(space.k.expand(B, -1, -1, -1).contiguous(), space.v.expand(B, -1, -1, -1).contiguous(),
                            page=16, seed=4, spare_pages=3)
    flat = pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg)
    paged = pipeline.tree_decode_shared(q, cache.k, cache.v, idx, pos, space.buckets, tree, cfg,
                                        slot_table=cache.slot_table)
    torch.cuda.synchronize()
    assert torch.equal(paged[2], flat[2])
    want = oracle.map_slots(_np(flat[1]), _np(flat[2]), _np(cache.slot_table), np.arange(B))
    assert np.array_equal(_np(paged[1]), want)
    assert torch.equal(paged[0], flat[0])


def test_tree_shared_decode_small_per_row_tables_fp16_d64():
    """Reduced knobs and the other types: fp16 K/V, head dim 64, 4 query heads a kv-head,
    bf16 scores, one bucket table and hierarchy a batch row (each row its own index space),
    two node levels of node size 4 in blocks of 16, beam 8, top_p 24, a window and sinks
    wider than some rows' context. Lists equal the beam select's on each row's own tables;
    outputs within the bar of the oracle."""
    T, Hq, Hkv, D = 4096, 16, 4, 64
    cfg = PortConfig(cluster_block_size=256, bucket_size=8, bucket_cap=16, top_p=24, top_k=256, window_size=100,
                     sink_size=4, node_bucket_size=4, node_cluster_block_size=16, top_level=2, beam_width=8)
    spaces = [workloads.index_space(T, Hq, Hkv, D, seed=s, config=cfg, dtype=torch.float16) for s in (8, 9, 10)]
    trees = [pipeline.build_hierarchy_gpu(s.idx_k, s.buckets, cfg) for s in spaces]
    assert all(len(t.levels) == 2 for t in trees)
    positions = [4095, 1500, 60]
    B = len(positions)
    print("case tree shared decode per-row tables fp16 d64 bf16 scores", flush=True)
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    q = torch.stack([s.q[0, p] for s, p in zip(spaces, positions)])[:, None].contiguous()
    k = torch.cat([s.k for s in spaces]).contiguous()
    v = torch.cat([s.v for s in spaces]).contiguous()
    idx = torch.stack([s.idx_q[p] for s, p in zip(spaces, positions)]).contiguous()
    bs = [s.buckets for s in spaces]
    stacked = dataclasses.replace(bs[0], centroids=torch.stack([b.centroids for b in bs]),
                                  members=torch.stack([b.members for b in bs]),
                                  sizes=torch.stack([b.sizes for b in bs]),
                                  centroids_f32=torch.stack([b.centroids_f32 for b in bs]),
                                  ends=torch.stack([b.ends for b in bs]))
    levels = [pipeline.NodeLevel(centroids=torch.stack([t.levels[l].centroids for t in trees]),
                                 children=torch.stack([t.levels[l].children for t in trees]))
              for l in range(2)]
    stacked_tree = pipeline.Hierarchy(levels=levels)
    out, lists, lengths = pipeline.tree_decode_shared(q, k, v, idx, pos, stacked, stacked_tree, cfg,
                                                      score_dtype="bf16")
    torch.cuda.synchronize()
    for b in range(B):
        wl, wn = pipeline.tree_select(idx[b:b + 1], pos[b:b + 1], bs[b], trees[b], cfg, score_dtype="bf16")
        assert torch.equal(lists[b:b + 1], wl) and torch.equal(lengths[b:b + 1], wn), b
        want = oracle.sparse_read(_np(q[b:b + 1]), _np(k[b:b + 1]), _np(v[b:b + 1]), _np(lists[b:b + 1])[None],
                                  _np(lengths[b:b + 1])[None], D ** -0.5)
        check_read(out[b:b + 1], want)


def test_tree_shared_decode_gives_up_and_recovers(space, tree):
    """The select workgroups withheld (a host test hook) with a tiny spin limit: every
    reader gives up at its first level's gather, sets the status word and still arrives;
    the next call raises and zeroes the counters, and the call after it is bit-identical
    to one before."""
    cfg = PortConfig()
    pos = torch.tensor([32767], device=DEV, dtype=torch.int32)
    q = space.q[0, pos.long()][:, None].contiguous()
    idx = space.idx_q[pos.long()].contiguous()
    run = lambda: pipeline.tree_decode_shared(q, space.k, space.v, idx, pos, space.buckets, tree, cfg)
    good = run()
    torch.cuda.synchronize()
    word = _abi.StatusWord.get(torch.device(DEV))
    assert int(word[0]) == 0
    lib = _abi.load()
    print("case tree shared decode give-up: skip_publish=1 spin_limit=64", flush=True)
    lib.lsa_debug_decode(1, 64)
    try:
        run()
        torch.cuda.synchronize()
    finally:
        lib.lsa_debug_decode(0, 0)
    assert int(word[0]) == 1
    with pytest.raises(_abi.LsaError, match="gave up"):
        run()
    assert int(word[0]) == 0
    again = run()
    torch.cuda.synchronize()
    for a, b in zip(good, again):
        assert torch.equal(a, b)


def test_tree_shared_decode_wide_table_gathers_from_l2():
    """A 64k context at the reference knobs: 8192 buckets under levels of 2048/512/128 nodes
    (10880 published keys a row, too many for the reader's LDS beside the walk), so each
    level gathers its candidates' keys from the published ones in L2 instead of from the
    LDS copy. Lists equal the beam select's, outputs within the bar of the oracle."""
    cfg = PortConfig()
    T = 65536
    ws = workloads.index_space(T)
    tree = pipeline.build_hierarchy_gpu(ws.idx_k, ws.buckets, cfg)
    assert ws.buckets.rows == 8192 and sum(lv.centroids.shape[0] for lv in tree.levels) == 2688
    positions = [T - 1, 40000]
    pos = torch.tensor(positions, device=DEV, dtype=torch.int32)
    print("case tree shared decode 64k (keys from L2)", flush=True)
    q = ws.q[0, pos.long()][:, None].contiguous()
    idx = ws.idx_q[pos.long()].contiguous()
    out, lists, lengths = pipeline.tree_decode_shared(q, ws.k, ws.v, idx, pos, ws.buckets, tree, cfg)
    want_l, want_n = pipeline.tree_select(idx, pos, ws.buckets, tree, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lists, want_l) and torch.equal(lengths, want_n)
    want = oracle.sparse_read(_np(q[:1]), _np(ws.k), _np(ws.v), _np(lists[:1])[None], _np(lengths[:1])[None],
                              128 ** -0.5)
    check_read(out[:1], want)
