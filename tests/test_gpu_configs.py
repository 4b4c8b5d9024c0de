"""The five benchmark geometries end to end on the GPU vs the CPU oracle.

Selections (index queries, lists, lengths) must be bit-exact; read outputs within
max-abs 2e-2 / mean-abs 2e-3 of the fp64 oracle for bf16 (fp32: 1e-4). Full-size
decode configs are checked whole; the 32k prefill and the 131k x 32 tree are checked
on reduced contexts plus sampled rows at full size.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline

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


def decode_step(q, k, v, buckets, config, score_dtype="bf16"):
    Hkv = k.shape[2]
    T = k.shape[1]
    idx = pipeline.index_queries(q[:, -1:], Hkv)[0]
    pos = torch.tensor([T - 1], device=DEV, dtype=torch.int32)
    lists, lengths = fused(idx, pos, buckets, config, score_dtype=score_dtype)
    out = pipeline.lsa_read(q[:, -1:], k, v, lists.unsqueeze(0), lengths.unsqueeze(0), q.shape[-1] ** -0.5)
    return idx, lists, lengths, out


def oracle_select(idx, buckets, config, T, score_dtype="bf16"):
    Hkv = idx.shape[1]
    lists, lengths = [], []
    for g in range(Hkv):
        cent = (buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float())[g].cpu().numpy()
        ve = pipeline.visible_ends(buckets)
        ends = None if ve is None else ve[g].cpu().numpy()
        l, n = oracle.flat_select(_np(idx[:, g]), np.array([T - 1]), cent, buckets.members[g].cpu().numpy(),
                                  cluster_block_size=config.cluster_block_size,
                                  block_buckets=config.block_bucket_count, top_p=config.top_p, top_k=config.top_k,
                                  window=config.window_size, sink=config.sink_size, mode=score_dtype, ends=ends)
        lists.append(l[0])
        lengths.append(n[0])
    return np.stack(lists), np.array(lengths)


def test_decode_2k_fp32_positional():
    T, Hq, Hkv, D = 2048, 8, 2, 64
    q, k, v = workloads.geometry(T, Hq, Hkv, D, dtype=torch.float32, seed=0, device=DEV)
    config = workloads.DECODE_2K
    buckets = pipeline.position_buckets(k, config, centroid="mean")
    idx, lists, lengths, out = decode_step(q, k, v, buckets, config, score_dtype="fp32")
    want_l, want_n = oracle_select(idx, buckets, config, T, "fp32")
    assert np.array_equal(_np(lists[0]), want_l) and np.array_equal(_np(lengths[0]), want_n)
    assert (want_n == 512).all()
    for g in range(Hkv):  # block 0 and the last block are always read
        sel = set(want_l[g][: want_n[g]].tolist())
        assert set(range(64)) <= sel and set(range(T - 64, T)) <= sel
    want = oracle.sparse_read(_np(q[:, -1:]), _np(k), _np(v), want_l[None, None], want_n[None, None])
    check_read(out, want, max_abs=1e-4, mean_abs=1e-5)
    # dense SDPA over the same indices
    for g in range(Hkv):
        sel = torch.as_tensor(want_l[g][: want_n[g]], device=DEV, dtype=torch.long)
        qs = q[:, -1:, g * 4:(g + 1) * 4].permute(0, 2, 1, 3)
        ks = k[:, sel, g:g + 1].permute(0, 2, 1, 3).expand(1, 4, -1, D)
        vs = v[:, sel, g:g + 1].permute(0, 2, 1, 3).expand(1, 4, -1, D)
        ref = torch.nn.functional.scaled_dot_product_attention(qs, ks, vs).permute(0, 2, 1, 3)
        assert torch.allclose(out[:, :, g * 4:(g + 1) * 4].float(), ref.float(), atol=1e-4, rtol=1e-4)


def test_block_sparse_32k_bf16():
    T, Hq, Hkv, D = 32768, 32, 8, 128
    q, k, v = workloads.geometry(T, Hq, Hkv, D, dtype=torch.bfloat16, seed=0, device=DEV)
    config = workloads.BLOCK_SPARSE_32K
    buckets = pipeline.position_buckets(k, config, centroid="mean")
    idx, lists, lengths, out = decode_step(q, k, v, buckets, config)
    want_l, want_n = oracle_select(idx, buckets, config, T)
    assert np.array_equal(_np(lists[0]), want_l) and np.array_equal(_np(lengths[0]), want_n)
    assert (want_n == 2176).all()  # 34 blocks of 64
    for g in range(Hkv):
        blocks = set((want_l[g][: want_n[g]] // 64).tolist())
        assert len(blocks) == 34 and {0, 510, 511} <= blocks
    want = oracle.sparse_read(_np(q[:, -1:]), _np(k), _np(v), want_l[None, None], want_n[None, None])
    check_read(out, want)
    # the same step through the fused decode kernel (window and sink tails, 34 parts a head)
    pos = torch.tensor([T - 1], device=DEV, dtype=torch.int32)
    out2, lists2, lengths2 = pipeline.flat_decode(q[:, -1:], k, v, pos, buckets, config)
    assert np.array_equal(_np(lists2[0]), want_l) and np.array_equal(_np(lengths2[0]), want_n)
    check_read(out2, want)


def test_flat_decode_32k_clustered():
    T, Hq, Hkv, D = 32768, 32, 8, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=512, seed=0, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    sizes = _np(buckets.sizes)
    assert sizes.min() >= 16 and sizes.max() <= 256 and abs(sizes.mean() - 64) < 1e-9
    config = workloads.FLAT_32K
    idx, lists, lengths, out = decode_step(data.q, data.k, data.v, buckets, config)
    want_l, want_n = oracle_select(idx, buckets, config, T)
    assert np.array_equal(_np(lists[0]), want_l) and np.array_equal(_np(lengths[0]), want_n)
    want = oracle.sparse_read(_np(data.q[:, -1:]), _np(data.k), _np(data.v), want_l[None, None], want_n[None, None])
    check_read(out, want)


@pytest.mark.parametrize("T", [4096, 32768])
def test_flat_prefill_chunked(T):
    Hq, Hkv, D, chunk = 32, 8, 128, 64
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=512 if T == 32768 else 64, seed=1, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    config = workloads.FLAT_32K
    C = T // chunk
    idx = pipeline.index_queries(data.q, Hkv, chunk)[0]  # [C, Hkv, D]
    q_np = _np(data.q)
    pos = torch.arange(C, device=DEV, dtype=torch.int32) * chunk - 1
    lists, lengths = fused(idx, pos, buckets, config)
    out = pipeline.lsa_read_chunked(data.q, data.k, data.v, lists.unsqueeze(0), lengths.unsqueeze(0),
                                    D ** -0.5, chunk)
    rng = np.random.default_rng(0)
    chunks = sorted({0, 1, C - 1, *rng.integers(0, C, 3).tolist()})
    idx_np = oracle.index_queries(q_np[:, : C * chunk], Hkv, chunk)[0]
    assert np.array_equal(_np(idx)[chunks], idx_np[chunks])
    k_np, v_np = _np(data.k), _np(data.v)
    for c in chunks:
        for g in range(Hkv):
            cent = buckets.centroids[g].float().cpu().numpy()
            l, n = oracle.flat_select(idx_np[c, g][None], np.array([c * chunk - 1]), cent,
                                      buckets.members[g].cpu().numpy(), cluster_block_size=64, block_buckets=1,
                                      top_p=32, top_k=8192, window=0, sink=0, mode="bf16",
                                      ends=buckets.ends[g].cpu().numpy())
            assert np.array_equal(_np(lists[c, g]), l[0]), (c, g)
            assert int(lengths[c, g]) == int(n[0])
            assert (l[0][: n[0]] < c * chunk).all()  # buckets end at or before the chunk start
        rows = [c * chunk, c * chunk + 31, c * chunk + chunk - 1]
        ids = np.full((1, len(rows), Hkv, 8192 + chunk), -1, np.int32)
        lens = np.zeros((1, len(rows), Hkv), np.int32)
        for j, t in enumerate(rows):
            for g in range(Hkv):
                r = oracle.chunk_row_ids(_np(lists[c, g]), int(lengths[c, g]), t, chunk)
                ids[0, j, g, : r.size] = r
                lens[0, j, g] = r.size
        want = oracle.sparse_read(q_np[:, rows], k_np, v_np, ids, lens)
        check_read(out[:, rows], want)


def test_tree_decode_batched_reduced():
    B, T, Hq, Hkv, D = 3, 16384, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=256, seed=2, B=B, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)  # 256 buckets per (seq, kv-head)
    tree = workloads.node_tree(buckets, node_size=16)          # 16 nodes of 16
    config = workloads.TREE_131K
    config = pipeline.PortConfig(**{**config.__dict__, "beam_width": 4, "top_p": 16})
    idx = pipeline.index_queries(data.q[:, -1:], Hkv)[:, 0]   # [B, Hkv, D]
    pos = torch.full((B,), T - 1, device=DEV, dtype=torch.int32)
    for score_dtype in ("fp32", "bf16"):
        lists, lengths = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype=score_dtype)
        lvl = tree.levels[0]
        for b in range(B):
            for g in range(Hkv):
                ncent = (lvl.centroids if score_dtype == "fp32" else lvl.centroids_bf16.float())[b, g]
                bcent = (buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float())[b, g]
                l, n, _ = oracle.tree_select_row(
                    _np(idx[b, g]), _np(ncent), _np(lvl.children[b, g]), _np(bcent), _np(buckets.members[b, g]),
                    T - 1, visible=buckets.rows, node_block=config.node_cluster_block_size, beam_width=4, top_p=16,
                    top_k=8192,
                    window=0, sink=0, mode=score_dtype)
                assert np.array_equal(_np(lists[b, g]), l), (score_dtype, b, g)
                assert int(lengths[b, g]) == n
    # span tables expand from their ends: the member rows give the same lists, also with a
    # window and sinks clipping the picks
    import dataclasses

    members_only = dataclasses.replace(buckets, spans=False)
    for cfg in (config, dataclasses.replace(config, window_size=200, sink_size=4)):
        a = pipeline.tree_select(idx, pos, buckets, tree, cfg)
        b = pipeline.tree_select(idx, pos, members_only, tree, cfg)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # the read over per-(sequence, kv-head) lists
    out = pipeline.lsa_read(data.q[:, -1:], data.k, data.v, lists.unsqueeze(1), lengths.unsqueeze(1), D ** -0.5)
    want = oracle.sparse_read(_np(data.q[:, -1:]), _np(data.k), _np(data.v), _np(lists)[:, None],
                              _np(lengths)[:, None])
    check_read(out, want)


def test_tree_decode_ragged_positions_follow_growth():
    """Rows early in the cache: each (sequence, kv-head) sees only the buckets whose span
    has ended, node growth covers whole 64-bucket blocks of them, and the rest are fresh
    candidates - lists bit-exact against the oracle's growth replay."""
    B, T, Hq, Hkv, D = 3, 16384, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=256, seed=5, B=B, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    tree = workloads.node_tree(buckets, node_size=16)
    config = pipeline.PortConfig(**{**workloads.TREE_131K.__dict__, "beam_width": 4, "top_p": 16,
                                    "window_size": 128, "sink_size": 4})
    pos = torch.tensor([T - 1, 9000, 2500], device=DEV, dtype=torch.int32)
    idx = pipeline.index_queries(data.q[:, -1:], Hkv)[:, 0]
    ends = _np(buckets.ends)
    lvl = tree.levels[0]
    for score_dtype in ("fp32", "bf16"):
        lists, lengths = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype=score_dtype)
        for b in range(B):
            for g in range(Hkv):
                visible = int((ends[b, g] <= int(pos[b]) + 1).sum())
                ncent = (lvl.centroids if score_dtype == "fp32" else lvl.centroids_bf16.float())[b, g]
                bcent = (buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float())[b, g]
                l, n, picks = oracle.tree_select_row(
                    _np(idx[b, g]), _np(ncent), _np(lvl.children[b, g]), _np(bcent), _np(buckets.members[b, g]),
                    int(pos[b]), visible=visible, node_block=config.node_cluster_block_size, beam_width=4, top_p=16,
                    top_k=config.top_k, window=128, sink=4, mode=score_dtype)
                assert np.array_equal(_np(lists[b, g]), l), (score_dtype, b, g)
                assert int(lengths[b, g]) == n
                assert (picks[picks >= 0] < visible).all()


@pytest.mark.parametrize("readers", [None, 1, 7, 64])
@pytest.mark.parametrize("spans", [True, False])
def test_fused_tree_decode_equals_select_then_read(spans, readers):
    """The one-launch tree decode (lsa_decode_tree): lists and lengths byte-identical to
    tree_select on the group-mean index queries, at ragged positions (growth covers only
    whole node blocks, the rest are fresh; a row early enough to see no bucket reads its
    window and sinks alone), with span tables or member rows, in both
    scoring types, at the default reader count and at 1 (no partials), 7 and 64 (more
    readers than some rows' lists have tiles); the output within the bf16 bar of the fp64
    read over those lists."""
    import dataclasses

    B, T, Hq, Hkv, D = 3, 16384, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=256, seed=6, B=B, device=DEV)
    buckets = dataclasses.replace(workloads.cluster_buckets(data, target=T // 64), spans=spans)
    tree = workloads.node_tree(buckets, node_size=16)
    config = pipeline.PortConfig(**{**workloads.TREE_131K.__dict__, "beam_width": 4, "top_p": 16,
                                    "window_size": 128, "sink_size": 4})
    pos = torch.tensor([T - 1, 2500, 40], device=DEV, dtype=torch.int32)  # the last row sees no bucket
    q = data.q[:, -1:].contiguous()
    idx = pipeline.index_queries(q, Hkv)[:, 0]
    for score_dtype in ("bf16", "fp32"):
        print(f"case fused tree spans={spans} readers={readers} {score_dtype}", flush=True)
        out, lists, lengths = pipeline.tree_decode(q, data.k, data.v, pos, buckets, tree, config,
                                                   score_dtype=score_dtype, readers=readers)
        want_l, want_n = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype=score_dtype)
        assert torch.equal(lists, want_l) and torch.equal(lengths, want_n), score_dtype
        want = oracle.sparse_read(_np(q.float()), _np(data.k.float()), _np(data.v.float()), _np(lists)[:, None],
                                  _np(lengths)[:, None], D ** -0.5)
        err = np.abs(_np(out.float()) - want)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (score_dtype, err.max(), err.mean())


def test_tree_decode_configured_geometry():
    """The batched tree decode at its configured size: B=32 sequences x 131072 tokens,
    Hq 32 / Hkv 8, D 128 bf16, 2048 buckets = 128 nodes x 16 per (sequence, kv-head), top-8
    nodes then top-32 buckets. All 256 selections bit-exact against the oracle; the split
    read of 4 sequences within the bf16 bar (max-abs 2e-2, mean-abs 2e-3)."""
    B, T, Hq, Hkv, D = 32, 131072, 32, 8, 128
    print("tree 131k x 32: building the workload", flush=True)
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=2048, seed=0, B=B, device=DEV, gen_device=DEV,
                               q_tokens=1)
    buckets = workloads.cluster_buckets(data, target=2048, workers=8)
    tree = workloads.node_tree(buckets, node_size=16)
    config = workloads.TREE_131K
    assert buckets.rows == 2048 and tree.levels[0].children.shape[-2:] == (128, 16)
    pos = torch.full((B,), T - 1, device=DEV, dtype=torch.int32)
    idx = pipeline.index_queries(data.q, Hkv)[:, 0]  # [B, Hkv, D]
    lists, lengths = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype="bf16")
    out = pipeline.lsa_read(data.q, data.k, data.v, lists.unsqueeze(1), lengths.unsqueeze(1), D ** -0.5)
    torch.cuda.synchronize()
    print("tree 131k x 32: checking 256 selections", flush=True)
    lvl = tree.levels[0]
    idx_np, nc_np = _np(idx), _np(lvl.centroids_bf16)
    kids_np, bc_np, mem_np = _np(lvl.children), _np(buckets.centroids), _np(buckets.members)
    lists_np, lengths_np = _np(lists), _np(lengths)
    for b in range(B):
        for g in range(Hkv):
            l, n, _ = oracle.tree_select_row(idx_np[b, g], nc_np[b, g], kids_np[b, g], bc_np[b, g], mem_np[b, g],
                                             T - 1, visible=2048, node_block=config.node_cluster_block_size,
                                             beam_width=8, top_p=32, top_k=config.top_k, window=0, sink=0,
                                             mode="bf16")
            assert np.array_equal(lists_np[b, g], l), (b, g)
            assert int(lengths_np[b, g]) == n, (b, g)
    print("tree 131k x 32: checking the read of 4 sequences", flush=True)
    for b in (0, 11, 22, 31):
        want = oracle.sparse_read(_np(data.q[b:b + 1]), _np(data.k[b:b + 1]), _np(data.v[b:b + 1]),
                                  lists_np[b:b + 1, None], lengths_np[b:b + 1, None], D ** -0.5)
        check_read(out[b:b + 1], want)


def test_refcfg_prefill_32k_per_row_selection():
    """The reference's prefill arm at its own knobs (port/bench.py:113-154 with
    phase="prefill"; PortConfig() defaults: 512-key blocks of 64 buckets (cap 16), top_p
    1024 of up to 4096 visible buckets, top_k 4096, window 512, sink 4, one index-space
    table): all 32768 query rows select their own lists (4612 slots) in one fused select
    launch, then the per-row read. 64 sampled rows - block edges (the visible count steps
    at every 512th position), the first rows (nothing visible), the window's reach past
    the sinks, random rows - are bit-exact against the oracle; the read of 8 of them is
    within the bf16 bar of the fp64 oracle."""
    from lsa_rocm_lab.port.pipeline import PortConfig
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    cfg = PortConfig()
    T, D = 32768, 128
    print("case refcfg prefill 32k", flush=True)
    ws = workloads.index_space(T)
    pos = torch.arange(T, device=DEV, dtype=torch.int32)
    lists, lengths = fused(ws.idx_q, pos, ws.buckets, cfg)
    assert lists.shape == (T, cfg.top_k + cfg.window_size + cfg.sink_size)
    out = sparse_read_auto(ws.q, ws.k, ws.v, lists[None], lengths[None], D ** -0.5)
    torch.cuda.synchronize()
    rng = np.random.default_rng(7)
    edges = [0, 1, 3, 4, 5, 511, 512, 513, 515, 516, 1023, 1024, 1535, 4095, 4096, 8191, 8192, 16383, 16384,
             20479, 24575, 24576, 32255, 32256, 32766, 32767]
    rows = sorted(set(edges) | set(rng.integers(0, T, 64 - len(edges)).tolist()))
    assert len(rows) >= 64
    want_l, want_n = oracle.flat_select(_np(ws.idx_q[rows]), np.array(rows), _np(ws.buckets.centroids.float()),
                                        _np(ws.buckets.members), cluster_block_size=cfg.cluster_block_size,
                                        block_buckets=cfg.block_bucket_count, top_p=cfg.top_p, top_k=cfg.top_k,
                                        window=cfg.window_size, sink=cfg.sink_size, mode="bf16")
    assert np.array_equal(_np(lengths[rows]), want_n)
    assert np.array_equal(_np(lists[rows]), want_l)
    assert int(lengths.max()) <= cfg.top_k + cfg.window_size + cfg.sink_size
    some = [0, 512, 1024, 8192, 20000, 32256, 32600, 32767]
    want = oracle.sparse_read(_np(ws.q[:, some]), _np(ws.k), _np(ws.v), _np(lists[some])[None],
                              _np(lengths[some])[None], D ** -0.5)
    check_read(out[:, some], want)
