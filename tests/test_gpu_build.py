"""The bucket-table build on the GPU (contiguous Ward-style segments from the keys) vs the
CPU oracle.

Segment starts must equal the oracle's bit for bit (the merge order depends on exact fp64
costs). Cases: fp32 / bf16 / fp16 keys, head dims 32 / 64 / 128, pool sizes 4 / 8 / 16, a
shorter last pool, several (batch, kv-head) tables with strided cache views, the 32k
table of the benchmark geometry, ties (identical keys merge leftmost first), a target no
merge can reach under max_size (reported without a sync: check_build raises ValueError), and
the tables feeding the fused decode
(lists equal the oracle's flat select over the same tables). The block-structured build
(the reference's closed cluster blocks, 64 buckets of at most 16 keys a 512-key block)
matches the oracle per block and drives the flat select; a cache extended block by block
as it grows equals one built once.
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


def oracle_starts(keys, pool, target, max_size):
    B, T, H, D = keys.shape
    kf = keys.float().cpu().numpy()
    return np.stack([np.stack([oracle.ward_segments_keys(kf[b, :, g], pool, target, max_size) for g in range(H)])
                     for b in range(B)])


def clustered_keys(B, T, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    centers = torch.randn(B, H, 16, D, generator=g)
    runs = torch.randint(0, 16, (B, H, T // 24 + 1), generator=g).repeat_interleave(24, dim=-1)[..., :T]
    k = torch.gather(centers, 2, runs[..., None].expand(B, H, T, D)) + 0.3 * torch.randn(B, H, T, D, generator=g)
    return k.permute(0, 2, 1, 3).contiguous().to(dtype)


@pytest.mark.parametrize("dtype,D,pool,T,target,max_size", [
    (torch.bfloat16, 128, 16, 2048, 32, 256),
    (torch.float32, 64, 8, 1000, 40, 96),
    (torch.float16, 32, 4, 777, 50, 64),
    (torch.bfloat16, 128, 16, 4096, 64, 128),
])
def test_segment_starts_equal_oracle(dtype, D, pool, T, target, max_size):
    keys = clustered_keys(2, T, 2, D, dtype, seed=T + D)
    print(f"case {dtype} D={D} pool={pool} T={T} target={target} max={max_size}", flush=True)
    got = pipeline.segment_starts(keys.to(DEV), target, pool, max_size).cpu().numpy()
    assert np.array_equal(got, oracle_starts(keys, pool, target, max_size))


def test_segment_starts_on_a_strided_cache_view():
    """K rows read in place from a view of a wider cache (token stride 3 Hkv D)."""
    base = clustered_keys(1, 1536, 6, 64, torch.bfloat16, seed=8)
    view = base.to(DEV)[:, :, 2:4]  # kv-heads 2 and 3 of 6
    got = pipeline.segment_starts(view, 24, 16, 256).cpu().numpy()
    assert np.array_equal(got, oracle_starts(base[:, :, 2:4], 16, 24, 256))


def test_segment_starts_32k_table():
    """The benchmark geometry's table size: 32768 positions, 2048 pools -> 512 segments."""
    data = workloads.clustered(32768, 8, 2, 128, n_clusters=512, seed=3, device=DEV)
    got = pipeline.segment_starts(data.k, 512, 16, 256).cpu().numpy()
    assert np.array_equal(got, oracle_starts(data.k, 16, 512, 256))


def test_ties_merge_leftmost_and_unreachable_target_raises():
    keys = torch.ones(1, 64, 1, 64, dtype=torch.float32, device=DEV)
    assert pipeline.segment_starts(keys, 3, 8, 64).cpu().tolist() == [[[0, 48, 56, 64]]]
    pipeline.segment_starts(keys, 3, 8, 8)
    with pytest.raises(ValueError, match="could not reach"):
        pipeline.check_build()


def test_built_tables_drive_the_fused_decode():
    """Tables built on the GPU feed the fused decode (span tables); its lists equal the
    oracle's flat select over the same tables and its output the oracle read."""
    from test_gpu_decode import check_decode

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=21, device=DEV)
    buckets = pipeline.segment_buckets(data.k, T // 64, 16, 256)
    assert buckets.spans and buckets.members.shape == (Hkv, T // 64, 256)
    ends = buckets.ends.cpu().numpy()
    starts = oracle_starts(data.k, 16, T // 64, 256)[0]
    assert np.array_equal(ends, starts[:, 1:])
    members = buckets.members.cpu().numpy()
    for g in range(Hkv):
        want = oracle.bucket_centroids(data.k[0, :, g].float().cpu().numpy(), members[g], "mean")
        assert np.abs(buckets.centroids_f32[g].cpu().numpy() - want).max() <= 1e-5
    pos = torch.tensor([T - 1], dtype=torch.int32)
    check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K, label="built tables")


def oracle_block_tables(keys_2d, config, pool, max_size):
    """Per closed block: the oracle's segments, made absolute, rows block after block."""
    block, bpb = config.cluster_block_size, config.block_bucket_count
    starts = []
    for blk in range(keys_2d.shape[0] // block):
        st = oracle.ward_segments_keys(keys_2d[blk * block:(blk + 1) * block], pool, bpb, max_size)
        starts.append(st[:-1] + blk * block)
        last = st[-1] + blk * block
    begin = np.concatenate(starts)
    end = np.concatenate([begin[1:], [last]])
    members = np.full((begin.shape[0], config.bucket_cap), -1, dtype=np.int32)
    for r, (a, b) in enumerate(zip(begin, end)):
        members[r, :b - a] = np.arange(a, b)
    return members, end


def test_build_buckets_reference_blocks_and_select():
    """The reference's block structure (512-key blocks, 64 buckets of at most 16 keys from
    pools of 4, normalized-sum centroids) on one index-space table: members equal the
    oracle's per-block segments, centroids the oracle's, and the flat select over the
    tables (closed blocks before the query's own visible) equals the oracle's."""
    config = pipeline.PortConfig(top_p=16, top_k=256, window_size=64, sink_size=4)
    T, d = 2048 + 100, 64
    keys = clustered_keys(1, T, 1, d, torch.float32, seed=31)[0, :, 0]
    buckets = pipeline.build_buckets(keys.to(DEV), config)
    want_members, _ = oracle_block_tables(keys.numpy(), config, config.pool_size, config.bucket_cap)
    # the closed-block rule decides visibility; the span ends serve the expansion
    assert buckets.block_visible and buckets.spans and buckets.ends is not None
    assert np.array_equal(buckets.members.cpu().numpy(), want_members)
    cent = oracle.bucket_centroids(keys.numpy(), want_members, "normalized")
    assert np.abs(buckets.centroids_f32.cpu().numpy() - cent).max() <= 1e-6
    q = torch.randn(5, d, generator=torch.Generator().manual_seed(2))
    pos = torch.tensor([600, 1100, 1535, 1536, T - 1], dtype=torch.int32)
    lists, lengths = pipeline.flat_select(q.to(DEV), pos.to(DEV), buckets, config)
    wl, wn = oracle.flat_select(q.numpy(), pos.numpy(), buckets.centroids.float().cpu().numpy(), want_members,
                                cluster_block_size=config.cluster_block_size, block_buckets=config.block_bucket_count,
                                top_p=config.top_p, top_k=config.top_k, window=config.window_size,
                                sink=config.sink_size, mode="bf16")
    assert np.array_equal(lengths.cpu().numpy(), wn) and np.array_equal(lists.cpu().numpy(), wl)


def test_extend_buckets_equals_a_full_build():
    """A cache built at 3 closed blocks and extended as it grows to 5 (one block at a time,
    and with no new block) equals the tables built once at 5 blocks, field for field."""
    config = pipeline.PortConfig(cluster_block_size=256, bucket_size=16, bucket_cap=32, pool_size=8)
    keys = clustered_keys(1, 5 * 256 + 40, 2, 64, torch.bfloat16, seed=41).to(DEV)
    for spans in (False, True):
        grown = pipeline.build_buckets(keys[:, :3 * 256 + 10], config, spans=spans)
        for T in (3 * 256 + 200, 4 * 256, 5 * 256 + 40):
            grown = pipeline.extend_buckets(grown, keys[:, :T], config)
        full = pipeline.build_buckets(keys, config, spans=spans)
        for f in ("centroids", "members", "sizes", "centroids_f32", "ends"):
            a, b = getattr(grown, f), getattr(full, f)
            assert (a is None and b is None) or torch.equal(a, b), f
        assert grown.spans and grown.block_visible == (not spans)
    members, end = oracle_block_tables(keys[0, :, 1].float().cpu().numpy(), config, 8, 32)
    assert np.array_equal(full.members[1].cpu().numpy(), members)
    assert np.array_equal(full.ends[1].cpu().numpy(), end)


def test_extend_buckets_keeps_centroid_kind_and_optional_fields():
    """Extension builds the new rows as the tables were built: bucket-mean centroids stay
    means without repeating the kind, member-row tables get no span ends, and tables that
    carry no fp32 centroids (as a file may load them) get none appended."""
    import dataclasses

    config = pipeline.PortConfig(cluster_block_size=256, bucket_size=16, bucket_cap=32, pool_size=8)
    keys = clustered_keys(1, 5 * 256 + 40, 2, 64, torch.bfloat16, seed=43).to(DEV)
    for spans in (False, True):
        full = pipeline.build_buckets(keys, config, spans=spans, centroid="mean")
        part = pipeline.build_buckets(keys[:, :3 * 256 + 10], config, spans=spans, centroid="mean")
        grown = pipeline.extend_buckets(part, keys, config)
        assert grown.centroid == "mean" and grown.spans and grown.block_visible == (not spans)
        for f in ("centroids", "members", "sizes", "centroids_f32", "ends"):
            a, b = getattr(grown, f), getattr(full, f)
            assert (a is None and b is None) or torch.equal(a, b), (spans, f)
        bare = dataclasses.replace(part, centroids_f32=None, centroid=None)
        grown = pipeline.extend_buckets(bare, keys, config, centroid="mean")
        assert grown.centroids_f32 is None and torch.equal(grown.centroids, full.centroids)


def test_grow_buckets_in_place_equals_a_full_build(tmp_path):
    """Capacity tables reserved at 3 closed blocks (96 rows, 80 needed at 5 blocks) grow in
    place as the cache grows (a step that closes no block, then one block, then one more):
    no tensor moves; the built rows equal the tables built once at 5 blocks, the reserved
    rows stay empty (members -1, size 0, zero centroids, span end INT32_MAX); the flat
    select (both implementations) and the fused decode give the same lists and outputs on
    the capacity tables as on the full build; growth past the capacity raises; a saved
    capacity table loads as its built rows."""
    import dataclasses

    from lsa_rocm_lab.port import tables

    config = pipeline.PortConfig(cluster_block_size=256, bucket_size=16, bucket_cap=32, pool_size=8, top_p=8,
                                 top_k=200, window_size=32, sink_size=4)
    T_full = 5 * 256 + 40
    keys = clustered_keys(1, T_full, 2, 64, torch.bfloat16, seed=47).to(DEV)
    gen = torch.Generator().manual_seed(48)
    vals = torch.randn(1, T_full, 2, 64, generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn(1, 1, 4, 64, generator=gen).to(torch.bfloat16).to(DEV)
    for spans in (False, True):
        full = pipeline.build_buckets(keys, config, spans=spans)
        grown = pipeline.reserve_buckets(pipeline.build_buckets(keys[:, :3 * 256 + 10], config, spans=spans), 96)
        assert grown.built_rows == 48 and grown.rows == 96
        fields = ("centroids", "members", "sizes", "centroids_f32", "ends")
        ptrs = {f: getattr(grown, f).data_ptr() for f in fields if getattr(grown, f) is not None}
        for T in (3 * 256 + 200, 4 * 256, T_full):
            assert pipeline.grow_buckets_(grown, keys[:, :T], config) is grown
        assert grown.built_rows == 80
        assert {f: getattr(grown, f).data_ptr() for f in ptrs} == ptrs
        for f in fields:
            a, b = getattr(grown, f), getattr(full, f)
            assert (a is None and b is None) or torch.equal(a[:, :80], b), (spans, f)
        assert bool((grown.members[:, 80:] == -1).all()) and bool((grown.sizes[:, 80:] == 0).all())
        assert bool((grown.centroids[:, 80:] == 0).all()) and bool((grown.centroids_f32[:, 80:] == 0).all())
        if spans:
            assert bool((grown.ends[:, 80:] == pipeline.UNBUILT_END).all())
        else:  # empty spans at the last built end
            assert bool((grown.ends[:, 80:] == grown.ends[:, 79:80]).all())
        idx = pipeline.index_queries(keys[:, -5:], 2)[0]  # five query rows [5, 2, 64]
        pos = torch.tensor([T_full - 1, 1300, 1100, 600, 250], dtype=torch.int32, device=DEV)
        for impl in ("fused", "reference"):
            os.environ["LSA_SELECT_IMPL"] = impl
            a = pipeline.flat_select(idx, pos, grown, config)
            b = pipeline.flat_select(idx, pos, full, config)
            assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), (spans, impl)
        os.environ.pop("LSA_SELECT_IMPL")
        last = torch.tensor([T_full - 1], dtype=torch.int32, device=DEV)
        out_g, lists_g, n_g = pipeline.flat_decode(q, keys, vals, last, grown, config, scale=0.125)
        out_f, lists_f, n_f = pipeline.flat_decode(q, keys, vals, last, full, config, scale=0.125)
        assert torch.equal(lists_g, lists_f) and torch.equal(n_g, n_f) and torch.equal(out_g, out_f), spans
        assert pipeline.extend_buckets(grown, keys, config) is grown  # capacity tables grow in place
        path = tmp_path / f"grown{int(spans)}.safetensors"
        tables.save_buckets(path, grown)
        back = tables.load_buckets(path, DEV)
        assert back.rows == 80 and torch.equal(back.members, full.members) and back.built_rows is None
    small = pipeline.reserve_buckets(pipeline.build_buckets(keys[:, :3 * 256], config), 64)
    with pytest.raises(ValueError, match="capacity"):
        pipeline.grow_buckets_(small, keys, config)
    with pytest.raises(ValueError, match="capacity"):
        pipeline.reserve_buckets(full, 40)
    with pytest.raises(ValueError, match="capacity tables"):
        pipeline.grow_buckets_(dataclasses.replace(full), keys, config)


def test_tables_saved_and_loaded_select_alike(tmp_path):
    """Span tables built on the GPU, written to disk and loaded back onto the GPU, give
    the same fused-select lists as the tables in memory (and equal them field for field)."""
    from lsa_rocm_lab.port import tables

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=5, device=DEV)
    built = pipeline.segment_buckets(data.k, T // 64, 16, 256)
    tables.save_buckets(tmp_path / "idx.safetensors", built)
    loaded = tables.load_buckets(tmp_path / "idx.safetensors", DEV)
    for f in ("centroids", "members", "sizes", "centroids_f32", "ends"):
        a, b = getattr(built, f), getattr(loaded, f)
        assert (a is None and b is None) or torch.equal(a, b), f
    assert loaded.spans
    idx = pipeline.index_queries(data.q[:, -1:], Hkv)[0]
    pos = torch.full((idx.shape[0],), T - 1, dtype=torch.int32, device=DEV)
    la, na = pipeline.flat_select(idx, pos, built, workloads.FLAT_32K)
    lb, nb = pipeline.flat_select(idx, pos, loaded, workloads.FLAT_32K)
    assert torch.equal(na, nb) and torch.equal(la, lb)
