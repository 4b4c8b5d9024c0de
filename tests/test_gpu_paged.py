"""Paged K/V caches on the GPU: the slot table (logical position -> cache row) applied where
the reference's expansion applies it (select_fused.py:147-205, MAP_SLOTS: every kept id and
the window/sink tail, chosen on logical positions, stored as its cache row).

For each entry that writes read lists - the fused decode (rank, exchange and replicated
forms; span and member tables), the tree decode, the three flat-select implementations, the
one-level tree and multi-level beam selects, the expansion from keys - the paged lists must
equal the oracle's logical lists mapped through the slot table (``oracle.map_slots``), bit
for bit, with the same lengths; the read over the row-shuffled pool must equal the unpaged
read bit for bit (the same rows in the same order, so the same arithmetic), and the unpaged
read stays within the dtype's bar of the fp64 oracle. The chunked prefill read maps its
causal block through the table (MFMA and gather kernels). Edge cases: page size 1 (every
token on its own) and 16, spare pool pages, batch rows with their own table rows, -1 table
entries and a table narrower than the positions (those ids list as -1 and are skipped).
"""

import dataclasses

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline, select_fused
from lsa_rocm_lab.port.pipeline import PortConfig
from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_chunked

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _mapped(lists, lengths, slot_table, slot_rows=None):
    """The oracle's map of logical GPU lists [R, ..., W] through the slot table."""
    R = lists.shape[0]
    rows = np.zeros(R, np.int64) if slot_rows is None else _np(slot_rows)
    return oracle.map_slots(_np(lists), _np(lengths), _np(slot_table), rows)


def _oracle_lists(idx, pos, buckets, config, score_dtype="bf16"):
    """Oracle flat-select lists [B, Hkv, W] / lengths [B, Hkv] on per-kv-head tables."""
    B, Hkv = idx.shape[:2]
    cents = buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float()
    ls, ns = [], []
    for b in range(B):
        lb, nb = [], []
        for g in range(Hkv):
            sel = (b, g) if buckets.members.dim() == 4 else (g,)
            ve = pipeline.visible_ends(buckets)
            ends = None if ve is None else _np(ve[sel])
            l, n = oracle.flat_select(_np(idx[b, g])[None], np.array([int(pos[b])]), _np(cents[sel]),
                                      _np(buckets.members[sel]), cluster_block_size=config.cluster_block_size,
                                      block_buckets=config.block_bucket_count, top_p=config.top_p,
                                      top_k=config.top_k, window=config.window_size, sink=config.sink_size,
                                      mode=score_dtype, ends=ends)
            lb.append(l[0])
            nb.append(n[0])
        ls.append(np.stack(lb))
        ns.append(np.array(nb))
    return np.stack(ls), np.stack(ns)


def _clustered(T=8192, Hq=8, Hkv=2, D=128, B=1, seed=11):
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=seed, B=B, device=DEV)
    return data, workloads.cluster_buckets(data, target=T // 64)


@pytest.mark.parametrize("form,splits", [("rank", None), ("exchange", 1), ("replicated", 0), ("members", None)])
@pytest.mark.parametrize("page", [1, 16])
def test_paged_flat_decode(form, splits, page):
    """The fused decode over a row-shuffled pool: lists = the oracle's logical lists mapped
    through the slot table, output = the unpaged decode's, bit for bit."""
    print(f"case paged flat decode form={form} page={page}", flush=True)
    data, buckets = _clustered()
    if form == "members":
        buckets = dataclasses.replace(buckets, spans=False)
    T = data.k.shape[1]
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    cfg = dataclasses.replace(workloads.FLAT_32K, window_size=64, sink_size=4, top_k=2048)
    pc = workloads.paged(data.k, data.v, page=page, seed=page, spare_pages=7)
    out0, l0, n0 = pipeline.flat_decode(q, data.k, data.v, pos, buckets, cfg, splits=splits)
    out1, l1, n1 = pipeline.flat_decode(q, pc.k, pc.v, pos, buckets, cfg, splits=splits, slot_table=pc.slot_table)
    want_l, want_n = _oracle_lists(pipeline.index_queries(q, 2)[:, 0], pos, buckets, cfg)
    assert np.array_equal(_np(l0), want_l) and np.array_equal(_np(n0), want_n)
    assert np.array_equal(_np(n1), want_n)
    assert np.array_equal(_np(l1), _mapped(l0, n0, pc.slot_table))
    assert torch.equal(out0, out1)
    pipeline.check_decode()


def test_paged_decode_batch_rows_share_one_pool():
    """Two sequences (own tables, own positions) in one pool: slot row b maps sequence b."""
    print("case paged decode B=2 one pool", flush=True)
    data, buckets = _clustered(B=2, seed=12)
    T = data.k.shape[1]
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1, T - 300], dtype=torch.int32, device=DEV)
    cfg = dataclasses.replace(workloads.FLAT_32K, window_size=32, sink_size=8, top_k=4096)
    pc = workloads.paged(data.k, data.v, page=8, seed=3)
    out0, l0, n0 = pipeline.flat_decode(q, data.k, data.v, pos, buckets, cfg)
    out1, l1, n1 = pipeline.flat_decode(q, pc.k, pc.v, pos, buckets, cfg, slot_table=pc.slot_table)
    rows = torch.arange(2, dtype=torch.int32)
    assert np.array_equal(_np(n1), _np(n0))
    assert np.array_equal(_np(l1), _mapped(l0, n0, pc.slot_table, rows))
    assert torch.equal(out0, out1)
    # slot rows given explicitly and swapped: the two sequences' tables are swapped
    swapped = torch.stack([pc.slot_table[1], pc.slot_table[0]])
    out2, l2, _ = pipeline.flat_decode(q, pc.k, pc.v, pos, buckets, cfg, slot_table=swapped,
                                       slot_rows=torch.tensor([1, 0], dtype=torch.int32, device=DEV))
    assert torch.equal(l2, l1) and torch.equal(out2, out1)
    pipeline.check_decode()


def test_paged_decode_holes_and_a_narrow_table():
    """Slot-table entries of -1 (no cache row) and a table narrower than the position: those
    ids list as -1 and the read skips them (the output equals the read of the mapped list)."""
    print("case paged decode holes", flush=True)
    data, buckets = _clustered(seed=13)
    T = data.k.shape[1]
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    cfg = dataclasses.replace(workloads.FLAT_32K, window_size=16, sink_size=4, top_k=2048)
    pc = workloads.paged(data.k, data.v, page=4, seed=5)
    table = pc.slot_table.clone()
    table[0, 100:300] = -1
    narrow = table[:, : T - 8].contiguous()  # the window's last 8 positions fall off the table
    out0, l0, n0 = pipeline.flat_decode(q, data.k, data.v, pos, buckets, cfg)
    out1, l1, n1 = pipeline.flat_decode(q, pc.k, pc.v, pos, buckets, cfg, slot_table=narrow)
    want = _mapped(l0, n0, narrow)
    assert (want == -1).sum() > (_np(l0) == -1).sum()  # holes were hit
    assert np.array_equal(_np(n1), _np(n0)) and np.array_equal(_np(l1), want)
    # the read skips the holes: the oracle's read of the logical list with those ids dropped
    logical = np.where(want >= 0, _np(l0), -1)
    ref = oracle.sparse_read(_np(q.float()), _np(data.k.float()), _np(data.v.float()), logical[:, None],
                             _np(n0)[:, None], 128 ** -0.5)
    err = np.abs(_np(out1.float()) - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
    pipeline.check_decode()


def test_paged_tree_decode():
    print("case paged tree decode", flush=True)
    data, buckets = _clustered(T=16384, seed=14)
    tree = workloads.node_tree(buckets, node_size=16)
    T = data.k.shape[1]
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    cfg = dataclasses.replace(workloads.TREE_131K, window_size=32, sink_size=4)
    pc = workloads.paged(data.k, data.v, page=16, seed=6)
    out0, l0, n0 = pipeline.tree_decode(q, data.k, data.v, pos, buckets, tree, cfg)
    out1, l1, n1 = pipeline.tree_decode(q, pc.k, pc.v, pos, buckets, tree, cfg, slot_table=pc.slot_table)
    assert np.array_equal(_np(n1), _np(n0))
    assert np.array_equal(_np(l1), _mapped(l0, n0, pc.slot_table))
    assert torch.equal(out0, out1)
    pipeline.check_decode()


@pytest.mark.parametrize("impl", ["reference", "fused", "fused_unpack"])
def test_paged_flat_select_every_implementation(impl, monkeypatch):
    """Positional block tables at the reference's default knobs (top_p 1024, top_k 4096,
    window 512, sink 4, one shared table), four query rows at different positions, each with
    its own slot-table row: lists = the oracle's logical lists mapped, lengths equal."""
    print(f"case paged flat select impl={impl}", flush=True)
    monkeypatch.setenv("LSA_SELECT_IMPL", impl)
    cfg = PortConfig()
    T, D = 16384, 128
    g = torch.Generator().manual_seed(21)
    keys = torch.randn(T, D, generator=g).to(DEV)
    buckets = pipeline.position_buckets(keys, cfg)
    idx = torch.randn(4, D, generator=g).to(DEV)
    pos = torch.tensor([T - 1, 9000, 1500, 511], dtype=torch.int32, device=DEV)
    table = torch.stack([torch.randperm(T + 64, generator=torch.Generator().manual_seed(s))[:T]
                         for s in range(3)]).to(torch.int32).to(DEV)
    rows = torch.tensor([2, 0, 1, 2], dtype=torch.int32, device=DEV)
    l1, n1 = pipeline.flat_select(idx, pos, buckets, cfg, slot_table=table, slot_rows=rows)
    want_l, want_n = oracle.flat_select(_np(idx), _np(pos), _np(buckets.centroids.float()), _np(buckets.members),
                                        cluster_block_size=cfg.cluster_block_size,
                                        block_buckets=cfg.block_bucket_count, top_p=cfg.top_p, top_k=cfg.top_k,
                                        window=cfg.window_size, sink=cfg.sink_size, mode="bf16")
    assert np.array_equal(_np(n1), want_n)
    assert np.array_equal(_np(l1), oracle.map_slots(want_l, want_n, _np(table), _np(rows)))


def test_paged_expand_from_keys():
    """select_fused.expand_in_order_from_keys with the slot map (the reference kernel's
    MAP_SLOTS path) against the oracle's expansion mapped."""
    print("case paged expand from keys", flush=True)
    g = torch.Generator().manual_seed(22)
    rows, cap, T = 256, 16, 4096
    members = torch.arange(rows * cap, dtype=torch.int32).view(rows, cap)
    members[::5, 9:] = -1
    scores = torch.randn(3, rows, generator=g)
    lengths = torch.tensor([rows, 100, 31], dtype=torch.int32)
    keys = select_fused.select_topk_scores(scores.to(DEV), lengths.to(DEV), 64)
    pos = torch.tensor([T - 1, 1700, 600], dtype=torch.int32)
    table = torch.randperm(T, generator=g).to(torch.int32)[None].to(DEV)
    l1, n1 = select_fused.expand_in_order_from_keys(keys, members.to(DEV), pos.to(DEV), 128, 4, 512,
                                                    slot_table=table)
    want_l, want_n = oracle.expand_in_order(oracle.unpack_ids(_np(keys)), _np(members), _np(pos), 128, 4, 512)
    assert np.array_equal(_np(n1), want_n)
    assert np.array_equal(_np(l1), oracle.map_slots(want_l, want_n, _np(table), np.zeros(3)))


@pytest.mark.parametrize("levels", [1, 3])
def test_paged_tree_and_beam_select(levels):
    """The one-level tree select and the 3-level beam with a slot map: the lists are their
    unpaged lists mapped, lengths equal."""
    print(f"case paged tree select levels={levels}", flush=True)
    cfg = PortConfig() if levels == 3 else dataclasses.replace(PortConfig(), top_level=1)
    T, D = 32768, 128
    g = torch.Generator().manual_seed(23)
    keys = torch.randn(T, D, generator=g).to(DEV)
    buckets = pipeline.build_buckets(keys, cfg)
    tree = pipeline.build_hierarchy_gpu(keys, buckets, cfg)
    assert len(tree.levels) == levels
    idx = torch.randn(3, D, generator=g).to(DEV)
    pos = torch.tensor([T - 1, 20000, 3000], dtype=torch.int32, device=DEV)
    table = torch.randperm(T, generator=g).to(torch.int32)[None].to(DEV)
    l0, n0 = pipeline.tree_select(idx, pos, buckets, tree, cfg)
    l1, n1 = pipeline.tree_select(idx, pos, buckets, tree, cfg, slot_table=table)
    assert np.array_equal(_np(n1), _np(n0))
    assert np.array_equal(_np(l1), _mapped(l0, n0, table))


@pytest.mark.parametrize("path", ["mfma", "gather"])
def test_paged_chunked_prefill_read(path):
    """The chunked prefill read over a shuffled pool: the chunk lists mapped through the
    table, the causal block mapped in the kernel; output = the unpaged read's, bit for bit,
    and the unpaged read within the bf16 bar of the oracle."""
    print(f"case paged chunked read path={path}", flush=True)
    T, Hq, Hkv, D, chunk, W = 512, 8, 2, 128, 64, 160
    g = torch.Generator().manual_seed(24)
    B = 2
    q = (torch.randn(B, T, Hq, D, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(B, T, Hkv, D, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    C = T // chunk
    ids = torch.full((B, C, Hkv, W), -1, dtype=torch.int32)
    lens = torch.zeros(B, C, Hkv, dtype=torch.int32)
    for b in range(B):
        for c in range(1, C):
            for h in range(Hkv):
                n = int(torch.randint(1, W + 1, (1,), generator=g))
                ids[b, c, h, :n] = torch.randint(0, c * chunk, (n,), generator=g, dtype=torch.int32)
                lens[b, c, h] = n
    ids, lens = ids.to(DEV), lens.to(DEV)
    pc = workloads.paged(k, v, page=16, seed=9, spare_pages=3)
    mapped = torch.from_numpy(np.stack([oracle.map_slots(_np(ids[b]).reshape(C, Hkv, W), _np(lens[b]),
                                                         _np(pc.slot_table), np.full(C, b))
                                        for b in range(B)])).to(DEV)
    out0 = sparse_read_chunked(q, k, v, ids, lens, None, chunk, path=path)
    out1 = sparse_read_chunked(q, pc.k, pc.v, mapped, lens, None, chunk, path=path, slot_table=pc.slot_table)
    assert torch.equal(out0, out1)
    want = oracle.sparse_read_chunked(_np(q.float()), _np(k.float()), _np(v.float()), _np(ids), _np(lens), chunk)
    err = np.abs(_np(out0.float()) - want)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_paged_decode_32k_full_size():
    """The 32k flat decode (Hq 32 / Hkv 8 / D 128 bf16, 512 Ward buckets a kv-head, top-32)
    over a pool of 16-token pages: lists bit-exact against the oracle's mapped lists on
    every kv-head, output equal to the unpaged decode's."""
    print("case paged decode 32k", flush=True)
    T = 32768
    data = workloads.clustered(T, 32, 8, 128, n_clusters=512, seed=0, device=DEV)
    buckets = workloads.cluster_buckets(data, target=512)
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    cfg = workloads.FLAT_32K
    pc = workloads.paged(data.k, data.v, page=16, seed=1)
    out0, l0, n0 = pipeline.flat_decode(q, data.k, data.v, pos, buckets, cfg)
    out1, l1, n1 = pipeline.flat_decode(q, pc.k, pc.v, pos, buckets, cfg, slot_table=pc.slot_table)
    want_l, want_n = _oracle_lists(pipeline.index_queries(q, 8)[:, 0], pos, buckets, cfg)
    assert np.array_equal(_np(n0), want_n) and np.array_equal(_np(l0), want_l)
    assert np.array_equal(_np(n1), want_n)
    assert np.array_equal(_np(l1), oracle.map_slots(want_l, want_n, _np(pc.slot_table), np.zeros(1)))
    assert torch.equal(out0, out1)
    pipeline.check_decode()


def test_grow_buckets_without_a_host_sync():
    """Index growth into capacity tables issues no host sync (torch's sync debug mode raises
    on any), and the grown tables equal the tables built at once."""
    print("case grow without sync", flush=True)
    cfg = PortConfig()
    T, D = 8192, 128
    g = torch.Generator().manual_seed(25)
    keys = torch.randn(1, T, 2, D, generator=g).to(torch.bfloat16).to(DEV)
    once = pipeline.build_buckets(keys, cfg, spans=True)
    tabs = pipeline.reserve_buckets(pipeline.build_buckets(keys[:, : T - 1024], cfg, spans=True), 2 * T // 8)
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        pipeline.grow_buckets_(tabs, keys, cfg)
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    pipeline.check_build()
    rows = once.rows
    assert tabs.built_rows == rows
    assert torch.equal(tabs.members[:, :rows], once.members) and torch.equal(tabs.ends[:, :rows], once.ends)
    assert torch.equal(tabs.centroids[:, :rows], once.centroids)


def test_build_failure_is_reported_without_a_sync():
    """A table that cannot reach its segment count under max_size (32 positions, pools of
    4, 2 segments of at most 8) holds the even cut and sets the pinned build word: the next
    build raises, and check_build raises too."""
    print("case build failure word", flush=True)
    keys = torch.randn(1, 32, 1, 128).to(torch.bfloat16).to(DEV)
    starts = pipeline.segment_starts(keys, target=2, pool=4, max_size=8)
    torch.cuda.synchronize()
    assert _np(starts[0, 0]).tolist() == [0, 16, 32]  # the even cut
    with pytest.raises(ValueError, match="could not reach"):
        pipeline.segment_starts(keys, target=4, pool=4, max_size=8)
    pipeline.segment_starts(keys, target=2, pool=4, max_size=8)
    with pytest.raises(ValueError, match="could not reach"):
        pipeline.check_build()
    pipeline.check_build()  # the word was cleared
