"""Synthetic select+read workloads: seeded q/k/v, clustered keys and the bucket tables
fed identically to the HIP path and to the CPU oracle.

Five geometries (batch B, context T, query heads Hq, kv-heads Hkv, head dim D):

* ``decode_2k_fp32``      B=1 T=2048 Hq=8 Hkv=2 D=64 fp32, positional blocks of 64,
                          block-mean centroids, top-8 blocks per kv-head with block 0
                          and the last block always in: 512 tokens per kv-head;
* ``block_sparse_32k``    B=1 T=32768 Hq=32 Hkv=8 D=128 bf16, 512 blocks of 64,
                          block-mean centroids, sink block 0 + the final 2 blocks as the
                          local window + the best 31 other blocks: 34 blocks (2176 tokens);
* ``flat_decode_32k``     same shape, keys from 512 Gaussian clusters per kv-head
                          (sigma 0.3, runs of 16-128 tokens), Ward-style buckets of
                          16-256 tokens (512 per kv-head), top-32 buckets, all members;
* ``flat_prefill_32k``    same keys, causal prefill in 64-token chunks sharing one
                          selection: chunk-mean query, buckets ending before the chunk,
                          top-32 + the chunk's causal block;
* ``tree_decode_131k``    B=32 T=131072, 2048 clusters, 2048 buckets = 128 nodes x 16,
                          top-8 nodes then top-32 of their 128 children.

Random draws use a seeded torch.Generator in a fixed order (q, then k's clusters and
noise, then v), on the CPU by default so every machine reproduces them bit for bit.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass

import numpy as np
import torch

from lsa_rocm_lab.port.pipeline import Buckets, Hierarchy, NodeLevel, PortConfig, bucket_centroids


@dataclass
class Clustered:
    """Clustered keys and their run structure (per table = per (batch, kv-head))."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    centers: torch.Tensor        # [B, Hkv, n_clusters, D] fp32 (CPU)
    run_lengths: torch.Tensor    # [B, Hkv, max_runs] int64 (CPU); runs cover T in order
    run_clusters: torch.Tensor   # [B, Hkv, max_runs] int64 (CPU)


def geometry(T: int, Hq: int, Hkv: int, D: int, dtype=torch.bfloat16, seed: int = 0, B: int = 1,
             device: str = "cuda") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v ~ N(0, 1), drawn q then k then v on a seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=g).to(dtype)
    k = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    return q.to(device), k.to(device), v.to(device)


def clustered(T: int, Hq: int, Hkv: int, D: int, n_clusters: int = 512, sigma: float = 0.3,
              dtype=torch.bfloat16, seed: int = 0, B: int = 1, device: str = "cuda",
              run_min: int = 16, run_max: int = 128, gen_device: str = "cpu",
              q_tokens: int | None = None) -> Clustered:
    """Keys from a mixture of Gaussian clusters: per (batch, kv-head) ``n_clusters`` centers
    ~ N(0, 1); the sequence is cut into runs of U{run_min..run_max} tokens, each run
    drawn from a cluster ~ U{0..n_clusters-1}; key = center + sigma * N(0, 1). q, v ~ N(0, 1).

    Draw order on the generator: q, centers, run lengths, run clusters, key noise, v.
    ``gen_device="cuda"`` draws the large tensors on the GPU's generator instead (fast
    for the 131k x 32 batch; reproducible on the same GPU, not bit-equal to the CPU draw).
    ``q_tokens``: draw only that many query rows (the last positions of a decode step,
    q [B, q_tokens, Hq, D]); a different draw from the full q.
    """
    g = torch.Generator().manual_seed(seed)
    gd = g if gen_device == "cpu" else torch.Generator(device=gen_device).manual_seed(seed)
    q = torch.randn(B, T if q_tokens is None else q_tokens, Hq, D, generator=gd, device=gen_device).to(dtype)
    centers = torch.randn(B, Hkv, n_clusters, D, generator=g)
    max_runs = T // run_min + 1
    run_lengths = torch.randint(run_min, run_max + 1, (B, Hkv, max_runs), generator=g)
    run_clusters = torch.randint(0, n_clusters, (B, Hkv, max_runs), generator=g)
    # token -> cluster per table
    ends = torch.cumsum(run_lengths, dim=-1)
    token = torch.arange(T)
    run_of_token = torch.searchsorted(ends, token.expand(B, Hkv, T).contiguous(), right=True)
    cluster_of_token = torch.gather(run_clusters, -1, run_of_token)  # [B, Hkv, T]
    noise = torch.randn(B, T, Hkv, D, generator=gd, device=gen_device)
    cdev = centers.to(gen_device)
    idx = cluster_of_token.to(gen_device)
    base = torch.gather(cdev, 2, idx[..., None].expand(B, Hkv, T, D))  # [B, Hkv, T, D]
    k = (base.permute(0, 2, 1, 3) + sigma * noise).to(dtype).contiguous()
    del base, noise
    v = torch.randn(B, T, Hkv, D, generator=gd, device=gen_device).to(dtype)
    return Clustered(q.to(device), k.to(device), v.to(device), centers, run_lengths, run_clusters)


def ward_segments(run_lengths: np.ndarray, run_clusters: np.ndarray, centers: np.ndarray, T: int,
                  target: int, max_size: int = 256, split_over: int = 64, min_size: int = 16) -> np.ndarray:
    """Ward-style contiguous buckets for one table: the cluster runs (the run cut at T
    joins its predecessor when shorter than ``min_size``), each run longer than
    ``split_over`` cut in two halves, then the adjacent pair with
    the smallest Ward cost n_a n_b / (n_a + n_b) * |mu_a - mu_b|^2 merged (mu = the
    size-weighted mean of the segment's cluster centers; a tie to the left pair; merges
    past ``max_size`` tokens are never taken) until ``target`` segments remain.
    Returns the segment start positions [target + 1] (last entry = T)."""
    sizes, mus = [], []
    pos = 0
    for n, c in zip(run_lengths.tolist(), run_clusters.tolist()):
        if pos >= T:
            break
        n = min(n, T - pos)
        if n < min_size and sizes:
            # the run cut by the end of the context joins the segment before it
            mus[-1] = (mus[-1] * sizes[-1] + centers[c].astype(np.float64) * n) / (sizes[-1] + n)
            sizes[-1] += n
            pos += n
            continue
        parts = [n // 2, n - n // 2] if n > split_over else [n]
        for p in parts:
            sizes.append(p)
            mus.append(centers[c].astype(np.float64))
        pos += n
    count = len(sizes)
    if count < target:
        raise ValueError(f"{count} segments cannot make {target} buckets")
    size = np.array(sizes, dtype=np.int64)
    sums = np.stack(mus) * size[:, None]
    left = np.arange(count) - 1
    right = np.arange(count) + 1
    right[-1] = -1
    alive = np.ones(count, dtype=bool)
    version = np.zeros(count, dtype=np.int64)

    def cost(a: int, b: int) -> float:
        na, nb = size[a], size[b]
        if na + nb > max_size:
            return float("inf")
        d = sums[a] / na - sums[b] / nb
        return float(na * nb / (na + nb) * (d @ d))

    heap = [(cost(i, i + 1), i, 0, 0) for i in range(count - 1)]
    heapq.heapify(heap)
    live = count
    while live > target:
        c, a, va, vb = heapq.heappop(heap)
        if c == float("inf"):
            raise ValueError("no admissible merge left under the size cap")
        b = right[a]
        if not alive[a] or b < 0 or version[a] != va or version[b] != vb:
            continue
        size[a] += size[b]
        sums[a] += sums[b]
        alive[b] = False
        right[a] = right[b]
        if right[b] >= 0:
            left[right[b]] = a
        version[a] += 1
        live -= 1
        if left[a] >= 0:
            la = left[a]
            heapq.heappush(heap, (cost(la, a), la, version[la], version[a]))
        if right[a] >= 0:
            ra = right[a]
            heapq.heappush(heap, (cost(a, ra), a, version[a], version[ra]))
    seg = size[alive]
    return np.concatenate([[0], np.cumsum(seg)]).astype(np.int64)


def segment_tables(starts: np.ndarray, cap: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Member tables of contiguous segments: starts [..., n + 1] -> members [..., n, cap]
    (-1 padded), sizes [..., n], exclusive ends [..., n]."""
    st = torch.as_tensor(starts, dtype=torch.int64, device=device)
    begin, end = st[..., :-1], st[..., 1:]
    sizes = (end - begin).to(torch.int32)
    slot = torch.arange(cap, device=device, dtype=torch.int64)
    members = begin[..., None] + slot
    members = torch.where(slot < sizes[..., None], members, torch.full_like(members, -1)).to(torch.int32)
    return members.contiguous(), sizes.contiguous(), end.to(torch.int32).contiguous()


def cluster_buckets(data: Clustered, target: int, cap: int = 256, max_size: int = 256,
                    workers: int = 1) -> Buckets:
    """Ward-style buckets per (batch, kv-head) with bucket-mean centroids. Tables are
    [Hkv, rows, ...] for B == 1, else [B, Hkv, rows, ...]. ``workers`` > 1 builds the
    tables in that many spawned CPU processes (they never touch the GPU)."""
    B, T, Hkv, D = data.k.shape
    starts = np.empty((B, Hkv, target + 1), dtype=np.int64)
    centers = data.centers.numpy()
    rl, rc = data.run_lengths.numpy(), data.run_clusters.numpy()
    jobs = [(b, g) for b in range(B) for g in range(Hkv)]
    if workers > 1 and len(jobs) > 1:
        import concurrent.futures
        import multiprocessing

        ctx = multiprocessing.get_context("spawn")
        with concurrent.futures.ProcessPoolExecutor(max_workers=workers, mp_context=ctx) as pool:
            futs = {pool.submit(ward_segments, rl[b, g], rc[b, g], centers[b, g], T, target, max_size): (b, g)
                    for b, g in jobs}
            for f, (b, g) in futs.items():
                starts[b, g] = f.result()
    else:
        for b, g in jobs:
            starts[b, g] = ward_segments(rl[b, g], rc[b, g], centers[b, g], T, target, max_size)
    if B == 1:
        starts = starts[0]
    members, sizes, ends = segment_tables(starts, cap, data.k.device)
    c32, c16 = bucket_centroids(data.k, members, "mean")
    # rows are exactly their spans when the segments start at 0 and none exceeds the cap
    spans = bool((starts[..., 0] == 0).all()) and int(sizes.max().item()) <= cap
    return Buckets(c16, members, sizes, centroids_f32=c32, ends=ends, spans=spans)


def node_tree(buckets: Buckets, node_size: int = 16) -> Hierarchy:
    """One node level over consecutive groups of ``node_size`` buckets; a node's centroid
    is the mean of its buckets' fp32 centroids (computed by the centroid kernel)."""
    c32 = buckets.centroids_f32
    lead = c32.shape[:-2]
    rows, D = c32.shape[-2:]
    n_nodes = rows // node_size
    children = torch.arange(n_nodes * node_size, device=c32.device, dtype=torch.int32).view(n_nodes, node_size)
    children = children.expand(*lead, n_nodes, node_size).contiguous()
    n_tables = int(np.prod(lead)) if len(lead) else 1
    keys = c32.reshape(n_tables, rows, 1, D)
    kids = children.reshape(n_tables, 1, n_nodes, node_size)
    n32, n16 = bucket_centroids(keys, kids, "mean")
    n32 = n32.reshape(*lead, n_nodes, D)
    n16 = n16.reshape(*lead, n_nodes, D)
    return Hierarchy(levels=[NodeLevel(n32, children, None, n16)])


@dataclass
class IndexSpace:
    """The reference's own benchmark inputs: q/k/v and one index-space table shared by
    every head (reference port/bench.py:75-81, :113-153)."""

    q: torch.Tensor      # [1, T, Hq, D]
    k: torch.Tensor      # [1, T, Hkv, D]
    v: torch.Tensor
    idx_q: torch.Tensor  # [T, D] fp32: the query heads' mean per position
    idx_k: torch.Tensor  # [T, D] fp32: the key heads' mean per position
    buckets: Buckets     # the closed blocks' bucket table over idx_k (one table)


def index_space(T: int = 32768, Hq: int = 32, Hkv: int = 8, D: int = 128, seed: int = 20261105,
                config: PortConfig | None = None, dtype=torch.bfloat16, device: str = "cuda") -> IndexSpace:
    """The reference's benchmark geometry at its default knobs: q/k/v ~ 0.2 N(0, 1) (drawn q,
    k, v on a seeded generator on ``device``), one index space shared by every head - here
    the mean over the query (key) heads, a stand-in for upstream's ``regroup`` - and its
    bucket table built block by block on the GPU (``build_buckets``: 512-key blocks of 64
    buckets of at most 16 keys, normalized-sum centroids)."""
    from lsa_rocm_lab.port.pipeline import build_buckets, index_queries

    config = PortConfig() if config is None else config
    gen = torch.Generator(device=device).manual_seed(seed)
    q, k, v = ((torch.randn(1, T, h, D, device=device, generator=gen) * 0.2).to(dtype) for h in (Hq, Hkv, Hkv))
    idx_k = index_queries(k, 1)[0, :, 0].contiguous()
    idx_q = index_queries(q, 1)[0, :, 0].contiguous()
    return IndexSpace(q, k, v, idx_q, idx_k, build_buckets(idx_k, config))


@dataclass
class PagedCache:
    """A cache moved into one pool of fixed-size pages, in shuffled page order."""

    k: torch.Tensor           # [1, pool_rows, Hkv, D]: every batch row's pages
    v: torch.Tensor
    slot_table: torch.Tensor  # [B, T] int32: (batch row, position) -> pool row


def paged(k: torch.Tensor, v: torch.Tensor, page: int = 16, seed: int = 0, spare_pages: int = 0) -> PagedCache:
    """A paged copy of a cache k/v [B, T, Hkv, D]: every batch row's positions cut into
    pages of ``page`` tokens, all rows' pages (plus ``spare_pages`` unused ones) placed in a
    seeded random order in one pool, and the slot table mapping each (row, position) to
    its pool row - the layout a serving engine's page allocator leaves behind (``page=1``:
    every token on its own, the worst case for locality)."""
    B, T, Hkv, D = k.shape
    per_row = -(-T // page)
    n_pages = B * per_row + spare_pages
    g = torch.Generator().manual_seed(seed)
    where = torch.randperm(n_pages, generator=g)[: B * per_row].view(B, per_row)  # page j of row b
    slots = (where[:, :, None] * page + torch.arange(page)).reshape(B, per_row * page)[:, :T]
    slots = slots.to(device=k.device, dtype=torch.int32).contiguous()
    pool_k = torch.zeros(1, n_pages * page, Hkv, D, dtype=k.dtype, device=k.device)
    pool_v = torch.zeros_like(pool_k)
    flat = slots.reshape(-1).long()
    pool_k[0, flat] = k.reshape(B * T, Hkv, D)
    pool_v[0, flat] = v.reshape(B * T, Hkv, D)
    return PagedCache(pool_k, pool_v, slots)


# ----------------------------------------------------------------------------- configs

DECODE_2K = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=64, top_p=7, top_k=384,
                       window_size=64, sink_size=64)
BLOCK_SPARSE_32K = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=64, top_p=33, top_k=1984,
                              window_size=128, sink_size=64)
FLAT_32K = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=256, top_p=32, top_k=8192,
                      window_size=0, sink_size=0)
TREE_131K = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=256, top_p=32, top_k=8192,
                       window_size=0, sink_size=0, node_bucket_size=16, beam_width=8)
