"""CPU oracle: a numpy restatement of the reference's select+read path.

TEST INFRASTRUCTURE. This module is what the HIP path is compared
against. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it; the product package never does.

Every function cites the reference file:line whose behaviour it restates
(paths are relative to the reference repository root). Where the reference
delegates to the un-vendored upstream ``lsa`` package (Prefrontal-AI/
latent-sparse-attention @ 5ebea732d639576d2a7579b0de40e6252f9001f5), the
restatement follows the reference's call sites and docs, and the header of the
function says what pins it.

Pinning (what each function is checked against in tests/test_oracle.py):
  ordered_bits / pack_keys       monotone vs float order (argsort), ties -> lower column,
                                 EMPTY sorts last; closed form on special values
  best_first_keys                numpy/torch full sort + slice (library routine)
  select_topk_scores             brute force: rank by (score desc, column asc)
  unpack_ids                     round trip with pack_keys
  expand_in_order                a literal per-element loop on tiny inputs + invariants
                                 (causality, tail counts, prefix = members of picks)
  canonical_scores               fp64 closed form (error <= 2^-24 rel), exact rationals
  index_queries                  torch mean in fp64 (tolerance) and exact pow2 cases
  bucket_centroids               fp64 closed form
  sparse_read                    torch SDPA on full causal lists (textbook), duplicate ->
                                 V row, empty -> 0 / NaN
  tree_select_row / tree_growth  brute-force sort of every candidate on tiny trees; the
                                 growth replay of _tree.py:100-142 restated literally
                                 (page ends, block counts) on small tables
  beam_growth / beam_select_row  the multi-level replay restated literally (every page
                                 end, every level's block closing); a brute-force walk of
                                 every level by plain sorting on tiny three-level trees
  build_hierarchy                level counts vs the reference loop's stop rule
                                 (:166-170) by hand; sums by linearity (a level's total =
                                 the buckets' total, fp64); unit-norm centroids. The
                                 grouping is this build's (the Ward pairing is upstream's).
  ward_pair_cost                 exact rational arithmetic (fractions) and math.fsum
  ward_segments_keys             brute force (every adjacent cost recomputed from the
                                 segments each step, no links), two-cluster closed form,
                                 invariants (contiguous cover, target count, max_size)
  map_slots                      the identity table is the identity; a permutation's inverse
                                 recovers the logical lists; the read over a row-shuffled
                                 pool with mapped lists equals the unpaged read
  window/sink tail order         PARITY UNPINNED (upstream _append_window_and_sink is not
                                 available); the tail SET is pinned by causality and the
                                 read output is order-invariant.
  NaN / -0.0 key bits            PARITY UNPINNED against upstream ordered_bits; the
                                 map used here is the standard signed-order map.
"""

from __future__ import annotations

import numpy as np

# Upstream keys.EMPTY (called at reference select_fused.py:43, pipeline.py:203-205):
# int64 min, sorts after every real key.
EMPTY = np.int64(-(1 << 63))
COL_TOP = np.int64(0x7FFFFFFF)
# Partial sums per dot product in the canonical score order (see canonical_scores).
SCORE_PARTIALS = 16


def next_pow2(n: int) -> int:
    """triton.next_power_of_2 (reference select_fused.py:123-124)."""
    n = int(n)
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


# --------------------------------------------------------------------------- numbers


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 with round-to-nearest-even, returned as fp32 (torch ``.to(bfloat16)``).

    Reference pipeline.py:228 rounds the index queries to bf16 before scoring.
    NaN becomes the canonical quiet NaN 0x7FC0.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32)
    out = np.where(np.isnan(x), np.uint32(0x7FC00000), out)
    return out.view(np.float32)


def ordered_bits(scores: np.ndarray) -> np.ndarray:
    """fp32 bits -> int32 whose signed order is the float order (upstream keys.ordered_bits).

    Called at reference select_fused.py:76. Non-negative floats keep their bits;
    negative floats flip the 31 magnitude bits. -0.0 orders just below +0.0.
    """
    bits = np.ascontiguousarray(scores, dtype=np.float32).view(np.int32)
    return bits ^ ((bits >> 31) & np.int32(0x7FFFFFFF))


def pack_keys(scores: np.ndarray, lengths: np.ndarray) -> np.ndarray:
    """Whole-path listing: every column packed, EMPTY at or past the row's length.

    Reference pipeline.py:266-267 (upstream ``TopK(top_p, exact=False).listed`` on
    the whole path, ``columns <= 4 * top_p``) and the in-register pack of
    select_fused.py:71-77: ``key = (ordered_bits(s) << 32) | (0x7FFFFFFF - column)``.
    """
    scores = np.asarray(scores, dtype=np.float32)
    rows, cols = scores.shape
    column = np.arange(cols, dtype=np.int64)
    keys = (ordered_bits(scores).astype(np.int64) << np.int64(32)) | (COL_TOP - column)[None, :]
    live = column[None, :] < np.asarray(lengths, dtype=np.int64).reshape(rows, 1)
    return np.where(live, keys, EMPTY)


def best_first_keys(keys: np.ndarray, top_p: int, counts: np.ndarray | None = None) -> np.ndarray:
    """The ``min(top_p, W)`` greatest keys per row, descending (reference pipeline.py:189-214).

    ``counts`` masks slots at or past each row's count to EMPTY first (:210-213).
    """
    keys = np.asarray(keys, dtype=np.int64)
    width = keys.shape[1]
    k = min(int(top_p), width)
    if counts is not None:
        listed = np.arange(width)[None, :] < np.asarray(counts, dtype=np.int64)[:, None]
        keys = np.where(listed, keys, EMPTY)
    return np.sort(keys, axis=1)[:, ::-1][:, :k].copy()


def unpack_ids(keys: np.ndarray) -> np.ndarray:
    """Key -> column (int32), -1 for EMPTY (upstream keys.unpack_ids / key_bucket;
    reference pipeline.py:268, select_fused.py:189; EXPERIMENT_DECISIONS.md:35)."""
    keys = np.asarray(keys, dtype=np.int64)
    col = COL_TOP - (keys & np.int64(0xFFFFFFFF))
    return np.where(keys == EMPTY, -1, col).astype(np.int32)


def select_topk_scores(scores: np.ndarray, lengths: np.ndarray, top_p: int) -> np.ndarray:
    """Fused pack + best-first top-k (reference select_fused.py:83-137, kernel :52-80).

    Output [R, K2], K2 = next_pow2(min(top_p, N)); EMPTY pads the tail. Rows wider than
    4 * top_p take the length-respecting fallback (:97-117): the same keys, at the width
    ``torch.topk(k=min(top_p, N))`` returns, [R, min(top_p, N)].
    """
    scores = np.asarray(scores, dtype=np.float32)
    rows, cols = scores.shape
    keep = min(int(top_p), cols)
    k2 = next_pow2(keep)
    best = best_first_keys(pack_keys(scores, lengths), keep)
    if cols > 4 * int(top_p):
        return best
    out = np.full((rows, k2), EMPTY, dtype=np.int64)
    out[:, :keep] = best
    return out


# --------------------------------------------------------------------------- expansion


def window_and_sink(position: int, window: int, sink: int) -> np.ndarray:
    """The list tail: the window [window_start, position] ascending, then the sinks
    [0, min(sink, window_start)) ascending.

    Reference contract: read_kernel.py:11-13 ("the expansion, the window, then the
    sinks") and select_fused.py:175, :203-213. The element order inside the tail is
    upstream's ``_append_window_and_sink`` and is PARITY UNPINNED; the set is fixed
    by causality (window ids <= position, sinks not already in the window).
    """
    window_start = max(0, int(position) + 1 - int(window))
    win = np.arange(window_start, int(position) + 1, dtype=np.int32)
    sinks = np.arange(0, min(int(sink), window_start), dtype=np.int32)
    return np.concatenate([win, sinks])


def expand_row(picks: np.ndarray, members: np.ndarray, position: int, window: int, sink: int,
               top_k: int) -> tuple[np.ndarray, int]:
    """One row of the rank-order expansion (reference select_fused.py:172-214).

    Picks in rank order, each bucket's member slots in table order; a member is kept
    iff ``bucket >= 0 and id >= sink and id < window_start`` (:195), the first
    ``top_k`` kept ids are stored (:196-201), then the window/sink tail follows.
    A pick outside ``[0, rows)`` contributes nothing (EMPTY / -1 picks, :187-194).
    """
    width = int(top_k) + int(window) + int(sink)
    out = np.full(width, -1, dtype=np.int32)
    window_start = max(0, int(position) + 1 - int(window))
    picks = np.asarray(picks, dtype=np.int64)
    picks = picks[(picks >= 0) & (picks < members.shape[0])]
    ids = members[picks].reshape(-1)
    kept = ids[(ids >= sink) & (ids < window_start)][: int(top_k)]
    out[: kept.size] = kept
    tail = window_and_sink(position, window, sink)
    out[kept.size: kept.size + tail.size] = tail
    return out, int(kept.size + tail.size)


def expand_in_order(picks: np.ndarray, members: np.ndarray, positions: np.ndarray, window: int,
                    sink: int, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """Upstream ``expand_in_order`` / port ``expand_in_order_from_keys`` (reference
    pipeline.py:269-271, select_fused.py:217-280): lists [R, top_k+window+sink]
    int32 (-1 padded) and lengths [R] int32. ``members`` is [rows, cap] shared by
    every row, or [R, rows, cap] (a table per row)."""
    picks = np.asarray(picks)
    rows = picks.shape[0]
    lists = np.full((rows, int(top_k) + int(window) + int(sink)), -1, dtype=np.int32)
    lengths = np.zeros(rows, dtype=np.int32)
    for r in range(rows):
        table = members if members.ndim == 2 else members[r]
        lists[r], lengths[r] = expand_row(picks[r], table, int(positions[r]), window, sink, top_k)
    return lists, lengths


def map_slots(lists: np.ndarray, lengths: np.ndarray, slot_table: np.ndarray,
              slot_rows: np.ndarray) -> np.ndarray:
    """A paged cache's read lists (reference select_fused.py:176-178, :197-199, :205, the
    ``MAP_SLOTS`` path of the expansion): every listed id - the kept ids and the
    window/sink tail, chosen on logical positions first - becomes
    ``slot_table[slot_rows[r], id]``; the -1 padding stays. An id at or past the table's
    width (or a table row outside the table) maps to -1 here, where the reference's masked
    load has no bound. lists [R, ..., W] with lengths [R, ...]; slot_table [n_rows, width],
    slot_rows [R]."""
    lists = np.asarray(lists)
    lengths = np.asarray(lengths)
    table = np.asarray(slot_table).reshape(-1, np.asarray(slot_table).shape[-1])
    out = np.full_like(lists, -1)
    width = lists.shape[-1]
    for r in range(lists.shape[0]):
        k = int(slot_rows[r])
        row = table[k] if 0 <= k < table.shape[0] else np.zeros(0, dtype=table.dtype)
        lr, nr = lists[r].reshape(-1, width), lengths[r].reshape(-1)
        o = out[r].reshape(-1, width)
        for g in range(lr.shape[0]):
            n = int(nr[g])
            ids = lr[g, :n].astype(np.int64)
            ok = (ids >= 0) & (ids < row.size)
            o[g, :n] = np.where(ok, row[np.where(ok, ids, 0)] if row.size else -1, -1)
    return out


def visible_counts(positions: np.ndarray, rows: int, cluster_block_size: int, block_buckets: int,
                   ends: np.ndarray | None = None) -> np.ndarray:
    """Buckets a query may score (reference pipeline.py:184-186).

    Without ``ends``: ``(pos // cluster_block_size * block_buckets).clamp_max(rows)``
    (floor division, negative counts list nothing). With ``ends`` (the exclusive end
    of each bucket's span, nondecreasing - the clustered tables): the number of
    buckets whose span ends at or before ``pos + 1``.
    """
    positions = np.asarray(positions, dtype=np.int64)
    if ends is None:
        return np.minimum((positions // cluster_block_size) * block_buckets, rows).astype(np.int32)
    return np.searchsorted(np.asarray(ends, dtype=np.int64), positions + 1, side="right").astype(np.int32)


# --------------------------------------------------------------------------- scoring


def canonical_scores(queries: np.ndarray, centroids: np.ndarray, mode: str = "bf16") -> np.ndarray:
    """``queries @ centroids.T`` in a fixed canonical arithmetic, fp32 out.

    Reference pipeline.py:217-232 (``torch.mm`` bf16 x bf16 -> fp32, or fp32 x fp32 on
    ``centroids_f32``). The reference's summation order is rocBLAS's; the oracle fixes
    one: operands rounded to the mode's type (bf16 RNE, or fp32), products and sums in
    fp64, 16 partial sums each over a contiguous D/16 slice accumulated in order, the
    16 partials combined by the tree (p, p+8), (p, p+4), (p, p+2), (p, p+1), then one
    rounding to fp32. Products of bf16 or fp32 operands are exact in fp64, so the GPU's
    fused multiply-add gives the same bits as this multiply-then-add.
    """
    q = np.asarray(queries, dtype=np.float32)
    c = np.asarray(centroids, dtype=np.float32)
    if mode == "bf16":
        q, c = bf16_round(q), bf16_round(c)
    elif mode != "fp32":
        raise ValueError(f"score mode must be bf16|fp32, got {mode!r}")
    rows, dim = q.shape
    cols = c.shape[0]
    if dim % SCORE_PARTIALS:
        raise ValueError(f"index dim {dim} must be a multiple of {SCORE_PARTIALS}")
    span = dim // SCORE_PARTIALS
    q64 = q.astype(np.float64).reshape(rows, 1, SCORE_PARTIALS, span)
    c64 = c.astype(np.float64).reshape(1, cols, SCORE_PARTIALS, span)
    out = np.empty((rows, cols), dtype=np.float32)
    step = max(1, (1 << 22) // max(1, cols * dim))
    for r0 in range(0, rows, step):
        prod = q64[r0:r0 + step] * c64
        acc = np.zeros(prod.shape[:3], dtype=np.float64)
        for j in range(span):
            acc = acc + prod[..., j]
        a = acc[..., :8] + acc[..., 8:]
        b = a[..., :4] + a[..., 4:]
        t = b[..., :2] + b[..., 2:]
        out[r0:r0 + step] = (t[..., 0] + t[..., 1]).astype(np.float32)
    return out


def index_queries(q: np.ndarray, heads_kv: int, chunk: int = 1) -> np.ndarray:
    """GQA-collapsed index queries: the mean over each kv-head's query group and over
    ``chunk`` consecutive tokens, fp32.

    Reference gates.py:50-59 collapses GQA through upstream ``regroup``; the benchmark
    geometry instead specifies the per-kv-head mean over the group (and the chunk mean
    for chunked prefill). Canonical order: fp32 sum over tokens of the chunk, within a
    token over the group's heads in order, then one fp32 division by the count.
    q [B, T, Hq, D] -> [B, T // chunk, Hkv, D].
    """
    q = np.asarray(q, dtype=np.float32)
    b, t, hq, d = q.shape
    group = hq // heads_kv
    n_chunks = t // chunk
    view = q[:, : n_chunks * chunk].reshape(b, n_chunks, chunk, heads_kv, group, d)
    acc = np.zeros((b, n_chunks, heads_kv, d), dtype=np.float32)
    for i in range(chunk):
        for h in range(group):
            acc = acc + view[:, :, i, :, h, :]
    return acc / np.float32(chunk * group)


def bucket_centroids(keys: np.ndarray, members: np.ndarray, mode: str = "mean") -> np.ndarray:
    """Bucket centroids from member keys, fp32.

    ``mean``: the bucket-mean key (the benchmark workloads). ``normalized``: the L2-normalized
    sum (reference pipeline.py:108-115, :396-403, F.normalize eps 1e-12). ``sum``: the
    plain sum (the hierarchy's key sums, pipeline.py:162-164). Canonical
    order: fp32 sum over member slots in table order; the norm is
    ``fp32(sqrt(sum_d fp64(s_d)^2))`` with the fp64 squares summed in dim order.
    keys [T, D], members [rows, cap] -> [rows, D].
    """
    keys = np.asarray(keys, dtype=np.float32)
    members = np.asarray(members)
    rows, cap = members.shape
    acc = np.zeros((rows, keys.shape[1]), dtype=np.float32)
    count = np.zeros(rows, dtype=np.int64)
    for j in range(cap):
        m = members[:, j]
        ok = m >= 0
        acc[ok] = acc[ok] + keys[m[ok]]
        count += ok
    if mode == "mean":
        return np.where(count[:, None] > 0, acc / np.maximum(count, 1).astype(np.float32)[:, None],
                        np.float32(0)).astype(np.float32)
    if mode == "sum":
        return acc
    if mode != "normalized":
        raise ValueError(f"centroid mode must be mean|normalized|sum, got {mode!r}")
    sq = np.zeros(rows, dtype=np.float64)
    for d in range(acc.shape[1]):
        sq = sq + acc[:, d].astype(np.float64) * acc[:, d].astype(np.float64)
    norm = np.sqrt(sq).astype(np.float32)
    return (acc / np.maximum(norm, np.float32(1e-12))[:, None]).astype(np.float32)


def position_members(blocks: int, cluster_block_size: int, bucket_size: int, bucket_cap: int) -> np.ndarray:
    """Positional buckets' member table: runs of ``bucket_size`` consecutive positions,
    -1 padded to the cap (reference pipeline.py:378-395)."""
    rows = blocks * (cluster_block_size // bucket_size)
    members = np.full((rows, bucket_cap), -1, dtype=np.int32)
    members[:, :bucket_size] = np.arange(rows * bucket_size, dtype=np.int32).reshape(rows, bucket_size)
    return members


WARD_LANES = 64  # partials of a segment-pair cost (one per lane of a 64-wide wave)


def ward_pool_sums(keys: np.ndarray, pool: int) -> tuple[np.ndarray, np.ndarray]:
    """Pools of ``pool`` consecutive positions (the last one shorter): fp64 key sums, the
    positions of a pool added in order, and the pool sizes. keys [T, D] -> ([P, D], [P]).

    The first step of the contiguous bucket build (the index build the reference runs as
    build_buckets_gpu, pipeline.py:71-116, which also pools keys before merging, :91-93)."""
    keys = np.asarray(keys, dtype=np.float32)
    T, D = keys.shape
    npool = -(-T // pool)
    sums = np.zeros((npool, D), dtype=np.float64)
    sizes = np.array([min(pool, T - i * pool) for i in range(npool)], dtype=np.int64)
    for j in range(pool):
        rows = np.arange(npool) * pool + j
        ok = rows < T
        sums[ok] = sums[ok] + keys[rows[ok]].astype(np.float64)
    return sums, sizes


def ward_pair_cost(sa: np.ndarray, sb: np.ndarray, na: int, nb: int, max_size: int) -> float:
    """Ward cost of merging adjacent segments with key sums ``sa``/``sb`` and sizes
    ``na``/``nb``: n_a n_b / (n_a + n_b) * |sa / n_a - sb / n_b|^2 (the merge criterion
    the reference's bucket build uses, pipeline.py:95-96), +inf past ``max_size``.

    Canonical fp64 order, no fused multiply-add: squared differences fold into 64
    partials (partial l = sum_k sq[l + 64 k], k ascending), then halve 32, 16, .., 1."""
    if na + nb > max_size:
        return float("inf")
    fa, fb = float(na), float(nb)
    diff = np.asarray(sa, dtype=np.float64) / fa - np.asarray(sb, dtype=np.float64) / fb
    sq = diff * diff
    part = np.zeros(WARD_LANES, dtype=np.float64)
    for k in range(0, sq.shape[0], WARD_LANES):
        chunk = sq[k:k + WARD_LANES]
        part[:chunk.shape[0]] = part[:chunk.shape[0]] + chunk
    h = WARD_LANES // 2
    while h >= 1:
        part[:h] = part[:h] + part[h:2 * h]
        h //= 2
    w = (fa * fb) / (fa + fb)
    return float(w * part[0])


def ward_segments_keys(keys: np.ndarray, pool: int, target: int, max_size: int) -> np.ndarray:
    """Contiguous Ward-style buckets from the keys of one table: pools of ``pool``
    positions, then the adjacent pair with the smallest ``ward_pair_cost`` merged (ties to
    the leftmost pair; pairs past ``max_size`` never merge) until ``target`` segments
    remain. keys [T, D] -> segment start positions [target + 1] (last = T).

    Raises ValueError when no pair can merge before ``target`` is reached."""
    sums, sizes = ward_pool_sums(keys, pool)
    npool = sums.shape[0]
    if target > npool:
        raise ValueError(f"target {target} exceeds the {npool} pools")
    size = sizes.copy()
    nxt = np.arange(1, npool + 1)
    nxt[-1] = -1
    prv = np.arange(-1, npool - 1)
    cost = np.full(npool, np.inf)
    for i in range(npool - 1):
        cost[i] = ward_pair_cost(sums[i], sums[i + 1], int(size[i]), int(size[i + 1]), max_size)
    alive = npool
    while alive > target:
        i = int(np.argmin(cost))  # first minimum: the leftmost pair
        if not cost[i] < np.inf:
            raise ValueError(f"no pair merges under max_size {max_size} with {alive} segments left")
        j = int(nxt[i])
        sums[i] = sums[i] + sums[j]
        size[i] += size[j]
        nxt[i] = nxt[j]
        if nxt[j] >= 0:
            prv[nxt[j]] = i
        cost[j] = np.inf
        if prv[i] >= 0:
            a = int(prv[i])
            cost[a] = ward_pair_cost(sums[a], sums[i], int(size[a]), int(size[i]), max_size)
        cost[i] = (ward_pair_cost(sums[i], sums[nxt[i]], int(size[i]), int(size[nxt[i]]), max_size)
                   if nxt[i] >= 0 else np.inf)
        alive -= 1
    starts = np.empty(target + 1, dtype=np.int64)
    p = 0
    for r in range(target):
        starts[r] = p * pool
        p = int(nxt[p])
    starts[target] = keys.shape[0]
    return starts


# --------------------------------------------------------------------------- selection


def flat_select_row_keys(query: np.ndarray, centroids: np.ndarray, visible: int, top_p: int,
                         mode: str) -> np.ndarray:
    """One row's best-first keys over its visible columns (pipeline.py:248-268)."""
    scores = canonical_scores(query[None, :], centroids, mode)
    return best_first_keys(pack_keys(scores, np.array([visible])), top_p)[0]


def flat_select(index_queries: np.ndarray, positions: np.ndarray, centroids: np.ndarray,
                members: np.ndarray, *, cluster_block_size: int, block_buckets: int, top_p: int,
                top_k: int, window: int, sink: int, mode: str = "bf16",
                ends: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Flat select for one bucket table (reference pipeline.py:248-271 / :274-316).

    index_queries [R, D], positions [R], centroids [rows, D], members [rows, cap]
    -> lists [R, top_k+window+sink], lengths [R].
    """
    rows = centroids.shape[0]
    counts = visible_counts(positions, rows, cluster_block_size, block_buckets, ends)
    scores = canonical_scores(index_queries, centroids, mode)
    ordered = best_first_keys(pack_keys(scores, np.maximum(counts, 0)), top_p)
    return expand_in_order(unpack_ids(ordered), members, positions, window, sink, top_k)


def tree_growth(visible: int, node_block: int, n_nodes: int, node_size: int) -> tuple[int, int]:
    """(covered buckets, made nodes) of a one-level tree for a row seeing ``visible``
    buckets (reference _tree.py:100-142 ``_growth_replay`` with top_level 1: every page end
    covers the whole ``node_cluster_block_size`` blocks of closed buckets not yet covered
    and makes ``block / node_bucket_size`` nodes of each; the page's end is the row's
    visible count, _tree.py:76-80). Capped by the nodes the table holds."""
    covered = min(max(visible, 0) // node_block * node_block, n_nodes * node_size)
    return covered, covered // node_size


def tree_select_row(query: np.ndarray, node_centroids: np.ndarray, children: np.ndarray,
                    bucket_centroids_: np.ndarray, members: np.ndarray, position: int, visible: int,
                    node_block: int, beam_width: int, top_p: int, top_k: int, window: int, sink: int,
                    mode: str = "fp32") -> tuple[np.ndarray, int, np.ndarray]:
    """Two-level beam for one (row, table) (reference _tree.py:318-373 ``_beam_pick_rows``
    with one node level, the growth of ``tree_growth``).

    Level 1: the made nodes [0, made) are the candidates (the start level whole,
    _tree.py:344-346); keep the best ``beam_width`` by score, a tie to the lower node
    (the stable descending argsort over ascending candidates, :350-351). Level 0: the
    kept nodes' children plus the fresh buckets ``[covered, visible)`` (:359-361), each
    bucket once (first-occurrence dedup, :306-315), children at or past ``visible``
    dropped (growth only makes nodes over closed buckets), the best ``top_p`` by score
    (tie -> lower bucket), -1 padded; then the flat expansion. Returns (list, length,
    picks).
    """
    n_nodes = node_centroids.shape[0]
    visible = max(int(visible), 0)
    covered, made = tree_growth(visible, node_block, n_nodes, children.shape[1])
    node_scores = canonical_scores(query[None, :], node_centroids, mode)
    nodes = unpack_ids(best_first_keys(pack_keys(node_scores, np.array([made])), beam_width))[0]
    kids = children[nodes[nodes >= 0]].reshape(-1)
    fresh = np.arange(covered, max(covered, visible))
    kids = kids[(kids >= 0) & (kids < visible)]
    cand = np.unique(np.concatenate([kids, fresh]).astype(np.int64))
    picks = np.full(top_p, -1, dtype=np.int32)
    if cand.size:
        scores = canonical_scores(query[None, :], bucket_centroids_[cand], mode)[0]
        keys = (ordered_bits(scores).astype(np.int64) << np.int64(32)) | (COL_TOP - cand)
        best = np.sort(keys)[::-1][:top_p]
        picks[: best.size] = unpack_ids(best)
    lst, length = expand_row(picks, members, position, window, sink, top_k)
    return lst, length, picks


def beam_growth(visible: int, n_levels: int, node_size: int, node_block: int, top_level: int,
                n_nodes: list[int] | None = None) -> tuple[int, list[int], list[int]]:
    """(covered buckets, made nodes per level, closed nodes per level) of a multi-level tree
    for a row seeing ``visible`` buckets (reference _tree.py:100-142 ``_growth_replay``,
    page end = the row's visible count): whole ``node_block`` blocks of buckets are covered
    and make ``node_block / node_size`` level-1 nodes each; a level's nodes close in whole
    blocks of ``node_block`` and make ``node_block / node_size`` nodes of the level above
    each, up to ``top_level`` levels (and the ``n_levels`` a tree holds). ``n_nodes`` caps
    each level at the nodes the table holds. Closed form of the replay (every page end
    covers all whole blocks not yet covered and closes all whole blocks of open nodes)."""
    levels = min(int(n_levels), int(top_level))
    visible = max(int(visible), 0)
    covered = visible // node_block * node_block
    made, closed = [0] * levels, [0] * levels
    if levels == 0:
        return 0, made, closed
    made[0] = covered // node_size
    if n_nodes is not None and made[0] > n_nodes[0]:
        made[0] = n_nodes[0]
        covered = made[0] * node_size
    for lv in range(1, levels):
        closed[lv - 1] = made[lv - 1] // node_block * node_block
        made[lv] = closed[lv - 1] // node_size
        if n_nodes is not None and made[lv] > n_nodes[lv]:
            made[lv] = n_nodes[lv]
            closed[lv - 1] = made[lv] * node_size
    return covered, made, closed


def build_hierarchy(bucket_key_sums: np.ndarray, node_size: int, node_block: int,
                    top_level: int) -> list[tuple[np.ndarray, np.ndarray, np.ndarray]]:
    """Node levels over one table's bucket key sums [rows, D] (reference pipeline.py:153-178
    ``build_hierarchy_gpu``): while the level below holds a full ``node_block`` block and
    fewer than ``top_level`` levels exist (:166-170), each full block's rows make
    ``node_block / node_size`` nodes; a node's sum is its rows' sums added in child order,
    its centroid the normalized sum (:175-177). A node takes ``node_size`` consecutive rows
    of its block (the reference pairs a block's rows by the Ward cost in an upstream
    Triton kernel that is not vendored). Returns [(centroids, children, sums)] bottom up."""
    sums = np.asarray(bucket_key_sums, dtype=np.float32)
    levels = []
    while sums.shape[0] // node_block and len(levels) < top_level:
        n = sums.shape[0] // node_block * node_block // node_size
        children = np.arange(n * node_size, dtype=np.int32).reshape(n, node_size)
        node_sums = bucket_centroids(sums, children, "sum")
        levels.append((bucket_centroids(sums, children, "normalized"), children, node_sums))
        sums = node_sums
    return levels


def beam_select_row(query: np.ndarray, levels: list[tuple[np.ndarray, np.ndarray]], bucket_centroids_: np.ndarray,
                    members: np.ndarray, position: int, visible: int, node_size: int, node_block: int,
                    top_level: int, beam_width: int, top_p: int, top_k: int, window: int, sink: int,
                    mode: str = "fp32") -> tuple[np.ndarray, int, np.ndarray]:
    """The multi-level beam for one (row, table) (reference _tree.py:318-373 ``_beam_pick_rows``
    with the growth of ``beam_growth``). levels[l] = (centroids [N_l, D], children [N_l,
    node_size]) of the level-(l+1) nodes; children are rows of the level below (buckets for
    l = 0).

    From the highest level holding a made node down to level 1: the candidates are the
    carried children plus the level's open nodes [closed, made) (at the start level: all
    its made nodes, :344-346), each once (first-occurrence dedup, :306-315); the best
    ``beam_width`` by score are kept (a tie to the lower node: the stable descending argsort
    over ascending candidates, :350-351) and their children carried (:353-355). Level 0:
    the carried buckets plus the fresh buckets [covered, visible) (:359-361), each once,
    the best ``top_p`` (tie -> lower bucket), -1 padded; then the flat expansion. Returns
    (list, length, picks)."""
    n_nodes = [lv[0].shape[0] for lv in levels]
    visible = max(int(visible), 0)
    covered, made, closed = beam_growth(visible, len(levels), node_size, node_block, top_level, n_nodes)
    start = sum(1 for m in made if m)
    carried = np.zeros(0, dtype=np.int64)
    for lv in range(start, 0, -1):
        first_open = 0 if lv == start else closed[lv - 1]
        cand = np.unique(np.concatenate([carried, np.arange(first_open, made[lv - 1])]).astype(np.int64))
        cent, children = levels[lv - 1]
        scores = canonical_scores(query[None, :], cent[cand], mode)[0]
        keys = (ordered_bits(scores).astype(np.int64) << np.int64(32)) | (COL_TOP - cand)
        kept = unpack_ids(np.sort(keys)[::-1][:beam_width]).astype(np.int64)
        carried = children[kept].reshape(-1).astype(np.int64)
    fresh = np.arange(covered, max(covered, visible))
    carried = carried[(carried >= 0) & (carried < visible)]
    cand = np.unique(np.concatenate([carried, fresh]).astype(np.int64))
    picks = np.full(top_p, -1, dtype=np.int32)
    if cand.size:
        scores = canonical_scores(query[None, :], bucket_centroids_[cand], mode)[0]
        keys = (ordered_bits(scores).astype(np.int64) << np.int64(32)) | (COL_TOP - cand)
        best = np.sort(keys)[::-1][:top_p]
        picks[: best.size] = unpack_ids(best)
    lst, length = expand_row(picks, members, position, window, sink, top_k)
    return lst, length, picks


# --------------------------------------------------------------------------- reading


def sparse_read(q: np.ndarray, k: np.ndarray, v: np.ndarray, ids: np.ndarray, lengths: np.ndarray,
                scale: float | None = None, empty: str = "zero") -> np.ndarray:
    """Attention over each row's read list (reference read_kernel_tiled.py:30-89, :121;
    v1 read_kernel.py:26-77).

    q [B,Tq,Hq,D], k/v [B,Tk,Hkv,D]; ids [B,Tq,W] shared by every head or
    [B,Tq,Hkv,W] per kv-head; lengths [B,Tq] or [B,Tq,Hkv]. Query head h reads kv head
    ``h // (Hq/Hkv)``; slots at or past min(length, W) and ids < 0 are skipped;
    duplicates count per occurrence; a row with nothing kept gives 0 (``empty="zero"``,
    the tiled contract) or NaN (``empty="nan"``, the v1 contract). Computed in fp64,
    returned fp32.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k)
    v = np.asarray(v)
    b_, tq, hq, d = q.shape
    hkv = k.shape[2]
    group = hq // hkv
    scale = d ** -0.5 if scale is None else float(scale)
    ids = np.asarray(ids)
    lengths = np.asarray(lengths)
    per_head = ids.ndim == 4
    width = ids.shape[-1]
    out = np.zeros((b_, tq, hq, d), dtype=np.float64)
    for b in range(b_):
        for t in range(tq):
            for g in range(hkv):
                row = ids[b, t, g] if per_head else ids[b, t]
                n = int(lengths[b, t, g] if per_head else lengths[b, t])
                sel = row[: max(0, min(n, width))]
                sel = sel[sel >= 0]
                keys = k[b, sel, g].astype(np.float64)
                vals = v[b, sel, g].astype(np.float64)
                for h in range(g * group, (g + 1) * group):
                    if sel.size == 0:
                        out[b, t, h] = np.nan if empty == "nan" else 0.0
                        continue
                    s = (keys @ q[b, t, h]) * scale
                    p = np.exp(s - s.max())
                    out[b, t, h] = (p @ vals) / p.sum()
    return out.astype(np.float32)


def chunk_row_ids(chunk_ids: np.ndarray, chunk_length: int, row: int, chunk: int) -> np.ndarray:
    """Keys query ``row`` reads in a chunked prefill: its chunk's shared list, then the
    chunk's own causal block ``[chunk_start, row]``."""
    start = (row // chunk) * chunk
    shared = np.asarray(chunk_ids)[: int(chunk_length)]
    return np.concatenate([shared, np.arange(start, row + 1, dtype=np.int32)])


def sparse_read_chunked(q, k, v, chunk_ids, chunk_lengths, chunk: int, scale: float | None = None) -> np.ndarray:
    """Chunked-prefill read: each query row reads its chunk's per-kv-head list plus the
    chunk's causal local block. chunk_ids [B, C, Hkv, W], chunk_lengths [B, C, Hkv].
    Stated as the per-row read over ``chunk_row_ids`` lists."""
    q = np.asarray(q, dtype=np.float32)
    b_, tq, hq, d = q.shape
    hkv = np.asarray(k).shape[2]
    width = np.asarray(chunk_ids).shape[-1] + chunk
    ids = np.full((b_, tq, hkv, width), -1, dtype=np.int32)
    lengths = np.zeros((b_, tq, hkv), dtype=np.int32)
    for b in range(b_):
        for t in range(tq):
            for g in range(hkv):
                row = chunk_row_ids(chunk_ids[b, t // chunk, g], chunk_lengths[b, t // chunk, g], t, chunk)
                ids[b, t, g, : row.size] = row
                lengths[b, t, g] = row.size
    return sparse_read(q, k, v, ids, lengths, scale)
