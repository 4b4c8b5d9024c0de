"""The LSA select+read call surface on MI355X (reference src/lsa_rocm_lab/port/pipeline.py).

Same names, arguments and errors as the reference's composition layer; every stage is
a HIP kernel in liblsa_rocm.so:

* ``visible_counts`` (pipeline.py:184-186), ``_production_scores`` (:217-232),
  ``best_first_keys`` (:189-214), ``flat_select_reference`` (:248-271) - the unfused
  chain: score kernel -> listing pack -> radix top-k -> unpack -> expansion walk;
* ``flat_select`` (:274-316) with the ``LSA_SELECT_IMPL`` switch: ``fused`` is ONE
  kernel from the index queries to the read lists (score + top-k + expansion, split
  over workgroups when there are few rows); ``fused_unpack`` keeps the listing +
  top-k and expands from the keys; ``reference`` is the unfused chain;
* ``tree_select`` (:319-337) over a one- to four-level hierarchy from
  ``build_hierarchy_gpu`` (:153-178), ``lsa_read`` (:373-375), ``position_buckets``
  (:378-403);
* ``dense_read`` (:340-370) stays torch SDPA - it is the dense comparator.

The index grows with the cache: ``extend_buckets`` appends newly closed blocks, and
capacity tables (``reserve_buckets``, allocated once for the longest context) take them
in place (``grow_buckets_``) with no tensor moved and no host sync (a table that cannot be
built is reported by a pinned status word: the next build raises, ``check_build`` syncs).

Paged caches (upstream's paged decode; the reference's expansion kernel maps ids through a
slot table, select_fused.py:147-205): every select, ``flat_decode``/``tree_decode`` and
``lsa_read_chunked`` take ``slot_table`` [n_rows, width] int32 (logical position -> cache
row) and ``slot_rows`` [R] int32 (each query row's table row). The expansion applies the
map once per listed id - the kept ids and the window/sink tail, kept or not by their
logical positions - so the lists hold cache rows and the read gathers them directly; K/V
may then be one pool [1, slots, Hkv, D] shared by every batch row.

Per-kv-head selection (the benchmark geometry) extends the shapes: index queries
[R, G, D] against tables with a leading group axis [G, rows, ...] (one table per
kv-head) or [R, G, rows, ...] (one per sequence and kv-head) give lists [R, G, W] and
lengths [R, G]. ``Buckets.ends`` (optional) carries each bucket's exclusive span end
for tables whose buckets are not the reference's fixed blocks; visibility is then the
buckets ending at or before ``position + 1``.
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from lsa_rocm_lab import _abi
from lsa_rocm_lab.port import keys as keys_mod


@dataclass(frozen=True)
class PortConfig:
    """The design's knobs (reference pipeline.py:32-54), same names and defaults."""

    cluster_block_size: int = 512
    pool_size: int = 4
    bucket_size: int = 8
    bucket_cap: int = 16
    top_p: int = 1024
    top_k: int = 4096
    window_size: int = 512
    sink_size: int = 4
    node_bucket_size: int = 4
    top_level: int = 3
    node_cluster_block_size: int = 64
    beam_width: int = 64
    start_nodes: int | None = None

    @property
    def block_bucket_count(self) -> int:
        return self.cluster_block_size // self.bucket_size


@dataclass
class Buckets:
    """A cache's bucket tables on the GPU (reference pipeline.py:57-68) plus optional
    span ends. Shapes: [rows, ...] (one table), [G, rows, ...] or [R, G, rows, ...]."""

    centroids: torch.Tensor  # [..., rows, index_dim] bf16 - what production scoring reads
    members: torch.Tensor  # [..., rows, bucket_cap] int32, absolute positions, -1 padded
    sizes: torch.Tensor  # [..., rows] int32
    centroids_f32: torch.Tensor | None = None  # [..., rows, index_dim] fp32 - fp32 scoring
    ends: torch.Tensor | None = None  # [..., rows] int32 exclusive span end, nondecreasing
    # True when every row j holds exactly the ids ends[j - 1] .. ends[j] - 1 (ends[-1] = 0),
    # in order (contiguous-segment tables): the fused decode then counts and expands a
    # pick's kept members from the ends alone
    spans: bool = False
    # how the centroids were made ("mean" or "normalized"), when a builder here made them;
    # extend_buckets builds appended rows the same way
    centroid: str | None = None
    # capacity tables (reserve_buckets): rows [0, built_rows) hold buckets, the rest are
    # reserved for blocks that have not closed yet (members -1, size 0, zero centroids,
    # span end INT32_MAX, so no query sees them); None: every row is built
    built_rows: int | None = None
    # True when the ends serve the span expansion only and a bucket is visible once its
    # cluster block has closed (the reference's rule for tables without ends): positional
    # block tables, whose spans end before their block closes
    block_visible: bool = False

    @property
    def rows(self) -> int:
        return self.centroids.shape[-2]


@dataclass
class NodeLevel:
    """One node level over the buckets (reference pipeline.py:119-125)."""

    centroids: torch.Tensor  # [..., N, index_dim] fp32
    children: torch.Tensor  # [..., N, node_bucket_size] bucket rows
    key_sums: torch.Tensor | None = None
    centroids_bf16: torch.Tensor | None = None


@dataclass
class Hierarchy:
    """Node levels over a cache's buckets (reference pipeline.py:128-133)."""

    levels: list[NodeLevel] = field(default_factory=list)
    bucket_key_sums: torch.Tensor | None = None


# ----------------------------------------------------------------------------- helpers


def _on_device(what: str, *tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"{what} is a ROCm kernel, got device {t.device}")
        device = t.device
    return device


class _Layout:
    """How query rows and groups map onto a stack of bucket tables."""

    def __init__(self, index_queries: torch.Tensor, table: torch.Tensor):
        if index_queries.dim() == 2:
            self.R, self.D = index_queries.shape
            self.G = 1
            self.grouped = False
        elif index_queries.dim() == 3:
            self.R, self.G, self.D = index_queries.shape
            self.grouped = True
        else:
            raise ValueError(f"index queries must be [R, d] or [R, G, D], got {tuple(index_queries.shape)}")
        lead = table.dim() - 2
        if lead == 0:
            self.row_tables, self.group_tables = 0, 0
        elif lead == 1:
            if table.shape[0] != self.G:
                raise ValueError(f"{table.shape[0]} tables for {self.G} groups")
            self.row_tables, self.group_tables = 0, 1
        elif lead == 2:
            if tuple(table.shape[:2]) != (self.R, self.G):
                raise ValueError(f"tables {tuple(table.shape[:2])} for rows x groups {(self.R, self.G)}")
            self.row_tables, self.group_tables = self.G, 1
        else:
            raise ValueError(f"bucket tables must have at most two leading axes, got {tuple(table.shape)}")
        self.rows = table.shape[-2]

    def out_shape(self, *tail: int) -> tuple[int, ...]:
        return (self.R, self.G, *tail) if self.grouped else (self.R, *tail)


def _positions32(positions: torch.Tensor, device) -> torch.Tensor:
    p = positions.to(device=device)
    return (p if p.dtype == torch.int32 else p.to(torch.int32)).contiguous()


def _score_table(buckets: Buckets, score_dtype: str) -> tuple[torch.Tensor, int]:
    if score_dtype == "fp32":
        if buckets.centroids_f32 is None:
            raise ValueError("fp32 scoring needs buckets.centroids_f32")
        return buckets.centroids_f32.float().contiguous(), _abi.SCORE_F32
    if score_dtype != "bf16":
        raise ValueError(f"score_dtype must be bf16|fp32, got {score_dtype!r}")
    return buckets.centroids.to(torch.bfloat16).contiguous(), _abi.SCORE_BF16


def _ends(buckets: Buckets) -> torch.Tensor | None:
    return None if buckets.ends is None else buckets.ends.to(torch.int32).contiguous()


def _table_flags(buckets: Buckets, ends: torch.Tensor | None) -> int:
    """The C ABI's table flags of a bucket table: span expansion, block visibility."""
    if ends is None:
        return 0
    return (_abi.TABLE_SPANS if buckets.spans else 0) | (_abi.TABLE_BLOCK_VISIBLE if buckets.block_visible else 0)


def visible_ends(buckets: Buckets) -> torch.Tensor | None:
    """The span ends that decide which buckets a position sees, or None when the
    closed-block rule decides (tables without ends, and block-visible tables)."""
    return None if buckets.block_visible else buckets.ends


def _queries(index_queries: torch.Tensor) -> torch.Tensor:
    if index_queries.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        index_queries = index_queries.float()
    return index_queries.contiguous()


_ROW_INDEX: dict[tuple, torch.Tensor] = {}


def _row_index(device, R: int, shared: bool) -> torch.Tensor:
    """The default slot rows of R query rows - all 0 (one table row) or 0..R-1 - made once
    per device and size and never written, so a call (or a captured graph) adds no fill."""
    key = (_abi.device_index(device), R, shared)
    t = _ROW_INDEX.get(key)
    if t is None:
        t = (torch.zeros(R, dtype=torch.int32, device=device) if shared
             else torch.arange(R, dtype=torch.int32, device=device))
        _ROW_INDEX[key] = t
    return t


def _slot_args(slot_table: torch.Tensor | None, slot_rows: torch.Tensor | None, R: int, device):
    """A paged cache's slot map for one call: (``const lsa_slot_map*`` or None, the tensors
    it points at, kept alive by the caller until the launch). ``slot_table`` [n_rows, width]
    (or [width]) maps logical positions to cache rows; ``slot_rows`` [R] names each query
    row's table row (default: row 0 for a one-row table, row r for a table of R rows)."""
    if slot_table is None:
        if slot_rows is not None:
            raise ValueError("slot_rows without a slot_table")
        return None, ()
    _on_device("the slot map", slot_table)
    table = slot_table.to(device=device, dtype=torch.int32)
    if table.dim() == 1:
        table = table[None]
    if table.dim() != 2 or table.shape[0] < 1 or table.shape[1] < 1:
        raise ValueError(f"slot_table must be [n_rows, width] with both >= 1, got {tuple(slot_table.shape)}")
    if table.stride(1) != 1:
        table = table.contiguous()
    if slot_rows is None:
        if table.shape[0] == 1:
            rows = _row_index(device, R, shared=True)
        elif table.shape[0] == R:
            rows = _row_index(device, R, shared=False)
        else:
            raise ValueError(f"slot_rows is needed: {table.shape[0]} slot-table rows for {R} query rows")
    else:
        rows = slot_rows.to(device=device, dtype=torch.int32).reshape(-1).contiguous()
        if rows.numel() != R:
            raise ValueError(f"slot_rows holds {rows.numel()} rows for {R} query rows")
    return _abi.slot_map(table, rows), (table, rows)


# ----------------------------------------------------------------------------- selection


def visible_counts(positions: torch.Tensor, buckets: Buckets, config: PortConfig,
                   groups: int | None = None) -> torch.Tensor:
    """Buckets each query sees - the closed blocks before its own (reference pipeline.py:184-186).

    With ``buckets.ends`` the buckets whose span ends at or before ``position + 1``.
    Returns [R] int32, or [R, G] for per-group tables.
    """
    device = _on_device("visible_counts", buckets.centroids)
    pos = _positions32(positions, device)
    R = pos.shape[0]
    lead = buckets.centroids.dim() - 2
    G = groups or (buckets.centroids.shape[-3] if lead >= 1 else 1)
    row_tables, group_tables = (0, 0) if lead == 0 else ((0, 1) if lead == 1 else (G, 1))
    counts = torch.empty(R * G, dtype=torch.int32, device=device)
    ends = None if buckets.block_visible else _ends(buckets)
    _abi.call("lsa_visible_counts", pos.data_ptr(), R, G, buckets.rows, config.cluster_block_size,
              config.block_bucket_count, _abi.ptr(ends), row_tables, group_tables, counts.data_ptr(),
              _abi.stream(device))
    return counts.view(R, G) if (lead or G > 1) else counts


def best_first_keys(keys: torch.Tensor, top_p: int, counts: torch.Tensor | None = None) -> torch.Tensor:
    """The best ``top_p`` packed keys per row, best first (reference pipeline.py:189-214).

    A radix select plus bitonic sort per row on the GPU; keys are unique per column, so
    the result is exactly ``torch.sort(keys, descending=True).values[:, :top_p]``.
    ``counts`` masks slots at or past each row's count to EMPTY first.
    """
    _on_device("best_first_keys", keys)
    keys = keys.contiguous()
    rows, width = keys.shape
    k = min(top_p, width)
    out = torch.empty(rows, k, dtype=torch.int64, device=keys.device)
    if rows == 0 or k == 0:
        return out
    cnt = None if counts is None else counts.to(device=keys.device, dtype=torch.int32).reshape(rows).contiguous()
    _abi.call("lsa_topk_keys", keys.data_ptr(), _abi.ptr(cnt), rows, width, k, out.data_ptr(),
              _abi.stream(keys.device))
    return out


def _production_scores(index_queries, positions, buckets, config, score_dtype):
    """The canonical scoring both select implementations share (reference pipeline.py:217-232).

    fp32 scores = the index queries (rounded to bf16 for ``score_dtype="bf16"``) against
    the bf16 centroids (or fp32 against ``centroids_f32``), products and partial sums
    in fp64 in a fixed order, one rounding to fp32.
    """
    if positions.shape[0] != index_queries.shape[0]:
        raise ValueError(
            f"a position a query: {index_queries.shape[0]} queries, {positions.shape[0]} positions"
        )
    device = _on_device("_production_scores", index_queries, buckets.centroids)
    layout = _Layout(index_queries, buckets.centroids)
    table, mode = _score_table(buckets, score_dtype)
    q = _queries(index_queries)
    counts = visible_counts(positions, buckets, config, layout.G)
    scores = torch.empty(layout.out_shape(layout.rows), dtype=torch.float32, device=device)
    _abi.call("lsa_score_rows", q.data_ptr(), _abi.dtype_code(q.dtype), layout.R, layout.G, layout.D,
              table.data_ptr(), layout.rows, layout.row_tables, layout.group_tables, mode, scores.data_ptr(),
              _abi.stream(device))
    return scores, counts


def _mask_for(scores: torch.Tensor, config: PortConfig, listed: torch.Tensor) -> torch.Tensor | None:
    """Listing counts for ``best_first_keys`` - None on the whole path (reference pipeline.py:235-245)."""
    return None if scores.shape[-1] <= keys_mod.WHOLE * config.top_p else listed


def _expand(picks: torch.Tensor, picks_are_keys: bool, layout: _Layout, members: torch.Tensor,
            positions: torch.Tensor, window: int, sink: int, top_k: int, slot_table=None, slot_rows=None):
    device = picks.device
    picks = picks.contiguous()
    members = members.to(device=device, dtype=torch.int32).contiguous()
    P = picks.shape[-1]
    width = top_k + window + sink
    lists = torch.empty(layout.out_shape(width), dtype=torch.int32, device=device)
    lengths = torch.empty(layout.out_shape(), dtype=torch.int32, device=device)
    slots, _keep = _slot_args(slot_table, slot_rows, layout.R, device)
    _abi.call("lsa_expand", picks.data_ptr(), 1 if picks_are_keys else 0, layout.R, layout.G, P,
              members.data_ptr(), members.shape[-2], members.shape[-1], layout.row_tables, layout.group_tables,
              positions.data_ptr(), slots, window, sink, top_k, lists.data_ptr(), lengths.data_ptr(),
              _abi.stream(device))
    return lists, lengths


def flat_select_reference(
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    config: PortConfig,
    top_k: int | None = None,
    score_dtype: str = "bf16",
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The unfused select chain (reference pipeline.py:248-271): scores, the whole-path
    listing, best-first keys, unpack, rank-order expansion - one HIP kernel each.
    ``slot_table`` / ``slot_rows``: a paged cache's slot map (see the module notes)."""
    top_k = config.top_k if top_k is None else top_k
    scores, counts = _production_scores(index_queries, positions, buckets, config, score_dtype)
    layout = _Layout(index_queries, buckets.centroids)
    flat_scores = scores.reshape(-1, layout.rows)
    keys, listed = keys_mod.listed(flat_scores, counts.reshape(-1))
    picked = keys_mod.unpack_ids(best_first_keys(keys, config.top_p, counts=_mask_for(flat_scores, config, listed)))
    pos = _positions32(positions, scores.device)
    return _expand(picked, False, layout, buckets.members, pos, config.window_size, config.sink_size, top_k,
                   slot_table, slot_rows)


def _select_splits(R: int, G: int, rows: int, top_p: int) -> int:
    """Workgroups per (row, group) of the fused select. A CU keeps only so many misses in
    flight, so with few rows the centroid scan is cut into ~32-column slices on separate
    CUs, whose keys the last slice to finish collects; with many rows each workgroup scores
    its whole table. ``LSA_SELECT_SPLITS`` overrides."""
    env = os.environ.get("LSA_SELECT_SPLITS")
    cap = max(1, min(rows, 256))
    if env:
        return max(1, min(int(env), cap))
    units = R * G
    if units >= 256:  # enough rows to fill the GPU: one workgroup per (row, group)
        return 1
    # few rows (decode): ~32 columns per workgroup, so the centroid scan spreads over CUs
    return max(1, min(math.ceil(rows / 32), cap, max(1, 2048 // max(units, 1))))


def _decode_splits(dtype, D: int, group: int, units: int, rows: int, top_p: int, score_mode: int,
                   table_flags: int) -> int:
    """Select workgroups per (row, kv-head) of the fused decode: the splits of the rank form
    (tables that fit it: every split publishes its columns' keys and each reader ranks
    them) or of the exchange form (the last split to arrive ranks the keys and publishes the
    picks), or 0 - the replicated form, where every reader selects for itself - when
    ``LSA_DECODE_MODE=rep`` asks for it (or ``auto`` with at most ``LSA_DECODE_REP_UNITS``
    (row, kv-head) units; 0 by default: at the 32k decode the replicated form's 128 KiB
    centroid scan per reader costs more round trips than the exchange saves)."""
    mode = os.environ.get("LSA_DECODE_MODE", "auto")
    if mode not in ("auto", "rep", "exchange"):
        raise ValueError(f"LSA_DECODE_MODE must be auto|rep|exchange, got {mode!r}")
    ok = bool(_abi.load().lsa_decode_flat_rep_ok(_abi.dtype_code(dtype), D, group, rows, top_p, score_mode,
                                                 table_flags))
    if mode == "rep" and not ok:
        raise ValueError("LSA_DECODE_MODE=rep: the replicated select does not apply to this shape")
    if ok and (mode == "rep" or (mode == "auto" and units <= _REP_MAX_UNITS)):
        return 0
    if os.environ.get("LSA_SELECT_SPLITS") or units >= 256:
        return _select_splits(units, 1, rows, top_p)
    cap = min(rows, 256, max(1, 2048 // max(units, 1)))
    if rows <= _RANK_MAX_ROWS and units * rows <= _RANK_MAX_SLOTS:
        # the rank form (every reader ranks the splits' published keys; no split collects):
        # ~16 columns a split (32k decode, 512 buckets, 24 readers: 18.4 us with 32 splits,
        # 19.0 with 24, 19.1 with 64, 19.7 with 8)
        return max(1, min(math.ceil(rows / 16), cap))
    # the exchange form: ~64 columns a select workgroup (32k decode, 512 buckets: 19.8 us
    # with 8 splits, 20.2 with 16, 21.4 with 4); its last split then collects half as many keys
    return max(1, min(math.ceil(rows / 64), cap))


# The fused decode's rank form serves tables of at most this many buckets, and at most
# this many (row, kv-head, bucket) key slots in all (csrc/decode_dev.h kRankMaxRows,
# kRankMaxSlots); other shapes take the exchange form.
_RANK_MAX_ROWS = 1024
_RANK_MAX_SLOTS = 1 << 16


# (row, kv-head) units up to which the fused decode selects in every reader
_REP_MAX_UNITS = int(os.environ.get("LSA_DECODE_REP_UNITS", "0"))


def _fused_select(index_queries, positions, buckets, config, top_k, score_dtype, slot_table=None, slot_rows=None):
    device = _on_device("flat_select", index_queries, buckets.centroids, buckets.members)
    if positions.shape[0] != index_queries.shape[0]:
        raise ValueError(
            f"a position a query: {index_queries.shape[0]} queries, {positions.shape[0]} positions"
        )
    layout = _Layout(index_queries, buckets.centroids)
    table, mode = _score_table(buckets, score_dtype)
    q = _queries(index_queries)
    members = buckets.members.to(device=device, dtype=torch.int32).contiguous()
    ends = _ends(buckets)
    pos = _positions32(positions, device)
    splits = _select_splits(layout.R, layout.G, layout.rows, config.top_p)
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(layout.out_shape(width), dtype=torch.int32, device=device)
    lengths = torch.empty(layout.out_shape(), dtype=torch.int32, device=device)
    nbytes = _abi.size("lsa_select_flat_scratch_bytes", layout.R, layout.G, config.top_p, layout.rows, splits)
    ws = _abi.Workspace.get(device, "select", nbytes)
    counters = _abi.Counters.get(device, layout.R * layout.G) if nbytes else None
    slots, _keep = _slot_args(slot_table, slot_rows, layout.R, device)
    _abi.call("lsa_select_flat", q.data_ptr(), _abi.dtype_code(q.dtype), layout.R, layout.G, layout.D,
              table.data_ptr(), members.data_ptr(), _abi.ptr(ends),
              _table_flags(buckets, ends), layout.rows, members.shape[-1],
              layout.row_tables, layout.group_tables, mode, pos.data_ptr(), slots, config.cluster_block_size,
              config.block_bucket_count, config.top_p, config.window_size, config.sink_size, top_k, splits,
              _abi.ptr(counters), _abi.ptr(ws), nbytes, lists.data_ptr(), lengths.data_ptr(), _abi.stream(device))
    return lists, lengths


def flat_select(
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    config: PortConfig,
    top_k: int | None = None,
    score_dtype: str = "bf16",
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Select each query's keys - the production composition, implementation-switched.

    ``LSA_SELECT_IMPL`` picks the implementation (default ``reference``):
    ``reference`` is the unfused chain (``flat_select_reference``); ``fused`` is one HIP
    kernel from the index queries to the read lists (canonical score, packed-key top-k,
    rank-order expansion); ``fused_unpack`` keeps the listing and best-first top-k and
    expands from the keys. All three produce byte-identical lists and lengths; unknown
    values fail loudly. ``slot_table`` / ``slot_rows`` (a paged cache) make the lists hold
    cache rows: every listed id goes through the slot table (see the module notes).
    """
    impl = os.environ.get("LSA_SELECT_IMPL", "reference")
    if impl not in ("reference", "fused", "fused_unpack"):
        raise ValueError(
            f"LSA_SELECT_IMPL must be reference|fused|fused_unpack, got {impl!r}"
        )
    if impl == "reference":
        return flat_select_reference(index_queries, positions, buckets, config, top_k, score_dtype, slot_table,
                                     slot_rows)
    top_k = config.top_k if top_k is None else top_k
    if impl == "fused":
        return _fused_select(index_queries, positions, buckets, config, top_k, score_dtype, slot_table, slot_rows)
    if impl == "fused_unpack":
        scores, counts = _production_scores(index_queries, positions, buckets, config, score_dtype)
        layout = _Layout(index_queries, buckets.centroids)
        flat_scores = scores.reshape(-1, layout.rows)
        keys, listed = keys_mod.listed(flat_scores, counts.reshape(-1))
        ordered = best_first_keys(keys, config.top_p, counts=_mask_for(flat_scores, config, listed))
        pos = _positions32(positions, scores.device)
        return _expand(ordered, True, layout, buckets.members, pos, config.window_size, config.sink_size, top_k,
                       slot_table, slot_rows)
    raise AssertionError(f"unreachable impl {impl!r}")


def tree_select(
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    hierarchy: Hierarchy,
    config: PortConfig,
    top_k: int | None = None,
    score_dtype: str = "fp32",
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Select each query's keys by a beam down the node levels (reference pipeline.py:319-337).

    See ``_tree.tree_select_batched``; ``slot_table`` / ``slot_rows`` as ``flat_select``.
    """
    from lsa_rocm_lab.port._tree import tree_select_batched

    return tree_select_batched(index_queries, positions, buckets, hierarchy, config, top_k, score_dtype,
                               slot_table, slot_rows)


# ----------------------------------------------------------------------------- reading


def dense_read(q, k, v, scale):
    """The dense causal baseline - torch SDPA (reference pipeline.py:340-370), the comparator.

    Query rows are the tail ``q_len`` positions of the ``kv_len`` cache: the square case
    keeps the fused causal flag, one row attends the whole cache unmasked, a chunk gets
    an explicit bottom-right-aligned causal mask (never top-left ``is_causal``).
    """
    heads_q, heads_kv = q.shape[2], k.shape[2]
    q_len, kv_len = q.shape[1], k.shape[1]
    if q_len > kv_len:
        raise ValueError(f"query rows {q_len} exceed the cache {kv_len}: no causal read exists")
    queries, keys, values = q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)
    gqa = heads_q != heads_kv
    if q_len == kv_len:
        out = F.scaled_dot_product_attention(queries, keys, values, is_causal=True, scale=scale, enable_gqa=gqa)
    elif q_len == 1:
        out = F.scaled_dot_product_attention(queries, keys, values, scale=scale, enable_gqa=gqa)
    else:
        causal = torch.arange(kv_len, device=q.device)[None, :] <= torch.arange(
            kv_len - q_len, kv_len, device=q.device
        )[:, None]
        out = F.scaled_dot_product_attention(
            queries, keys, values, attn_mask=causal, scale=scale, enable_gqa=gqa
        )
    return out.permute(0, 2, 1, 3)


def lsa_read(q, k, v, read_lists, lengths, scale):
    """The sparse read over selected lists (reference pipeline.py:373-375)."""
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    return sparse_read_auto(q, k, v, read_lists, lengths, scale)


def flat_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    config: PortConfig,
    scale: float | None = None,
    top_k: int | None = None,
    score_dtype: str = "bf16",
    splits: int | None = None,
    readers: int | None = None,
    status: torch.Tensor | None = None,
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode step - index queries, flat select, sparse read - in one HIP launch.

    The reference's decode step (port/bench.py:147-153) is ``flat_select`` on the GQA
    group-mean index queries followed by ``lsa_read``; this is that composition fused.
    q [B, 1, Hq, D] (the token being decoded, at ``positions[b]``), k/v [B, Tk, Hkv, D],
    bucket tables per kv-head ([Hkv, rows, ...]) or per row and kv-head. Returns
    ``(out [B, 1, Hq, D], lists [B, Hkv, W], lengths [B, Hkv])``; lists and lengths are
    byte-identical to ``flat_select(index_queries(q, Hkv)[:, 0], ...)``'s. ``splits``: select
    workgroups per (row, kv-head) (default as ``flat_select``); ``readers``: reader
    workgroups per (row, kv-head) (default: ``LSA_DECODE_READERS`` or the library's
    choice). ``status``: an int32 [1] tensor (device or pinned host) that a launch sets to
    1 when a reader gives up waiting for its unit's selection; by default the library's
    pinned word, checked at the start of every call without a device sync: if an earlier
    launch gave up, the arrival counters are zeroed again and ``LsaError`` is raised
    (``check_decode`` makes the same check after a sync); a caller that passes its own
    ``status`` checks it and, when it is set, calls ``reset_decode`` before the next launch.
    ``slot_table`` / ``slot_rows`` (a paged cache; rows default to the batch row): the
    lists hold cache rows and K/V may be one pool [1, slots, Hkv, D] for every batch row.
    """
    from lsa_rocm_lab.port.read_kernel_tiled import _kv_layout

    device = _on_device("flat_decode", q, k, v, buckets.centroids, buckets.members)
    if q.dim() != 4 or q.shape[1] != 1:
        raise ValueError(f"flat_decode takes one query token per batch row: q [B, 1, Hq, D], got {tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    B, _, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    if k.dim() != 4 or k.shape != v.shape or k.shape[0] not in (B, 1) or k.shape[3] != D:
        raise ValueError(f"k/v must be [B={B} or 1, Tk, Hkv, D={D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads do not group onto {Hkv} kv-heads")
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool read by every batch row
        sb = 0
    layout = _Layout(torch.empty((B, Hkv, D), device="meta"), buckets.centroids)
    table, mode = _score_table(buckets, score_dtype)
    members = buckets.members.to(device=device, dtype=torch.int32).contiguous()
    ends = _ends(buckets)
    flags = _table_flags(buckets, ends)
    pos = _positions32(positions, device)
    if pos.numel() != B:
        raise ValueError(f"a position a batch row: {B} rows, {pos.numel()} positions")
    top_k = config.top_k if top_k is None else top_k
    scale = D ** -0.5 if scale is None else scale
    if splits is None:
        splits = _decode_splits(q.dtype, D, Hq // Hkv, B * Hkv, layout.rows, config.top_p, mode, flags)
    rows, cap = layout.rows, members.shape[-1]
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(B, Hkv, width, dtype=torch.int32, device=device)
    lengths = torch.empty(B, Hkv, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    dt = _abi.dtype_code(q.dtype)
    readers = int(os.environ.get("LSA_DECODE_READERS", "0")) if readers is None else readers
    n_counters = _abi.size("lsa_decode_flat_counters", B, Hkv, rows, config.top_p)
    nbytes = _abi.size("lsa_decode_flat_scratch_bytes", dt, B, Hq, Hkv, D, rows, config.top_p,
                       config.window_size, config.sink_size, splits, readers)
    if status is None:
        status = _abi.StatusWord.get(device)
        if int(status[0]) != 0:
            _decode_gave_up(device, status)
    ws = _abi.Workspace.get(device, "decode", nbytes)
    counters = _abi.Counters.get(device, max(n_counters, 1))
    slots, _keep = _slot_args(slot_table, slot_rows, B, device)
    _abi.call("lsa_decode_flat", q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, Tk, Hq, Hkv, D, sb, st, sh,
              table.data_ptr(), members.data_ptr(), _abi.ptr(ends), flags, rows, cap, layout.row_tables,
              layout.group_tables, mode, pos.data_ptr(), slots, config.cluster_block_size, config.block_bucket_count,
              config.top_p, config.window_size, config.sink_size, top_k, float(scale), splits, readers,
              counters.data_ptr(), counters.numel(), _abi.ptr(ws), nbytes, lists.data_ptr(), lengths.data_ptr(),
              out.data_ptr(), _abi.ptr(status), _abi.stream(device))
    return out, lists, lengths


def flat_decode_shared(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    config: PortConfig,
    scale: float | None = None,
    top_k: int | None = None,
    score_dtype: str = "bf16",
    splits: int | None = None,
    readers: int | None = None,
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode step over the reference's own layout in one HIP launch: one index-space
    selection a batch row, shared by every head (the reference's decode step, port/bench.py:
    147-153: ``flat_select`` on the index queries, then ``lsa_read`` over lists shared by
    the heads), at any of its knobs up to 4096 buckets and 1024 picks (its defaults:
    top_p 1024, top_k 4096, window 512, sink 4).

    q [B, 1, Hq, D] (bf16 / fp16, D 64 or 128), k/v [B or 1, Tk, Hkv, D], index_queries
    [B, d] fp32 (``make_index_space``'s queries for the decoded token), one span table for
    every row ([rows, ...]) or one a row ([B, rows, ...]). Returns ``(out [B, 1, Hq, D],
    lists [B, W], lengths [B])``; lists and lengths are byte-identical to
    ``flat_select(index_queries, positions, buckets, config)``'s (any LSA_SELECT_IMPL) and
    out is the read of those lists. ``splits`` / ``readers``: select workgroups a row and
    reader workgroups a (row, kv-head) (default: the library's). Slot map as ``flat_decode``."""
    from lsa_rocm_lab.port.read_kernel_tiled import _kv_layout

    device = _on_device("flat_decode_shared", q, k, v, index_queries, buckets.centroids)
    if q.dim() != 4 or q.shape[1] != 1:
        raise ValueError(f"flat_decode_shared takes one query token per batch row: q [B, 1, Hq, D], got "
                         f"{tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    B, _, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    if k.dim() != 4 or k.shape != v.shape or k.shape[0] not in (B, 1) or k.shape[3] != D:
        raise ValueError(f"k/v must be [B={B} or 1, Tk, Hkv, D={D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads do not group onto {Hkv} kv-heads")
    if buckets.ends is None or not buckets.spans:
        raise ValueError("flat_decode_shared expands picks from span ends: the tables need ends and spans")
    idx = index_queries.reshape(B, -1).to(device=device, dtype=torch.float32).contiguous()
    cent = buckets.centroids
    if cent.dim() == 2:
        row_tables = 0
    elif cent.dim() == 3 and cent.shape[0] == B:
        row_tables = 1
    else:
        raise ValueError(f"one bucket table for every row [rows, d] or one a row [B, rows, d], got "
                         f"{tuple(cent.shape)}")
    if idx.shape[1] != cent.shape[-1] or idx.shape[1] != D:
        raise ValueError(f"index queries of dim {idx.shape[1]} for centroids of dim {cent.shape[-1]}: both must be "
                         f"the head dim {D}")
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool read by every batch row
        sb = 0
    table, mode = _score_table(buckets, score_dtype)
    ends = _ends(buckets)
    flags = _table_flags(buckets, ends)
    pos = _positions32(positions, device)
    if pos.numel() != B:
        raise ValueError(f"a position a batch row: {B} rows, {pos.numel()} positions")
    top_k = config.top_k if top_k is None else top_k
    scale = D ** -0.5 if scale is None else scale
    rows = buckets.rows
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(B, width, dtype=torch.int32, device=device)
    lengths = torch.empty(B, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    dt = _abi.dtype_code(q.dtype)
    readers = int(os.environ.get("LSA_DECODE_READERS", "0")) if readers is None else readers
    splits = int(os.environ.get("LSA_SELECT_SPLITS", "0")) if splits is None else splits
    n_counters = _abi.size("lsa_decode_shared_counters", B, Hkv, rows)
    nbytes = _abi.size("lsa_decode_shared_scratch_bytes", dt, B, Hq, Hkv, D, rows, config.top_p, config.window_size,
                       config.sink_size, top_k, readers)
    status = _abi.StatusWord.get(device)
    if int(status[0]) != 0:
        _decode_gave_up(device, status)
    ws = _abi.Workspace.get(device, "decode_shared", nbytes)
    counters = _abi.Counters.get(device, max(n_counters, 1))
    slots, _keep = _slot_args(slot_table, slot_rows, B, device)
    _abi.call("lsa_decode_shared", q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, Tk, Hq, Hkv, D, sb, st, sh,
              idx.data_ptr(), table.data_ptr(), ends.data_ptr(), flags, rows, row_tables, mode, pos.data_ptr(),
              slots, config.cluster_block_size, config.block_bucket_count, config.top_p, config.window_size,
              config.sink_size, top_k, float(scale), splits, readers, counters.data_ptr(), counters.numel(),
              _abi.ptr(ws), nbytes, lists.data_ptr(), lengths.data_ptr(), out.data_ptr(), _abi.ptr(status),
              _abi.stream(device))
    return out, lists, lengths


def tree_decode_shared(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    hierarchy: Hierarchy,
    config: PortConfig,
    scale: float | None = None,
    top_k: int | None = None,
    score_dtype: str = "fp32",
    splits: int | None = None,
    readers: int | None = None,
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The tree arm of the reference's decode step in one HIP launch: one multi-level beam
    selection a batch row over the index-space hierarchy, shared by every head (port/bench.py:
    147-153 with ``tree_select``, pipeline.py:319-337, then ``lsa_read``), at any of its
    knobs up to 8192 buckets / nodes a level and 1024 picks (its defaults: node size 4,
    node blocks of 64, 3 levels, beam 64, top_p 1024, top_k 4096, window 512, sink 4).

    Shapes as ``flat_decode_shared``; ``hierarchy`` as ``tree_select``'s (its levels' tables
    one for every row or one a row, like the buckets'). Returns ``(out [B, 1, Hq, D], lists
    [B, W], lengths [B])``; lists and lengths are byte-identical to ``tree_select(
    index_queries, positions, buckets, hierarchy, config, score_dtype=score_dtype)``'s."""
    from lsa_rocm_lab.port.read_kernel_tiled import _kv_layout

    device = _on_device("tree_decode_shared", q, k, v, index_queries, buckets.centroids,
                        *[level.centroids for level in hierarchy.levels])
    if q.dim() != 4 or q.shape[1] != 1:
        raise ValueError(f"tree_decode_shared takes one query token per batch row: q [B, 1, Hq, D], got "
                         f"{tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    B, _, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    if k.dim() != 4 or k.shape != v.shape or k.shape[0] not in (B, 1) or k.shape[3] != D:
        raise ValueError(f"k/v must be [B={B} or 1, Tk, Hkv, D={D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads do not group onto {Hkv} kv-heads")
    if buckets.ends is None or not buckets.spans:
        raise ValueError("tree_decode_shared expands picks from span ends: the tables need ends and spans")
    n_levels = len(hierarchy.levels)
    if not 1 <= n_levels <= _abi.BEAM_MAX_LEVELS:
        raise NotImplementedError(f"tree_decode_shared covers 1 to {_abi.BEAM_MAX_LEVELS} node levels, got {n_levels}")
    if config.start_nodes is not None:
        raise NotImplementedError("tree_decode_shared covers start_nodes=None (the top level down)")
    idx = index_queries.reshape(B, -1).to(device=device, dtype=torch.float32).contiguous()
    cent = buckets.centroids
    if cent.dim() == 2:
        row_tables = 0
    elif cent.dim() == 3 and cent.shape[0] == B:
        row_tables = 1
    else:
        raise ValueError(f"one bucket table for every row [rows, d] or one a row [B, rows, d], got "
                         f"{tuple(cent.shape)}")
    if idx.shape[1] != cent.shape[-1] or idx.shape[1] != D:
        raise ValueError(f"index queries of dim {idx.shape[1]} for centroids of dim {cent.shape[-1]}: both must be "
                         f"the head dim {D}")
    for level in hierarchy.levels:
        if level.centroids.dim() != cent.dim() or level.centroids.shape[:-2] != cent.shape[:-2]:
            raise ValueError("node and bucket tables must share the same leading axes")
    if score_dtype == "fp32":
        if buckets.centroids_f32 is None:
            raise ValueError("fp32 scoring needs buckets.centroids_f32")
        ncents = [level.centroids.float() for level in hierarchy.levels]
        bcent, mode = buckets.centroids_f32.float(), _abi.SCORE_F32
    elif score_dtype == "bf16":
        ncents = [level.centroids_bf16 if level.centroids_bf16 is not None else level.centroids.to(torch.bfloat16)
                  for level in hierarchy.levels]
        bcent, mode = buckets.centroids.to(torch.bfloat16), _abi.SCORE_BF16
    else:
        raise ValueError(f"score_dtype must be bf16|fp32, got {score_dtype!r}")
    ncents = [c.contiguous() for c in ncents]
    bcent = bcent.contiguous()
    kids = [level.children.to(device=device, dtype=torch.int32).contiguous() for level in hierarchy.levels]
    node_size = kids[0].shape[-1]
    if any(kk.shape[-1] != node_size for kk in kids):
        raise ValueError("every node level must hold node_bucket_size children a node")
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool read by every batch row
        sb = 0
    ends = _ends(buckets)
    flags = _table_flags(buckets, ends)
    pos = _positions32(positions, device)
    if pos.numel() != B:
        raise ValueError(f"a position a batch row: {B} rows, {pos.numel()} positions")
    top_k = config.top_k if top_k is None else top_k
    scale = D ** -0.5 if scale is None else scale
    rows = buckets.rows
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(B, width, dtype=torch.int32, device=device)
    lengths = torch.empty(B, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    dt = _abi.dtype_code(q.dtype)
    readers = int(os.environ.get("LSA_DECODE_READERS", "0")) if readers is None else readers
    splits = int(os.environ.get("LSA_SELECT_SPLITS", "0")) if splits is None else splits
    cent_ptrs = (ctypes.c_void_p * n_levels)(*[c.data_ptr() for c in ncents])
    kid_ptrs = (ctypes.c_void_p * n_levels)(*[kk.data_ptr() for kk in kids])
    n_nodes = (ctypes.c_int32 * n_levels)(*[kk.shape[-2] for kk in kids])
    levels = min(n_levels, config.top_level)
    n_counters = _abi.size("lsa_decode_tree_shared_counters", B, Hkv, levels, ctypes.addressof(n_nodes), rows)
    nbytes = _abi.size("lsa_decode_shared_scratch_bytes", dt, B, Hq, Hkv, D, rows, config.top_p, config.window_size,
                       config.sink_size, top_k, readers)
    status = _abi.StatusWord.get(device)
    if int(status[0]) != 0:
        _decode_gave_up(device, status)
    ws = _abi.Workspace.get(device, "decode_shared", nbytes)
    counters = _abi.Counters.get(device, max(n_counters, 1))
    slots, _keep = _slot_args(slot_table, slot_rows, B, device)
    _abi.call("lsa_decode_tree_shared", q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, Tk, Hq, Hkv, D, sb, st, sh,
              idx.data_ptr(), n_levels, ctypes.addressof(cent_ptrs), ctypes.addressof(kid_ptrs),
              ctypes.addressof(n_nodes), node_size, config.node_cluster_block_size, config.top_level,
              bcent.data_ptr(), ends.data_ptr(), flags, rows, row_tables, mode, pos.data_ptr(), slots,
              config.cluster_block_size, config.block_bucket_count, config.beam_width, config.top_p,
              config.window_size, config.sink_size, top_k, float(scale), splits, readers, counters.data_ptr(),
              counters.numel(), _abi.ptr(ws), nbytes, lists.data_ptr(), lengths.data_ptr(), out.data_ptr(),
              _abi.ptr(status), _abi.stream(device))
    return out, lists, lengths


def tree_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    hierarchy: Hierarchy,
    config: PortConfig,
    scale: float | None = None,
    top_k: int | None = None,
    score_dtype: str = "bf16",
    readers: int | None = None,
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One decode step over a one-level node tree - index queries, tree select, sparse
    read - in one HIP launch (the reference's decode step, port/bench.py:147-153, with
    ``tree_select``, pipeline.py:319-337, in place of ``flat_select``). Shapes and the slot
    map as ``flat_decode``; the lists and lengths are byte-identical to
    ``tree_select(index_queries(q, Hkv)[:, 0], positions, buckets, hierarchy, config,
    score_dtype=score_dtype)``'s. Deeper hierarchies take ``tree_select`` + ``lsa_read``."""
    from lsa_rocm_lab.port.read_kernel_tiled import _kv_layout

    if len(hierarchy.levels) != 1:
        raise NotImplementedError(f"tree_decode walks one node level, got {len(hierarchy.levels)}")
    if config.start_nodes is not None:
        raise NotImplementedError("tree_decode covers start_nodes=None (the top level down)")
    level = hierarchy.levels[0]
    device = _on_device("tree_decode", q, k, v, buckets.centroids, buckets.members, level.centroids)
    if q.dim() != 4 or q.shape[1] != 1:
        raise ValueError(f"tree_decode takes one query token per batch row: q [B, 1, Hq, D], got {tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    B, _, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    if k.dim() != 4 or k.shape != v.shape or k.shape[0] not in (B, 1) or k.shape[3] != D:
        raise ValueError(f"k/v must be [B={B} or 1, Tk, Hkv, D={D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads do not group onto {Hkv} kv-heads")
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool read by every batch row
        sb = 0
    layout = _Layout(torch.empty((B, Hkv, D), device="meta"), buckets.centroids)
    node_layout = _Layout(torch.empty((B, Hkv, D), device="meta"), level.centroids)
    if (node_layout.row_tables, node_layout.group_tables) != (layout.row_tables, layout.group_tables):
        raise ValueError("node and bucket tables must share the same leading axes")
    table, mode = _score_table(buckets, score_dtype)
    if mode == _abi.SCORE_BF16:
        ncent = level.centroids_bf16 if level.centroids_bf16 is not None else level.centroids.to(torch.bfloat16)
    else:
        ncent = level.centroids.float()
    ncent = ncent.contiguous()
    children = level.children.to(device=device, dtype=torch.int32).contiguous()
    members = buckets.members.to(device=device, dtype=torch.int32).contiguous()
    ends = _ends(buckets)
    flags = _table_flags(buckets, ends)
    pos = _positions32(positions, device)
    if pos.numel() != B:
        raise ValueError(f"a position a batch row: {B} rows, {pos.numel()} positions")
    top_k = config.top_k if top_k is None else top_k
    scale = D ** -0.5 if scale is None else scale
    rows, cap = layout.rows, members.shape[-1]
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(B, Hkv, width, dtype=torch.int32, device=device)
    lengths = torch.empty(B, Hkv, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    dt = _abi.dtype_code(q.dtype)
    readers = int(os.environ.get("LSA_DECODE_READERS", "0")) if readers is None else readers
    n_counters = _abi.size("lsa_decode_flat_counters", B, Hkv, rows, config.top_p)
    nbytes = _abi.size("lsa_decode_flat_scratch_bytes", dt, B, Hq, Hkv, D, rows, config.top_p,
                       config.window_size, config.sink_size, 1, readers)
    status = _abi.StatusWord.get(device)
    if int(status[0]) != 0:
        _decode_gave_up(device, status)
    ws = _abi.Workspace.get(device, "decode", nbytes)
    counters = _abi.Counters.get(device, max(n_counters, 1))
    slots, _keep = _slot_args(slot_table, slot_rows, B, device)
    _abi.call("lsa_decode_tree", q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, Tk, Hq, Hkv, D, sb, st, sh,
              ncent.data_ptr(), children.data_ptr(), children.shape[-2], children.shape[-1],
              config.node_cluster_block_size, config.beam_width, table.data_ptr(), members.data_ptr(),
              _abi.ptr(ends), flags, rows, cap, layout.row_tables, layout.group_tables, mode, pos.data_ptr(), slots,
              config.cluster_block_size, config.block_bucket_count, config.top_p, config.window_size,
              config.sink_size, top_k, float(scale), readers, counters.data_ptr(), counters.numel(), _abi.ptr(ws),
              nbytes, lists.data_ptr(), lengths.data_ptr(), out.data_ptr(), _abi.ptr(status), _abi.stream(device))
    return out, lists, lengths


def _decode_gave_up(device: torch.device, status: torch.Tensor) -> None:
    """A fused decode launch gave up waiting: its outputs were invalid and a late record
    may sit in the counters. Zero them (outside graph capture) and raise."""
    if torch.cuda.is_current_stream_capturing():
        raise _abi.LsaError(-6, "flat_decode: an earlier launch gave up waiting for its selection; "
                                "the counters need a reset outside graph capture")
    torch.cuda.synchronize(device)
    _abi.Counters.reset(device)
    torch.cuda.synchronize(device)
    status.zero_()
    raise _abi.LsaError(-6, "flat_decode: an earlier launch gave up waiting for its selection and its "
                            "outputs are invalid; the arrival counters were zeroed")


def check_decode(device: torch.device | int | None = None) -> None:
    """Synchronizes the device and raises ``LsaError`` (after zeroing the counters) if a
    fused decode launch on it gave up waiting since the last check."""
    device = torch.device("cuda", _abi.device_index(device))
    torch.cuda.synchronize(device)
    status = _abi.StatusWord.get(device)
    if int(status[0]) != 0:
        _decode_gave_up(device, status)


def reset_decode(device: torch.device | int | None = None) -> None:
    """Zeroes the fused decode's arrival counters and hand-off words on a device (outside
    graph capture, with no launch in flight). Needed after a launch that gave up waiting
    and reported it through a caller's own ``status`` word: such a launch may leave a late
    record or published keys in the shared counters, which the next launch would read."""
    device = torch.device("cuda", _abi.device_index(device))
    if torch.cuda.is_current_stream_capturing():
        raise _abi.LsaError(-6, "reset_decode: the counters cannot be reset under graph capture")
    torch.cuda.synchronize(device)
    _abi.Counters.reset(device)
    torch.cuda.synchronize(device)


def lsa_read_chunked(q, k, v, chunk_lists, chunk_lengths, scale, chunk_size: int = 64,
                     slot_table: torch.Tensor | None = None, slot_rows: torch.Tensor | None = None):
    """Chunked prefill read: every query row of a ``chunk_size`` chunk reads the chunk's
    shared per-kv-head list plus the chunk's own causal block.

    q [B, T, Hq, D] (query row t at cache position t), k/v [B, Tk, Hkv, D], chunk_lists
    [B, C, Hkv, W] / chunk_lengths [B, C, Hkv] (or without B for B == 1). A paged cache:
    the lists hold cache rows (a select given the slot map made them), ``slot_table`` maps
    the causal block's positions (``slot_rows`` [B], default row b for batch row b) and K/V
    may be one pool [1, slots, Hkv, D].
    """
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_chunked

    return sparse_read_chunked(q, k, v, chunk_lists, chunk_lengths, scale, chunk_size, slot_table=slot_table,
                               slot_rows=slot_rows)


# ----------------------------------------------------------------------------- index build


def index_queries(q: torch.Tensor, heads_kv: int, chunk: int = 1) -> torch.Tensor:
    """Per-kv-head index queries: the fp32 mean over each GQA group and ``chunk``
    consecutive tokens. q [B, T, Hq, D] -> [B, T // chunk, Hkv, D] fp32."""
    device = _on_device("index_queries", q)
    q = q.contiguous()
    B, T, Hq, D = q.shape
    out = torch.empty(B, T // chunk, heads_kv, D, dtype=torch.float32, device=device)
    _abi.call("lsa_index_queries", q.data_ptr(), _abi.dtype_code(q.dtype), B, T, Hq, heads_kv, D, chunk,
              out.data_ptr(), _abi.stream(device))
    return out


def bucket_centroids(keys: torch.Tensor, members: torch.Tensor, centroid: str = "mean"):
    """Bucket centroids (fp32, bf16) from member keys: the mean key, the L2-normalized sum
    (reference pipeline.py:108-115), or the plain sum ("sum": the hierarchy's key sums,
    :163-164). keys [T, d] with members [rows, cap], or keys
    [B, T, Hkv, D] with members [Hkv, rows, cap] (B == 1) / [B, Hkv, rows, cap]."""
    device = _on_device("bucket_centroids", keys, members)
    keys = keys.contiguous()
    members = members.to(torch.int32).contiguous()
    mode = {"mean": _abi.CENTROID_MEAN, "normalized": _abi.CENTROID_NORMALIZED, "sum": _abi.CENTROID_SUM}[centroid]
    rows, cap = members.shape[-2:]
    if keys.dim() == 2:
        T, D = keys.shape
        kv_heads, token_stride, batch_stride, n_tables = 1, D, 0, 1
    else:
        B, T, kv_heads, D = keys.shape
        token_stride, batch_stride = kv_heads * D, T * kv_heads * D
        n_tables = B * kv_heads
        if members.numel() != n_tables * rows * cap:
            raise ValueError(f"members {tuple(members.shape)} do not give one table per (batch, kv-head)")
    out32 = torch.empty(*members.shape[:-1], D, dtype=torch.float32, device=device)
    out16 = torch.empty(*members.shape[:-1], D, dtype=torch.bfloat16, device=device)
    _abi.call("lsa_bucket_centroids", keys.data_ptr(), _abi.dtype_code(keys.dtype), T, token_stride, batch_stride,
              kv_heads, D, members.data_ptr(), n_tables, rows, cap, mode, out32.data_ptr(), out16.data_ptr(),
              _abi.stream(device))
    return out32, out16


def segment_starts(keys: torch.Tensor, target: int, pool: int = 16, max_size: int = 256) -> torch.Tensor:
    """Contiguous Ward-style segments of every (batch, kv-head) key table, built on the GPU
    (the index build before the path; the reference's build_buckets_gpu, pipeline.py:71-116,
    pools keys and merges them by the Ward cost - here the merges join adjacent segments
    only, so every bucket is a run of consecutive positions).

    keys [B, T, Hkv, D] (fp32 / bf16 / fp16, read in place when rows are contiguous): pools
    of ``pool`` positions, then the adjacent pair with the smallest Ward cost
    n_a n_b / (n_a + n_b) |mu_a - mu_b|^2 merges (ties to the leftmost pair, merges past
    ``max_size`` positions skipped) until ``target`` segments remain. Returns the segment
    start positions [B, Hkv, target + 1] int64 (last = T).

    No host sync: a table that cannot reach ``target`` under ``max_size`` gets the even cut
    (valid positions) and sets the device's pinned build status word, so the next build
    call raises ValueError (``check_build`` syncs and raises at once)."""
    device = _on_device("segment_starts", keys)
    if keys.dim() != 4:
        raise ValueError(f"keys must be [B, T, Hkv, D], got {tuple(keys.shape)}")
    _build_failed(device)
    if keys.stride(-1) != 1 or keys.data_ptr() % 16:
        keys = keys.contiguous()
    B, T, Hkv, D = keys.shape
    tables = B * Hkv
    nbytes = _abi.load().lsa_ward_segments_scratch_bytes(tables, T, D, pool)
    scratch = torch.empty(max(int(nbytes), 8), dtype=torch.uint8, device=device)
    starts = torch.empty(tables, target + 1, dtype=torch.int32, device=device)
    status = torch.empty(tables, dtype=torch.int32, device=device)
    _abi.call("lsa_ward_segments", keys.data_ptr(), _abi.dtype_code(keys.dtype), B, T, Hkv, D, keys.stride(0),
              keys.stride(1), keys.stride(2), pool, target, max_size, scratch.data_ptr(), scratch.numel(),
              starts.data_ptr(), status.data_ptr(), _abi.StatusWord.get(device, "build").data_ptr(),
              _abi.stream(device))
    return starts.view(B, Hkv, target + 1).long()


def _build_failed(device: torch.device) -> None:
    """Raises (and clears the word) if an earlier bucket-table build on the device could not
    reach its segment count; reads the pinned status word, no device sync."""
    word = _abi.StatusWord.get(device, "build")
    if int(word[0]) != 0:
        word.zero_()
        raise ValueError("segment_starts: an earlier build could not reach its segment count under max_size "
                         "(that table holds the even cut instead)")


def check_build(device: torch.device | int | None = None) -> None:
    """Synchronizes the device and raises ValueError if a bucket-table build on it could not
    reach its segment count since the last check."""
    device = torch.device("cuda", _abi.device_index(device))
    torch.cuda.synchronize(device)
    _build_failed(device)


def segment_buckets(keys: torch.Tensor, target: int, pool: int = 16, max_size: int = 256, cap: int | None = None,
                    centroid: str = "mean") -> Buckets:
    """Bucket tables of contiguous Ward-style segments built on the GPU from the keys
    (``segment_starts``): member rows ids start .. end - 1 (-1 padded to ``cap``, default
    ``max_size``), span ends, and centroids from the member keys (``bucket_centroids``).
    Tables are [Hkv, rows, ...] for B == 1, else [B, Hkv, rows, ...], as the selects take
    them; ``spans`` is set, so the fused decode expands picks from the ends."""
    cap = max_size if cap is None else cap
    if cap < max_size:
        raise ValueError(f"cap {cap} below max_size {max_size}: segments would not fit their rows")
    st = segment_starts(keys, target, pool, max_size)
    if keys.shape[0] == 1:
        st = st[0]
    begin, end = st[..., :-1], st[..., 1:]
    sizes = (end - begin).to(torch.int32)
    slot = torch.arange(cap, device=st.device, dtype=torch.int64)
    members = torch.where(slot < sizes[..., None], begin[..., None] + slot, torch.full_like(slot, -1))
    members = members.to(torch.int32).contiguous()
    c32, c16 = bucket_centroids(keys, members, centroid)
    return Buckets(c16, members, sizes.contiguous(), centroids_f32=c32, ends=end.to(torch.int32).contiguous(),
                   spans=True, centroid=centroid)


def build_buckets(keys: torch.Tensor, config: PortConfig, pool: int | None = None, max_size: int | None = None,
                  centroid: str = "normalized", spans: bool = False, first_block: int = 0) -> Buckets:
    """Bucket tables of the closed cluster blocks, built on the GPU (reference
    build_buckets_gpu, pipeline.py:71-116: every closed block of ``cluster_block_size``
    keys pooled by ``pool_size`` and merged by the Ward cost into ``block_bucket_count``
    buckets of at most ``bucket_cap`` keys, rows block after block, centroids the
    normalized member-key sum). The merges here join adjacent segments only
    (``segment_starts`` per block), so every bucket is a run of consecutive positions.

    keys [T, d] (one index-space table) or [B, T, Hkv, D] (per-kv-head tables: [Hkv, rows,
    ...] for B == 1, else [B, Hkv, rows, ...]). Blocks ``first_block`` .. T // block - 1 are
    built (``extend_buckets`` appends newly closed blocks). The tables always carry their
    span ends, so the selects and the decode expand picks from them with no member-row
    loads. Visibility: by default the reference's rule - a query sees the buckets of the
    closed blocks before its own (``block_visible``); ``spans=True`` makes a bucket visible
    once its span has ended instead."""
    device = _on_device("build_buckets", keys)
    block, bpb, cap = config.cluster_block_size, config.block_bucket_count, config.bucket_cap
    pool = config.pool_size if pool is None else pool
    max_size = cap if max_size is None else max_size
    if max_size > cap:
        raise ValueError(f"max_size {max_size} exceeds the bucket cap {cap}")
    flat = keys.dim() == 2
    k4 = keys.view(1, keys.shape[0], 1, keys.shape[1]) if flat else keys
    if k4.stride(-1) != 1 or k4.data_ptr() % 16:
        k4 = k4.contiguous()
    B, T, Hkv, D = k4.shape
    blocks = T // block - first_block
    if blocks <= 0:
        raise ValueError(f"no closed block past block {first_block} in {T} keys (block {block})")
    per_b = []
    for b in range(B):
        # the closed blocks as a batch of tables: batch stride = one block of positions
        st = k4.stride(1)
        view = torch.as_strided(k4, (blocks, block, Hkv, D), (block * st, st, k4.stride(2), 1),
                                k4.storage_offset() + b * k4.stride(0) + first_block * block * st)
        starts = segment_starts(view, bpb, pool, max_size)  # [blocks, Hkv, bpb + 1], block-local
        base = (first_block + torch.arange(blocks, device=device, dtype=torch.int64)) * block
        starts = starts + base[:, None, None]
        begin = starts[..., :-1].permute(1, 0, 2).reshape(Hkv, blocks * bpb)
        end = starts[..., 1:].permute(1, 0, 2).reshape(Hkv, blocks * bpb)
        per_b.append((begin, end))
    begin = torch.stack([x[0] for x in per_b])  # [B, Hkv, rows]
    end = torch.stack([x[1] for x in per_b])
    sizes = (end - begin).to(torch.int32)
    slot = torch.arange(cap, device=device, dtype=torch.int64)
    members = torch.where(slot < sizes[..., None], begin[..., None] + slot, torch.full_like(slot, -1)).to(torch.int32)
    end = end.to(torch.int32)
    if flat:  # one table: [rows, ...]
        members, sizes, end = members[0, 0], sizes[0, 0], end[0, 0]
    elif B == 1:  # per-kv-head tables of one sequence: [Hkv, rows, ...]
        members, sizes, end = members[0], sizes[0], end[0]
    members = members.contiguous()
    c32, c16 = bucket_centroids(keys if flat else k4, members, centroid)
    return Buckets(c16, members, sizes.contiguous(), centroids_f32=c32, ends=end.contiguous(), spans=True,
                   centroid=centroid, block_visible=not spans)


def extend_buckets(buckets: Buckets, keys: torch.Tensor, config: PortConfig, **build_kw) -> Buckets:
    """The tables with the blocks closed since they were built appended (a decode cache
    grows one token a step; a block's buckets are built once, when it closes): the rows of
    blocks rows // block_bucket_count .. T // cluster_block_size - 1, built as
    ``build_buckets`` builds them, concatenated after the existing rows. The new rows keep
    the tables' centroid kind (``buckets.centroid``, else ``build_kw["centroid"]``), span
    flag and optional tensors: a table without ``centroids_f32`` or ``ends`` gets none.
    Capacity tables (``reserve_buckets``) grow in place instead (``grow_buckets_``)."""
    if buckets.built_rows is not None:  # capacity tables grow in place
        return grow_buckets_(buckets, keys, config, **build_kw)
    bpb = config.block_bucket_count
    have = buckets.rows // bpb
    T = keys.shape[0] if keys.dim() == 2 else keys.shape[1]
    if T // config.cluster_block_size <= have:
        return buckets
    kind = buckets.centroid or build_kw.pop("centroid", "normalized")
    build_kw.pop("centroid", None)
    has_ends = buckets.ends is not None
    if buckets.spans and not has_ends:
        raise ValueError("extend_buckets: span tables need their ends")
    new = build_buckets(keys, config, first_block=have, spans=not buckets.block_visible, centroid=kind, **build_kw)
    return Buckets(torch.cat([buckets.centroids, new.centroids], dim=-2),
                   torch.cat([buckets.members, new.members], dim=-2),
                   torch.cat([buckets.sizes, new.sizes], dim=-1),
                   centroids_f32=(None if buckets.centroids_f32 is None
                                  else torch.cat([buckets.centroids_f32, new.centroids_f32], dim=-2)),
                   ends=torch.cat([buckets.ends, new.ends], dim=-1) if has_ends else None,
                   spans=buckets.spans, centroid=kind, block_visible=buckets.block_visible)


def position_buckets(index_keys: torch.Tensor, config: PortConfig, centroid: str = "normalized") -> Buckets:
    """Positional block-sparse buckets - runs of ``bucket_size`` consecutive keys (reference
    pipeline.py:378-403). index_keys [T, d] gives one table; [B, T, Hkv, D] one table per
    kv-head ([Hkv, rows, ...] for B == 1, else [B, Hkv, rows, ...]). ``centroid`` is the
    reference's normalized sum or the bucket-mean key. Every row is a run of consecutive
    ids, so the tables carry span ends (the decode then expands picks from them, with no
    member-row loads); a bucket is still visible only once its block has closed
    (``block_visible``, the reference's rule for these tables, pipeline.py:184-186), and
    only when the span ends cover the rows exactly (``bucket_cap >= bucket_size``)."""
    device = _on_device("position_buckets", index_keys)
    block, size, cap = config.cluster_block_size, config.bucket_size, config.bucket_cap
    T = index_keys.shape[0] if index_keys.dim() == 2 else index_keys.shape[1]
    blocks = T // block
    rows = blocks * config.block_bucket_count
    local = torch.arange(rows * size, device=device, dtype=torch.int32).view(rows, size)
    members = F.pad(local, (0, cap - size), value=-1)
    if index_keys.dim() == 4:
        B, _, Hkv, _ = index_keys.shape
        lead = (Hkv,) if B == 1 else (B, Hkv)
        members = members.expand(*lead, rows, cap).contiguous()
    sizes = (members >= 0).sum(-1, dtype=torch.int32)
    c32, c16 = bucket_centroids(index_keys, members, centroid)
    ends = None
    if cap >= size:  # row j is exactly the ids j * size .. (j + 1) * size - 1
        ends = (torch.arange(1, rows + 1, device=device, dtype=torch.int32) * size).expand(sizes.shape).contiguous()
    return Buckets(c16, members, sizes, centroids_f32=c32, centroid=centroid, ends=ends, spans=ends is not None,
                   block_visible=ends is not None)


def build_hierarchy_gpu(index_keys: torch.Tensor, buckets: Buckets, config: PortConfig) -> Hierarchy:
    """Node levels over the buckets (reference pipeline.py:153-178 build_hierarchy_gpu).

    The bucket key sums (the sum of each bucket's member index keys, :162-164) are the
    level-0 sums. While the level below holds a full ``node_cluster_block_size`` block and
    fewer than ``top_level`` levels exist, every full block of its rows becomes
    ``block / node_bucket_size`` nodes of ``node_bucket_size`` rows each; a node's key sum
    is the sum of its rows' key sums and its centroid the L2-normalized key sum (:175-177).
    Children are rows of the level below, block after block (:170-173). The reference
    groups a block's rows by the Ward pairing cost (the upstream Triton pairing kernel);
    here a node takes consecutive rows of its block - a grouping that follows the
    bucket order, and one the walk treats like any other: the beam only assumes a node's
    children lie in the blocks closed before it was made. Sums and centroids come from
    the centroid kernel (``LSA_CENTROID_SUM`` / ``LSA_CENTROID_NORMALIZED``).

    index_keys [T, D] with one bucket table, or [B, T, Hkv, D] with tables [Hkv, ...]
    (B == 1) / [B, Hkv, ...]; node tables share the bucket tables' leading axes.
    """
    device = _on_device("build_hierarchy_gpu", index_keys, buckets.members)
    sums, _ = bucket_centroids(index_keys, buckets.members, "sum")
    hierarchy = Hierarchy(bucket_key_sums=sums)
    size, block = config.node_bucket_size, config.node_cluster_block_size
    if size < 1 or block < size or block % size:
        raise ValueError(f"node_cluster_block_size ({block}) must be a positive multiple of "
                         f"node_bucket_size ({size})")
    lead = sums.shape[:-2]
    n_tables = math.prod(lead)
    D = sums.shape[-1]
    while True:
        below = sums.shape[-2]
        blocks = below // block
        if not blocks or len(hierarchy.levels) >= config.top_level:
            break
        n_nodes = blocks * block // size
        children = torch.arange(n_nodes * size, device=device, dtype=torch.int32).view(n_nodes, size)
        children = children.expand(*lead, n_nodes, size).contiguous()
        keys = sums.reshape(n_tables, below, 1, D)
        kids = children.reshape(n_tables, n_nodes, size)
        node_sums, _ = bucket_centroids(keys, kids, "sum")
        c32, c16 = bucket_centroids(keys, kids, "normalized")
        sums = node_sums.reshape(*lead, n_nodes, D)
        hierarchy.levels.append(NodeLevel(c32.reshape(*lead, n_nodes, D), children, sums.clone(),
                                          c16.reshape(*lead, n_nodes, D)))
    return hierarchy


UNBUILT_END = 0x7FFFFFFF  # span end of a reserved row: never <= position + 1


def reserve_buckets(buckets: Buckets, capacity: int) -> Buckets:
    """Capacity tables for in-place growth (the decode cache's incremental index,
    reference pipeline.py:184-186 visibility as blocks close; docs/PORT_NOTES.md:12-14):
    every table of ``buckets`` copied into tables of ``capacity`` rows, allocated once. The
    rows past the built ones are reserved: members -1, size 0, zero centroids and span ends
    that keep them out of every list - ``UNBUILT_END`` where the ends decide visibility, an
    empty span at the last built end where the closed-block rule does. Every select and
    decode entry takes the capacity tables as they are (``rows`` = capacity);
    ``grow_buckets_`` writes newly closed blocks into the reserved rows without moving any
    tensor, so pointers captured in a HIP graph stay valid.

    Visibility: where the ends decide, a reserved row is never visible. Under the
    reference's block rule ``pos // cluster_block_size * block_bucket_count`` a reserved row
    is reached only for a position past the blocks built, so a caller grows the tables
    before it queries a position in a newly closed block (as a decode step does: the block
    closes, the index grows, then the step selects); a reserved row reached anyway holds
    nothing."""
    built = buckets.rows if buckets.built_rows is None else buckets.built_rows
    if capacity < built:
        raise ValueError(f"reserve_buckets: capacity {capacity} < the {built} rows built")
    lead = buckets.centroids.shape[:-2]
    device = buckets.centroids.device

    def grown(t, fill):
        axis = len(lead)  # the row axis
        out = torch.full((*lead, capacity, *t.shape[axis + 1:]), fill, dtype=t.dtype, device=device)
        out.narrow(axis, 0, built).copy_(t.narrow(axis, 0, built))
        return out

    ends = None
    if buckets.ends is not None:
        ends = grown(buckets.ends, UNBUILT_END)
        if buckets.block_visible and built > 0:  # reserved rows: empty spans at the last built end
            ends.narrow(len(lead), built, capacity - built).copy_(
                buckets.ends.narrow(len(lead), built - 1, 1).expand(*lead, capacity - built))
    return Buckets(grown(buckets.centroids, 0), grown(buckets.members, -1), grown(buckets.sizes, 0),
                   centroids_f32=None if buckets.centroids_f32 is None else grown(buckets.centroids_f32, 0),
                   ends=ends,
                   spans=buckets.spans, centroid=buckets.centroid, built_rows=built,
                   block_visible=buckets.block_visible)


def grow_buckets_(buckets: Buckets, keys: torch.Tensor, config: PortConfig, **build_kw) -> Buckets:
    """In place: the blocks closed since the tables were built (blocks built_rows //
    block_bucket_count .. T // cluster_block_size - 1 of ``keys``), built as
    ``build_buckets`` builds them (same centroid kind, span ends when the tables carry
    them), copied into the reserved rows of the capacity tables from ``reserve_buckets``.
    No tensor is reallocated. Returns ``buckets`` with ``built_rows`` advanced; raises
    ValueError when the capacity is exhausted."""
    if buckets.built_rows is None:
        raise ValueError("grow_buckets_ takes capacity tables (reserve_buckets); extend_buckets grows others")
    bpb = config.block_bucket_count
    have = buckets.built_rows // bpb
    T = keys.shape[0] if keys.dim() == 2 else keys.shape[1]
    blocks = T // config.cluster_block_size
    if blocks <= have:
        return buckets
    new_rows = (blocks - have) * bpb
    if buckets.built_rows + new_rows > buckets.rows:
        raise ValueError(f"grow_buckets_: {buckets.built_rows + new_rows} rows exceed the capacity {buckets.rows}")
    kind = buckets.centroid or build_kw.pop("centroid", "normalized")
    build_kw.pop("centroid", None)
    new = build_buckets(keys, config, first_block=have, spans=not buckets.block_visible, centroid=kind, **build_kw)
    lo, hi = buckets.built_rows, buckets.built_rows + new_rows
    buckets.centroids[..., lo:hi, :].copy_(new.centroids)
    buckets.members[..., lo:hi, :].copy_(new.members)
    buckets.sizes[..., lo:hi].copy_(new.sizes)
    if buckets.centroids_f32 is not None:
        buckets.centroids_f32[..., lo:hi, :].copy_(new.centroids_f32)
    if buckets.ends is not None:
        buckets.ends[..., lo:hi].copy_(new.ends)
        if buckets.block_visible and hi < buckets.rows:  # reserved rows: empty spans at the new last end
            buckets.ends[..., hi:].copy_(buckets.ends[..., hi - 1:hi].expand_as(buckets.ends[..., hi:]))
    buckets.built_rows = hi
    return buckets
