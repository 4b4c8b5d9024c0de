"""The tree beam on the GPU (reference src/lsa_rocm_lab/port/_tree.py), one HIP kernel a call.

Per (query row, kv-head) one workgroup replays the row's growth (reference :100-142:
nodes are made over whole ``node_cluster_block_size`` blocks of the row's visible
buckets, and a level's nodes close in whole blocks into the level above, up to
``top_level`` levels), walks the levels from the highest one holding a made node down
(candidates: the carried children plus the level's open nodes, each once), keeps the
best ``beam_width`` a level (a tie to the lower node), then the best ``top_p`` of the
carried buckets plus the fresh buckets ``[covered, visible)`` (a tie to the lower
bucket), and expands them in rank order - the semantics of the reference's
``_beam_pick_rows`` (:318-373) with ``_dedup_scores`` (:306-315). A one-level tree runs
``lsa_select_tree``, deeper ones ``lsa_select_beam``. Invalid candidates are never
picked (the list tail is -1).
"""

from __future__ import annotations

import ctypes
import os

import torch

from lsa_rocm_lab import _abi
from lsa_rocm_lab.port.pipeline import (
    Buckets,
    Hierarchy,
    PortConfig,
    _Layout,
    _ends,
    _on_device,
    _positions32,
    _queries,
    _slot_args,
    _table_flags,
)


def tree_select_batched(
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    hierarchy: Hierarchy,
    config: PortConfig,
    top_k: int | None = None,
    score_dtype: str = "fp32",
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
):
    """Select by the beam, expand in rank order - see ``pipeline.tree_select``.

    ``LSA_TREE_IMPL`` (reference _tree.py:53) is read for compatibility; ``per_page``
    and ``batched`` name the same kernel here.
    """
    os.environ.get("LSA_TREE_IMPL", "per_page")
    top_k = config.top_k if top_k is None else top_k
    n_levels = len(hierarchy.levels)
    if not 1 <= n_levels <= _abi.BEAM_MAX_LEVELS:
        raise NotImplementedError(f"tree_select covers 1 to {_abi.BEAM_MAX_LEVELS} node levels, got {n_levels}")
    if config.start_nodes is not None:
        raise NotImplementedError("tree_select covers start_nodes=None (the top level down)")
    device = _on_device("tree_select", index_queries, buckets.centroids,
                        *[level.centroids for level in hierarchy.levels])
    if positions.shape[0] != index_queries.shape[0]:
        raise ValueError(
            f"a position a query: {index_queries.shape[0]} queries, {positions.shape[0]} positions"
        )
    layout = _Layout(index_queries, buckets.centroids)
    for level in hierarchy.levels:
        node_layout = _Layout(index_queries, level.centroids)
        if (node_layout.row_tables, node_layout.group_tables) != (layout.row_tables, layout.group_tables):
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
    if any(k.shape[-1] != node_size for k in kids):
        raise ValueError("every node level must hold node_bucket_size children a node")
    members = buckets.members.to(device=device, dtype=torch.int32).contiguous()
    q = _queries(index_queries)
    pos = _positions32(positions, device)
    ends = _ends(buckets)
    flags = _table_flags(buckets, ends)
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(layout.out_shape(width), dtype=torch.int32, device=device)
    lengths = torch.empty(layout.out_shape(), dtype=torch.int32, device=device)
    slots, _keep = _slot_args(slot_table, slot_rows, layout.R, device)
    if n_levels == 1:
        _abi.call("lsa_select_tree", q.data_ptr(), _abi.dtype_code(q.dtype), layout.R, layout.G, layout.D,
                  ncents[0].data_ptr(), kids[0].data_ptr(), kids[0].shape[-2], node_size, bcent.data_ptr(),
                  members.data_ptr(), _abi.ptr(ends), flags, layout.rows, members.shape[-1], layout.row_tables,
                  layout.group_tables, mode, pos.data_ptr(), slots, config.cluster_block_size,
                  config.block_bucket_count,
                  config.node_cluster_block_size, config.beam_width, config.top_p, config.window_size,
                  config.sink_size, top_k, lists.data_ptr(), lengths.data_ptr(), _abi.stream(device))
        return lists, lengths
    cent_ptrs = (ctypes.c_void_p * n_levels)(*[c.data_ptr() for c in ncents])
    kid_ptrs = (ctypes.c_void_p * n_levels)(*[k.data_ptr() for k in kids])
    n_nodes = (ctypes.c_int32 * n_levels)(*[k.shape[-2] for k in kids])
    _abi.call("lsa_select_beam", q.data_ptr(), _abi.dtype_code(q.dtype), layout.R, layout.G, layout.D, n_levels,
              ctypes.addressof(cent_ptrs), ctypes.addressof(kid_ptrs), ctypes.addressof(n_nodes), node_size,
              config.node_cluster_block_size, config.top_level, bcent.data_ptr(), members.data_ptr(),
              _abi.ptr(ends), flags, layout.rows, members.shape[-1], layout.row_tables, layout.group_tables, mode,
              pos.data_ptr(), slots, config.cluster_block_size, config.block_bucket_count, config.beam_width,
              config.top_p, config.window_size, config.sink_size, top_k, lists.data_ptr(), lengths.data_ptr(),
              _abi.stream(device))
    return lists, lengths


def tree_select_per_page(index_queries, positions, buckets, hierarchy, config, top_k=None, score_dtype="fp32",
                         slot_table=None, slot_rows=None):
    """Reference _tree.py:63-85 entry name; the same kernel as ``tree_select_batched``."""
    return tree_select_batched(index_queries, positions, buckets, hierarchy, config, top_k, score_dtype,
                               slot_table, slot_rows)
