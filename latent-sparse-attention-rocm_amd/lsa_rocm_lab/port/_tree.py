"""The tree beam on the GPU (reference src/lsa_rocm_lab/port/_tree.py), one HIP kernel.

Scope: a node tree of ONE level over the buckets (e.g. 128 nodes of 16 buckets). Per
(query row, kv-head) one workgroup replays the row's growth (reference :100-142 with one
level: nodes are made over whole ``node_cluster_block_size`` blocks of the row's visible
buckets), scores the made nodes, keeps the best ``beam_width`` (a tie to the lower
node), gathers their visible children plus the fresh buckets ``[covered, visible)``,
removes duplicates, keeps the best ``top_p`` (a tie to the lower bucket), and expands
them in rank order - the semantics of the reference's ``_beam_pick_rows`` (:318-373)
with one level, whose start level is taken whole. Invalid candidates are never picked
(the list tail is -1).
"""

from __future__ import annotations

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
)


def tree_select_batched(
    index_queries: torch.Tensor,
    positions: torch.Tensor,
    buckets: Buckets,
    hierarchy: Hierarchy,
    config: PortConfig,
    top_k: int | None = None,
    score_dtype: str = "fp32",
):
    """Select by the one-level beam, expand in rank order - see ``pipeline.tree_select``.

    ``LSA_TREE_IMPL`` (reference _tree.py:53) is read for compatibility; ``per_page``
    and ``batched`` name the same kernel here.
    """
    os.environ.get("LSA_TREE_IMPL", "per_page")
    top_k = config.top_k if top_k is None else top_k
    if len(hierarchy.levels) != 1:
        raise NotImplementedError(
            f"tree_select covers a one-level node tree, got {len(hierarchy.levels)} levels"
        )
    if config.start_nodes is not None:
        raise NotImplementedError("tree_select covers start_nodes=None (the top level down)")
    level = hierarchy.levels[0]
    device = _on_device("tree_select", index_queries, buckets.centroids, level.centroids)
    if positions.shape[0] != index_queries.shape[0]:
        raise ValueError(
            f"a position a query: {index_queries.shape[0]} queries, {positions.shape[0]} positions"
        )
    layout = _Layout(index_queries, buckets.centroids)
    node_layout = _Layout(index_queries, level.centroids)
    if (node_layout.row_tables, node_layout.group_tables) != (layout.row_tables, layout.group_tables):
        raise ValueError("node and bucket tables must share the same leading axes")
    if score_dtype == "fp32":
        if buckets.centroids_f32 is None:
            raise ValueError("fp32 scoring needs buckets.centroids_f32")
        ncent, bcent, mode = level.centroids.float(), buckets.centroids_f32.float(), _abi.SCORE_F32
    elif score_dtype == "bf16":
        nb = level.centroids_bf16 if level.centroids_bf16 is not None else level.centroids.to(torch.bfloat16)
        ncent, bcent, mode = nb, buckets.centroids.to(torch.bfloat16), _abi.SCORE_BF16
    else:
        raise ValueError(f"score_dtype must be bf16|fp32, got {score_dtype!r}")
    ncent, bcent = ncent.contiguous(), bcent.contiguous()
    children = level.children.to(device=device, dtype=torch.int32).contiguous()
    members = buckets.members.to(device=device, dtype=torch.int32).contiguous()
    n_nodes, node_size = children.shape[-2], children.shape[-1]
    q = _queries(index_queries)
    pos = _positions32(positions, device)
    ends = _ends(buckets)
    width = top_k + config.window_size + config.sink_size
    lists = torch.empty(layout.out_shape(width), dtype=torch.int32, device=device)
    lengths = torch.empty(layout.out_shape(), dtype=torch.int32, device=device)
    _abi.call("lsa_select_tree", q.data_ptr(), _abi.dtype_code(q.dtype), layout.R, layout.G, layout.D,
              ncent.data_ptr(), children.data_ptr(), n_nodes, node_size, bcent.data_ptr(), members.data_ptr(),
              _abi.ptr(ends), _abi.TABLE_SPANS if (buckets.spans and ends is not None) else 0, layout.rows,
              members.shape[-1], layout.row_tables, layout.group_tables, mode,
              pos.data_ptr(), config.cluster_block_size, config.block_bucket_count, config.node_cluster_block_size,
              config.beam_width, config.top_p, config.window_size, config.sink_size, top_k, lists.data_ptr(),
              lengths.data_ptr(), _abi.stream(device))
    return lists, lengths


def tree_select_per_page(index_queries, positions, buckets, hierarchy, config, top_k=None, score_dtype="fp32"):
    """Reference _tree.py:63-85 entry name; the same kernel as ``tree_select_batched``."""
    return tree_select_batched(index_queries, positions, buckets, hierarchy, config, top_k, score_dtype)
