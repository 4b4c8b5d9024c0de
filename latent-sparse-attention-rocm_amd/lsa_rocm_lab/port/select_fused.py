"""Fused selection kernels (reference src/lsa_rocm_lab/port/select_fused.py).

``select_topk_scores`` (reference :83-137): fp32 score rows to their best
``min(top_p, N)`` packed keys, descending, in one HIP kernel per row (pack in
registers, radix select of the k-th key in LDS, bitonic sort of the k winners).
Rows wider than ``4 * top_p`` keep the reference's visible "sampled listing"
warning; the kernel computes the same length-respecting best-k there.

``expand_in_order_from_keys`` (reference :217-280) and ``expand_in_order`` (the
upstream walk it fuses, called at pipeline.py:269-271): the rank-order expansion
as a block-wide prefix-sum compaction over (pick, member slot) in rank order.
"""

from __future__ import annotations

import warnings

import torch

from lsa_rocm_lab import _abi

WHOLE_FACTOR = 4


def _next_pow2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def select_topk_scores(scores: torch.Tensor, lengths: torch.Tensor, top_p: int) -> torch.Tensor:
    """The whole-path listing + best-first keys, fused (reference select_fused.py:83-137).

    Args:
        scores: Score matrix [R, N] fp32.
        lengths: Columns each row sees [R] int32, at most N.
        top_p: Best keys per row.

    Returns:
        Ordered packed keys [R, K2] int64, K2 = next_pow2(min(top_p, N)), EMPTY-padded;
        on the sampled-listing path (N > 4 * top_p, reference :97-117) [R, min(top_p, N)],
        the width ``torch.topk`` gives there.
    """
    rows, columns = scores.shape
    sampled = columns > WHOLE_FACTOR * top_p
    if sampled:
        warnings.warn(
            f"select_topk_scores: {columns} columns > {WHOLE_FACTOR} * top_p {top_p} "
            "- sampled listing contract, using the length-respecting pack+topk "
            "(upstream TopK.best() semantics)",
            stacklevel=2,
        )
    if scores.device.type != "cuda":
        raise ValueError(f"select_topk_scores is a ROCm kernel, got device {scores.device}")
    if scores.dtype != torch.float32:
        raise ValueError(f"scores must be the GEMM's fp32 output, got {scores.dtype}")
    keep = min(top_p, columns)
    k2 = _next_pow2(keep)
    out = torch.empty(rows, k2, device=scores.device, dtype=torch.int64)
    if rows == 0:
        return out[:, :keep] if sampled else out
    scores = scores.contiguous()
    lengths = lengths.to(device=scores.device, dtype=torch.int32).reshape(rows).contiguous()
    _abi.call("lsa_select_topk_scores", scores.data_ptr(), lengths.data_ptr(), rows, columns, top_p,
              out.data_ptr(), _abi.stream(scores.device))
    return out[:, :keep].contiguous() if sampled and keep != k2 else out


def _expand(picks, picks_are_keys, bucket_members, positions, window_size, sink_size, top_k, slot_table=None,
            slot_rows=None):
    from lsa_rocm_lab.port.pipeline import _slot_args

    device = picks.device
    picks = picks.contiguous()
    rows = picks.shape[0]
    members = bucket_members.to(device=device, dtype=torch.int32).contiguous()
    pos = positions.to(device=device, dtype=torch.int32).reshape(rows).contiguous()
    width = top_k + window_size + sink_size
    out = torch.empty(rows, width, device=device, dtype=torch.int32)
    lengths = torch.empty(rows, device=device, dtype=torch.int32)
    if rows == 0:
        return out, lengths
    slots, _keep = _slot_args(slot_table, slot_rows, rows, device)
    _abi.call("lsa_expand", picks.data_ptr(), 1 if picks_are_keys else 0, rows, 1, picks.shape[1],
              members.data_ptr(), members.shape[0], members.shape[1], 0, 0, pos.data_ptr(), slots, window_size,
              sink_size, top_k, out.data_ptr(), lengths.data_ptr(), _abi.stream(device))
    return out, lengths


def expand_in_order_from_keys(
    ordered_keys: torch.Tensor,
    bucket_members: torch.Tensor,
    positions: torch.Tensor,
    window_size: int,
    sink_size: int,
    top_k: int,
    slot_table: torch.Tensor | None = None,
    slot_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Read lists from ordered packed keys (reference select_fused.py:217-280).

    Args:
        ordered_keys: Packed keys [R, W] int64, best first, EMPTY-padded tail.
        bucket_members: Members of each cache row [rows, bucket_cap] int32, -1 padded.
        positions: Each row's position [R] int32.
        window_size: Recent positions read whole.
        sink_size: First positions read whole.
        top_k: Bucket members read at most.
        slot_table: A paged cache's slot table [n_rows, width] int32 (the kernel's
            ``MAP_SLOTS`` path, :147-205): every listed id is stored as its cache row.
        slot_rows: Each row's slot-table row [R] int32.

    Returns:
        Read lists [R, top_k + window_size + sink_size] int32, -1 padded, and lengths [R].
    """
    if ordered_keys.device.type != "cuda":
        raise ValueError(f"expand_in_order_from_keys is a ROCm kernel, got device {ordered_keys.device}")
    bucket_cap = bucket_members.size(1)
    decoding = ordered_keys.size(0) <= 32
    tile = max(1, (4096 if decoding else 1024) // bucket_cap)
    if (tile * bucket_cap) & (tile * bucket_cap - 1):
        # the reference's walk tile must be a power of two; the same inputs are refused here
        raise ValueError(
            f"bucket_cap {bucket_cap} yields a non-power-of-two walk tile {tile * bucket_cap} "
            "- use a power-of-two bucket_cap (production: 16)"
        )
    return _expand(ordered_keys, True, bucket_members, positions, window_size, sink_size, top_k, slot_table,
                   slot_rows)


def expand_in_order(
    picked: torch.Tensor,
    bucket_members: torch.Tensor,
    positions: torch.Tensor,
    window_size: int,
    sink_size: int,
    top_k: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Upstream ``expand_in_order`` on int32 picks (-1 = none), as the reference chain
    calls it (pipeline.py:269-271): same contract as ``expand_in_order_from_keys``."""
    if picked.device.type != "cuda":
        raise ValueError(f"expand_in_order is a ROCm kernel, got device {picked.device}")
    return _expand(picked.to(torch.int32), False, bucket_members, positions, window_size, sink_size, top_k)
