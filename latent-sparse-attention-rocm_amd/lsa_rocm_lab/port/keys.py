"""Packed selection keys on the GPU - the layout the reference takes from upstream ``keys``.

``key = (ordered_bits(score) << 32) | (0x7FFFFFFF - column)``; ``EMPTY`` (int64 min)
sorts after every real key, so best-first order is descending key order and a score
tie goes to the lower column (reference select_fused.py:71-77, pipeline.py:189-214,
docs/v0.4.0/EXPERIMENT_DECISIONS.md:35). ``ordered_bits`` maps fp32 bits to an int32
whose signed order is the float order: non-negative floats keep their bits, negative
floats flip the 31 magnitude bits.
"""

from __future__ import annotations

import torch

from lsa_rocm_lab import _abi

EMPTY = -(1 << 63)
# Listing contract: rows up to WHOLE * top_p columns are packed whole (reference
# select_fused.py:45-49, pipeline.py:245).
WHOLE = 4


def _cuda(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} is a ROCm kernel, got device {t.device}")


def listed(scores: torch.Tensor, counts: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Upstream ``TopK(top_p, exact=False).listed`` (reference pipeline.py:266-267): every
    column of the fp32 score rows packed, EMPTY at or past each row's count. Returns
    (keys [R, N] int64, listed counts [R] int32). Every slot is written, so the listing is
    the whole row at any width - a superset of every row's best keys."""
    _cuda(scores, "listed")
    if scores.dtype != torch.float32:
        raise ValueError(f"scores must be fp32, got {scores.dtype}")
    scores = scores.contiguous()
    rows, cols = scores.shape
    counts = counts.to(device=scores.device, dtype=torch.int32).reshape(rows).contiguous()
    keys = torch.empty(rows, cols, dtype=torch.int64, device=scores.device)
    _abi.call("lsa_pack_listing", scores.data_ptr(), counts.data_ptr(), rows, cols, keys.data_ptr(),
              _abi.stream(scores.device))
    return keys, counts


def unpack_ids(keys: torch.Tensor) -> torch.Tensor:
    """Key -> int32 column, -1 for EMPTY (upstream ``unpack_ids``, reference pipeline.py:268)."""
    _cuda(keys, "unpack_ids")
    keys = keys.contiguous()
    ids = torch.empty(keys.shape, dtype=torch.int32, device=keys.device)
    _abi.call("lsa_unpack_ids", keys.data_ptr(), keys.numel(), ids.data_ptr(), _abi.stream(keys.device))
    return ids


def pack_keys(scores: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """Upstream ``pack_keys``: column ids >= 0 packed with their scores, -1 ids EMPTY
    (reference select_fused.py:113-116). The ids must be each row's column index or -1,
    which is what every call site passes; they are realised as listing counts."""
    _cuda(scores, "pack_keys")
    live = ids >= 0
    counts = live.sum(1, dtype=torch.int32)
    keys, _ = listed(scores, counts)
    return keys
