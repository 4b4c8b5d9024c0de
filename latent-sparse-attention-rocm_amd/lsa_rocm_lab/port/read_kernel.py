"""The v1 sparse read contract (reference src/lsa_rocm_lab/port/read_kernel.py).

Same gather kernel as ``read_kernel_tiled``; the only difference the reference's v1
has is its zero-length hazard: a row with no keys gives 0/0 = NaN (reference
read_kernel.py:76). Kept so callers and A/B tests that pin that contract still run.
"""

from __future__ import annotations

import torch

from lsa_rocm_lab.port.read_kernel_tiled import _sparse_read


def sparse_read(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    read_ids: torch.Tensor,
    lengths: torch.Tensor,
    scale: float | None = None,
    block: int = 64,
) -> torch.Tensor:
    """Attention over each query row's read list, v1 contract (reference read_kernel.py:80-120).

    ``block`` is accepted for signature parity. Returns output like ``q``; rows with
    no keys are NaN.
    """
    return _sparse_read(q, k, v, read_ids, lengths, scale, empty_nan=True, splits=1)
