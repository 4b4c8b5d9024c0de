"""The sparse read (reference src/lsa_rocm_lab/port/read_kernel_tiled.py).

One HIP gather-attention kernel serves every launch shape. A workgroup owns one
(query row, kv-head) and a slice of its read list; the kv-head's whole GQA group
shares each gathered K/V row, fetched once as 16-byte coalesced loads; scores and
the online softmax are fp32; when there are few rows (decode) each list is split
over several workgroups and the last one to finish merges their softmax partials.
Contract as the reference: -1 ids and slots past a row's length are skipped,
duplicates count per occurrence, a row with no keys gives zeros, the output has q's
dtype. Lists are [B, Tq, W] shared by all heads or [B, Tq, Hkv, W] per kv-head
(lengths [B, Tq] or [B, Tq, Hkv]).
"""

from __future__ import annotations

import math
import os

import torch

from lsa_rocm_lab import _abi

DECODE_ROW_LIMIT = 32


MAX_SPLITS = 256


def _read_splits(units: int, width: int, tile: int) -> int:
    """Spans per (row, kv-head), aiming at about 512 workgroups: with few rows (B=1
    decode: 8 units) a list is cut into spans of one tile so ~every CU gets a workgroup;
    with many rows each list stays whole or nearly, and a workgroup streams its span with
    the next tile's loads in flight (B=32 x 131k tree read: 2 spans a list, 58 us; 16
    spans took 62.7 us, the partials and their combine costing more than the spread)."""
    env = os.environ.get("LSA_READ_SPLITS")
    if env:
        return max(1, min(int(env), MAX_SPLITS))
    tiles = max(1, math.ceil(width / tile))
    return max(1, min(tiles, max(1, 512 // max(units, 1)), MAX_SPLITS))


def _kv_layout(k: torch.Tensor, v: torch.Tensor):
    """K/V as the kernel reads them: rows of D contiguous elements at shared batch/token/
    head strides, read in place (a cache view costs no copy); other layouts are made dense."""
    aligned = all(x % 16 == 0 for x in (k.data_ptr(), v.data_ptr()))
    if k.stride(-1) != 1 or v.stride(-1) != 1 or k.stride() != v.stride() or not aligned:
        k, v = k.contiguous(), v.contiguous()
    return k, v, k.stride(0), k.stride(1), k.stride(2)


def _sparse_read(q, k, v, read_ids, lengths, scale, empty_nan: bool, splits: int | None = None):
    assert q.is_cuda and k.is_cuda and v.is_cuda, "the sparse read is a GPU kernel"
    B, Tq, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    assert Hq % Hkv == 0, "query heads must group evenly onto KV heads"
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    if k.shape[0] not in (B, 1) or k.shape != v.shape:
        raise ValueError(f"k/v {tuple(k.shape)} / {tuple(v.shape)} must hold {B} batch rows (or one shared pool)")
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool (a paged cache) read by every batch row
        sb = 0
    rows = B * Tq
    width = read_ids.shape[-1]
    per_head = Hkv > 1 and lengths.numel() == rows * Hkv and lengths.numel() != rows
    ids = read_ids.to(torch.int32).reshape(-1, width).contiguous()
    lens = lengths.to(device=q.device, dtype=torch.int32).reshape(-1).contiguous()
    expect = rows * Hkv if per_head else rows
    if ids.shape[0] != expect or lens.numel() != expect:
        raise ValueError(f"read lists {tuple(read_ids.shape)} / lengths {tuple(lengths.shape)} do not match "
                         f"{rows} query rows" + (f" x {Hkv} kv-heads" if per_head else ""))
    out = torch.empty_like(q)
    if rows == 0:
        return out
    if splits is None:
        tile = _abi.size("lsa_read_tile_tokens", _abi.dtype_code(q.dtype), D, Hq // Hkv)
        splits = _read_splits(rows * Hkv, width, max(tile, 1))
    nbytes = _abi.size("lsa_read_scratch_bytes", rows, Hq, Hkv, D, splits)
    ws = _abi.Workspace.get(q.device, "read", nbytes)
    counters = _abi.Counters.get(q.device, rows * Hkv) if nbytes else None
    _abi.call("lsa_read", q.data_ptr(), k.data_ptr(), v.data_ptr(), _abi.dtype_code(q.dtype), B, Tq, Tk, Hq, Hkv, D,
              sb, st, sh, ids.data_ptr(), lens.data_ptr(), width, 1 if per_head else 0, float(D ** -0.5 if scale is None else scale),
              1 if empty_nan else 0, splits, _abi.ptr(counters), _abi.ptr(ws), nbytes, out.data_ptr(),
              _abi.stream(q.device))
    return out


def sparse_read_tiled(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    read_ids: torch.Tensor,
    lengths: torch.Tensor,
    scale: float | None = None,
    tile_rows: int = 4,
    chunk: int = 64,
    num_warps: int = 4,
) -> torch.Tensor:
    """Attention over each query row's read list (reference read_kernel_tiled.py:92-136).

    ``tile_rows``/``chunk``/``num_warps`` are the reference kernel's tunables; they are
    accepted and do not change the HIP launch, whose shape comes from the list layout.
    Returns attention output, same shape/dtype/device as ``q``.
    """
    return _sparse_read(q, k, v, read_ids, lengths, scale, empty_nan=False)


def sparse_read_auto(q, k, v, read_ids, lengths, scale=None):
    """The production sparse read entry (reference read_kernel_tiled.py:147-156)."""
    return _sparse_read(q, k, v, read_ids, lengths, scale, empty_nan=False)


def sparse_read_chunked(q, k, v, chunk_lists, chunk_lengths, scale=None, chunk_size: int = 64, path: str | None = None,
                        slot_table=None, slot_rows=None):
    """Chunked-prefill read: query row t reads chunk ``t // chunk_size``'s per-kv-head list
    and the chunk's causal block [chunk start, t]. chunk_lists [B, C, Hkv, W] (or
    [C, Hkv, W] for B == 1), chunk_lengths [B, C, Hkv] (or [C, Hkv]).

    ``path`` (default ``LSA_PREFILL_READ`` or ``auto``): ``auto`` runs the MFMA tile kernel
    where it applies (bf16/fp16, D 64/128, power-of-two chunk 16..256) and the gather kernel
    elsewhere; ``gather`` / ``mfma`` force one (``mfma`` raises where it does not apply).
    ``slot_table`` / ``slot_rows`` (a paged cache): the causal block's positions go through
    the slot table (rows default to the batch row); K/V may be one pool [1, slots, Hkv, D]."""
    from lsa_rocm_lab.port.pipeline import _slot_args

    assert q.is_cuda and k.is_cuda and v.is_cuda, "the sparse read is a GPU kernel"
    B, T, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    assert Hq % Hkv == 0, "query heads must group evenly onto KV heads"
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    if k.shape[0] not in (B, 1) or k.shape != v.shape:
        raise ValueError(f"k/v {tuple(k.shape)} / {tuple(v.shape)} must hold {B} batch rows (or one shared pool)")
    C = -(-T // chunk_size)
    width = chunk_lists.shape[-1]
    ids = chunk_lists.to(torch.int32).reshape(B * C * Hkv, width).contiguous()
    lens = chunk_lengths.to(device=q.device, dtype=torch.int32).reshape(B * C * Hkv).contiguous()
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    if k.shape[0] != B:  # one pool (a paged cache) read by every batch row
        sb = 0
    out = torch.empty_like(q)
    if B * T == 0:
        return out
    path = os.environ.get("LSA_PREFILL_READ", "auto") if path is None else path
    codes = {"auto": _abi.CHUNKED_AUTO, "gather": _abi.CHUNKED_GATHER, "mfma": _abi.CHUNKED_MFMA}
    if path not in codes:
        raise ValueError(f"chunked read path must be auto|gather|mfma, got {path!r}")
    slots, _keep = _slot_args(slot_table, slot_rows, B, q.device)
    _abi.call("lsa_read_chunked", q.data_ptr(), k.data_ptr(), v.data_ptr(), _abi.dtype_code(q.dtype), B, T, Tk, Hq,
              Hkv, D, sb, st, sh, ids.data_ptr(), lens.data_ptr(), width, chunk_size, slots,
              float(D ** -0.5 if scale is None else scale), codes[path], out.data_ptr(), _abi.stream(q.device))
    return out
