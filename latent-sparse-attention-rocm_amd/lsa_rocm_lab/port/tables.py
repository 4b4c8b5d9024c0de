"""Bucket tables on disk: one safetensors file a cache index.

The reference rebuilds its bucket tables from the keys whenever it needs them
(pipeline.py:71-116 build_buckets_gpu, :378-403 position_buckets); a serving cache keeps
them instead, so they are written once and loaded where the cache is attached. The file
stores the member lists in CSR form, every row of every table in order:

  offsets        int64 [n_rows + 1]   row r holds member_ids[offsets[r] : offsets[r + 1]]
  member_ids     int32 [offsets[-1]]  absolute key positions, in the row's order
  centroids      bf16  [*lead, rows, index_dim]   what production scoring reads
  centroids_f32  fp32  same shape, optional       fp32 scoring
  ends           int32 [*lead, rows], optional    exclusive span ends

n_rows is the product of the table shape (*lead, rows). The metadata holds the format tag
("lsa-bucket-tables/1"), the member row width (bucket_cap), the span flag and the block
visibility flag (positional tables: visible once their block closes). Loading
checks every invariant the select kernels rely on (offsets start at 0 and never decrease,
no row wider than bucket_cap, member ids >= 0, shapes agree, ends nondecreasing along each
table's rows, span tables hold exactly their span) and raises ValueError otherwise;
safetensors executes nothing from the file.
"""

from __future__ import annotations

import os

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from lsa_rocm_lab.port.pipeline import Buckets

FORMAT = "lsa-bucket-tables/1"


def save_buckets(path: str | os.PathLike, buckets: Buckets) -> None:
    """Write `buckets` (any device) to `path` in the CSR format above. Capacity tables
    (reserve_buckets) write their built rows only."""
    if buckets.built_rows is not None:
        b = buckets.built_rows
        buckets = Buckets(buckets.centroids[..., :b, :], buckets.members[..., :b, :], buckets.sizes[..., :b],
                          centroids_f32=None if buckets.centroids_f32 is None else buckets.centroids_f32[..., :b, :],
                          ends=None if buckets.ends is None else buckets.ends[..., :b], spans=buckets.spans,
                          centroid=buckets.centroid, block_visible=buckets.block_visible)
    members = buckets.members.detach().to("cpu", torch.int32)
    sizes = buckets.sizes.detach().to("cpu", torch.int64)
    if members.dim() < 2 or tuple(sizes.shape) != tuple(members.shape[:-1]):
        raise ValueError(f"save_buckets: members {tuple(members.shape)} and sizes {tuple(sizes.shape)} disagree")
    cap = members.shape[-1]
    flat_sizes = sizes.reshape(-1)
    if bool((flat_sizes < 0).any()) or bool((flat_sizes > cap).any()):
        raise ValueError("save_buckets: a row size lies outside [0, bucket_cap]")
    rows2d = members.reshape(-1, cap)
    keep = torch.arange(cap)[None, :] < flat_sizes[:, None]
    if bool(((rows2d >= 0) != keep).any()) or bool((rows2d < -1).any()):
        raise ValueError("save_buckets: every row must hold its `sizes` real ids (>= 0) first, then -1 padding")
    offsets = torch.zeros(flat_sizes.numel() + 1, dtype=torch.int64)
    torch.cumsum(flat_sizes, 0, out=offsets[1:])
    tensors = {
        "offsets": offsets,
        "member_ids": rows2d[keep].contiguous(),
        "centroids": buckets.centroids.detach().to("cpu", torch.bfloat16).contiguous(),
    }
    if buckets.centroids_f32 is not None:
        tensors["centroids_f32"] = buckets.centroids_f32.detach().to("cpu", torch.float32).contiguous()
    if buckets.ends is not None:
        tensors["ends"] = buckets.ends.detach().to("cpu", torch.int32).contiguous()
    meta = {"format": FORMAT, "bucket_cap": str(cap), "spans": "1" if buckets.spans else "0",
            "block_visible": "1" if buckets.block_visible else "0"}
    save_file(tensors, os.fspath(path), metadata=meta)


def load_buckets(path: str | os.PathLike, device: str | torch.device = "cpu") -> Buckets:
    """Read a file written by save_buckets onto `device`; ValueError on a malformed file."""
    with safe_open(os.fspath(path), framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"load_buckets: not a bucket-table file (format {meta.get('format')!r})")
        names = set(f.keys())
        for need in ("offsets", "member_ids", "centroids"):
            if need not in names:
                raise ValueError(f"load_buckets: missing tensor {need!r}")
        t = {n: f.get_tensor(n) for n in names}
    try:
        cap = int(meta["bucket_cap"])
        spans = meta["spans"] == "1"
        block_visible = meta.get("block_visible", "0") == "1"
    except (KeyError, ValueError) as e:
        raise ValueError(f"load_buckets: bad metadata {meta}") from e
    offsets, ids, cent = t["offsets"], t["member_ids"], t["centroids"]
    if offsets.dtype != torch.int64 or ids.dtype != torch.int32 or cent.dtype != torch.bfloat16:
        raise ValueError("load_buckets: offsets must be int64, member_ids int32, centroids bf16")
    if cent.dim() < 2 or cap < 1:
        raise ValueError("load_buckets: centroids need a [..., rows, index_dim] shape and bucket_cap >= 1")
    shape = tuple(cent.shape[:-1])
    n_rows = 1
    for s in shape:
        n_rows *= s
    if offsets.dim() != 1 or offsets.numel() != n_rows + 1 or int(offsets[0]) != 0:
        raise ValueError(f"load_buckets: offsets must be [{n_rows + 1}] starting at 0")
    sizes = offsets[1:] - offsets[:-1]
    if bool((sizes < 0).any()) or bool((sizes > cap).any()):
        raise ValueError("load_buckets: a row's offsets decrease or exceed bucket_cap")
    if int(offsets[-1]) != ids.numel() or ids.dim() != 1:
        raise ValueError(f"load_buckets: {ids.numel()} member ids for offsets ending at {int(offsets[-1])}")
    if bool((ids < 0).any()):
        raise ValueError("load_buckets: member ids must be >= 0 (-1 only pads a row past its size)")
    members = torch.full((n_rows, cap), -1, dtype=torch.int32)
    keep = torch.arange(cap)[None, :] < sizes[:, None]
    members[keep] = ids
    for opt in ("centroids_f32", "ends"):
        if opt in t:
            want = shape + ((cent.shape[-1],) if opt == "centroids_f32" else ())
            if tuple(t[opt].shape) != want:
                raise ValueError(f"load_buckets: {opt} {tuple(t[opt].shape)} != {want}")
    if "centroids_f32" in t and t["centroids_f32"].dtype != torch.float32:
        raise ValueError("load_buckets: centroids_f32 must be fp32")
    ends = t.get("ends")
    if ends is not None and ends.dtype != torch.int32:
        raise ValueError("load_buckets: ends must be int32")
    if ends is not None and shape[-1] > 1:
        e2 = ends.reshape(-1, shape[-1])
        if bool((e2[:, 1:] < e2[:, :-1]).any()):
            raise ValueError("load_buckets: ends decrease along a table's rows")
    if spans:
        if ends is None:
            raise ValueError("load_buckets: a span table needs its ends")
        e = ends.reshape(-1, shape[-1]).to(torch.int64)
        begin = torch.cat([torch.zeros_like(e[:, :1]), e[:, :-1]], dim=1).reshape(-1)
        if bool((e.reshape(-1) - begin != sizes).any()):
            raise ValueError("load_buckets: span rows do not hold exactly their spans")
        want = begin[:, None] + torch.arange(cap)[None, :]
        if not torch.equal(torch.where(keep, want, -1).to(torch.int32), members):
            raise ValueError("load_buckets: span rows do not hold exactly their spans")
    dev = torch.device(device)
    return Buckets(
        centroids=cent.to(dev),
        members=members.reshape(*shape, cap).to(dev),
        sizes=sizes.to(torch.int32).reshape(shape).to(dev),
        centroids_f32=t["centroids_f32"].to(dev) if "centroids_f32" in t else None,
        ends=ends.to(dev) if ends is not None else None,
        spans=spans,
        block_visible=block_visible and ends is not None,
    )
