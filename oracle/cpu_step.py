"""A vectorized pure-PyTorch CPU restatement of one decode step (select + read).

TEST INFRASTRUCTURE / CPU COMPARATOR. ``bench.py``'s ``cpu_baseline`` leg times this on
the host cores (``torch.set_num_threads``), and ``tests/test_cpu_step.py`` holds it equal
to the numpy oracle (``oracle.lsa_oracle``): lists and lengths bit for bit, the read within
the fp32 bar. The product package never imports it.

It is the same computation as the reference's decode step (port/bench.py:147-153: the
flat select of pipeline.py:248-271 on the GQA group-mean index queries, then the sparse
read of read_kernel_tiled.py:30-89), written as whole-tensor torch ops, not per-row
loops, so that it is a representative CPU path:

* index query: fp32 sum of the group's query heads in head order, one division
  (gates.py:50-59 as the benchmark geometry states it);
* canonical score: operands rounded to the scoring type, fp64 products, 16 in-order
  partial sums over contiguous D/16 slices, the tree (p, p+8), (p, p+4), (p, p+2),
  (p, p+1), one rounding to fp32 (pipeline.py:217-232 with a fixed summation order);
* packed keys and the best ``top_p`` by ``torch.topk`` (pipeline.py:189-214,
  select_fused.py:71-77);
* rank-order expansion: picks in rank order, member slots in table order, ids with
  ``sink <= id < window_start`` until ``top_k``, then the window, then the sinks
  (select_fused.py:172-214);
* read: fp32 softmax(scale q K^T) V over the listed rows per query head
  (read_kernel_tiled.py:50-89), an empty list giving 0.
"""

from __future__ import annotations

import torch

EMPTY = -(1 << 63)
PARTIALS = 16


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def index_queries(q: torch.Tensor, heads_kv: int) -> torch.Tensor:
    """q [B, Hq, D] (one token a row) -> [B, Hkv, D] fp32 group means, heads summed in order."""
    b, hq, d = q.shape
    g = hq // heads_kv
    view = q.float().view(b, heads_kv, g, d)
    acc = view[:, :, 0].clone()
    for h in range(1, g):
        acc = acc + view[:, :, h]
    return acc / float(g)


def canonical_scores(queries: torch.Tensor, centroids: torch.Tensor, mode: str = "bf16") -> torch.Tensor:
    """queries [..., D] against centroids [..., N, D] (same leading dims) -> [..., N] fp32."""
    q, c = queries.float(), centroids.float()
    if mode == "bf16":
        q, c = bf16_round(q), bf16_round(c)
    d = q.shape[-1]
    span = d // PARTIALS
    prod = q.double()[..., None, :] * c.double()  # [..., N, D], exact products
    prod = prod.reshape(*prod.shape[:-1], PARTIALS, span)
    acc = prod[..., 0]
    for j in range(1, span):
        acc = acc + prod[..., j]
    a = acc[..., :8] + acc[..., 8:]
    b = a[..., :4] + a[..., 4:]
    t = b[..., :2] + b[..., 2:]
    return (t[..., 0] + t[..., 1]).float()


def ordered_bits(scores: torch.Tensor) -> torch.Tensor:
    bits = scores.contiguous().view(torch.int32)
    return bits ^ ((bits >> 31) & 0x7FFFFFFF)


def select(idx: torch.Tensor, centroids: torch.Tensor, members: torch.Tensor, positions: torch.Tensor,
           visible: torch.Tensor, *, top_p: int, top_k: int, window: int, sink: int,
           mode: str = "bf16") -> tuple[torch.Tensor, torch.Tensor]:
    """Flat select for U units at once: idx [U, D], centroids [U, N, D], members [U, N, cap],
    positions [U], visible [U] (buckets each unit may score) -> lists [U, top_k+window+sink]
    int32 (-1 padded), lengths [U] int32."""
    units, n = centroids.shape[0], centroids.shape[1]
    scores = canonical_scores(idx, centroids, mode)  # [U, N]
    col = torch.arange(n, dtype=torch.int64)
    keys = (ordered_bits(scores).to(torch.int64) << 32) | (0x7FFFFFFF - col)[None, :]
    keys = torch.where(col[None, :] < visible[:, None].to(torch.int64), keys, torch.full_like(keys, EMPTY))
    k = min(top_p, n)
    best = torch.topk(keys, k, dim=1, sorted=True).values
    picks = torch.where(best == EMPTY, torch.full_like(best, -1), 0x7FFFFFFF - (best & 0xFFFFFFFF))
    cap = members.shape[-1]
    rows = members.gather(1, picks.clamp_min(0)[..., None].expand(units, k, cap))  # [U, K, cap]
    rows = torch.where(picks[..., None] >= 0, rows, torch.full_like(rows, -1))
    pos = positions.to(torch.int64)
    wstart = (pos + 1 - window).clamp_min(0)
    ids = rows.reshape(units, k * cap).to(torch.int64)
    keep = (ids >= sink) & (ids < wstart[:, None])
    rank = torch.cumsum(keep.to(torch.int64), dim=1) - 1  # slot of each kept id, in rank order
    keep &= rank < top_k
    width = top_k + window + sink
    lists = torch.full((units, width + 1), -1, dtype=torch.int64)
    lists.scatter_(1, torch.where(keep, rank, torch.full_like(rank, width)), torch.where(keep, ids, -1))
    lists = lists[:, :width]
    kept = keep.sum(1)
    n_win = (pos + 1 - wstart).clamp_min(0)
    n_sink = torch.minimum(torch.full_like(wstart, sink), wstart)
    slot = torch.arange(width, dtype=torch.int64)[None, :] - kept[:, None]  # tail slot index
    tail = torch.where(slot < n_win[:, None], wstart[:, None] + slot, slot - n_win[:, None])
    in_tail = (slot >= 0) & (slot < (n_win + n_sink)[:, None])
    lists = torch.where(in_tail, tail, lists)
    return lists.to(torch.int32), (kept + n_win + n_sink).to(torch.int32)


def read(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lists: torch.Tensor, lengths: torch.Tensor,
         scale: float) -> torch.Tensor:
    """One decode token per row: q [B, Hq, D], k/v [B, T, Hkv, D], lists [B, Hkv, W], lengths
    [B, Hkv] -> out [B, Hq, D] fp32."""
    b_, hq, d = q.shape
    hkv = k.shape[2]
    g = hq // hkv
    out = torch.zeros(b_, hq, d, dtype=torch.float32)
    for b in range(b_):
        for h in range(hkv):
            n = int(lengths[b, h])
            sel = lists[b, h, :n].to(torch.int64)
            sel = sel[sel >= 0]
            if sel.numel() == 0:
                continue
            kk = k[b, sel, h].float()  # [n, D]
            vv = v[b, sel, h].float()
            qq = q[b, h * g:(h + 1) * g].float()  # [G, D]
            p = torch.softmax((qq @ kk.T) * scale, dim=-1)
            out[b, h * g:(h + 1) * g] = p @ vv
    return out


def decode_step(q, k, v, centroids, members, ends, positions, *, cluster_block_size: int, block_buckets: int,
                top_p: int, top_k: int, window: int, sink: int, scale: float, mode: str = "bf16"):
    """The whole decode step for B rows of one token: q [B, Hq, D], k/v [B, T, Hkv, D],
    tables per kv-head ([Hkv, N, ...]) or per row and kv-head ([B, Hkv, N, ...]); ends
    optional. Returns (lists [B, Hkv, W], lengths [B, Hkv], out [B, Hq, D])."""
    b_, hq, d = q.shape
    hkv = k.shape[2]
    idx = index_queries(q, hkv).reshape(b_ * hkv, d)
    lead = centroids.shape[:-2]
    if len(lead) == 1:
        centroids = centroids.expand(b_, *centroids.shape)
        members = members.expand(b_, *members.shape)
        ends = None if ends is None else ends.expand(b_, *ends.shape)
    n = centroids.shape[-2]
    cent = centroids.reshape(b_ * hkv, n, d)
    mem = members.reshape(b_ * hkv, n, members.shape[-1])
    pos = positions.to(torch.int64).repeat_interleave(hkv)
    if ends is None:
        vis = torch.div(pos, cluster_block_size, rounding_mode="floor") * block_buckets
        vis = vis.clamp(max=n)
    else:
        vis = (ends.reshape(b_ * hkv, n).to(torch.int64) <= (pos + 1)[:, None]).sum(1)
    lists, lengths = select(idx, cent, mem, pos, vis, top_p=top_p, top_k=top_k, window=window, sink=sink, mode=mode)
    lists, lengths = lists.view(b_, hkv, -1), lengths.view(b_, hkv)
    return lists, lengths, read(q, k, v, lists, lengths, scale)
