#!/usr/bin/env python3
"""Select+read benchmark on one MI355X: 32k bf16 decode µs/step + HBM GB/s, prefill tok/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Decode workload (the headline): D-LSA Flat at B=1, context 32768, Hq=32, Hkv=8, D=128,
bf16, keys from 512 Gaussian clusters per kv-head (sigma 0.3, runs of 16-128 tokens),
512 Ward-style buckets per kv-head (16-256 tokens, mean 64) with bucket-mean centroids,
top-32 buckets per kv-head, rank-order expansion, split-K sparse read. One step is what
a decode layer pays: GQA-collapsed index queries, the flat select and the sparse read
(reference port/bench.py:147-153 ``step``: select + read on a built index), here fused
into one kernel launch; the unfused three-launch composition is timed beside it.

Timing: the K timed steps are replayed from HIP graphs (one graph = a rotation of
``--rotate`` steps, each on its own resident copy of the cache, so consecutive steps
never find their K/V rows in the 256 MiB MALL) between ``torch.cuda.synchronize()``
brackets; ``value`` = wall µs per step. The step's kernel is also timed alone for the
roofline: a HIP graph of back-to-back launches over the rotation, HIP events around its
replays on the stream it runs on; algorithmic bytes (gathered K and V rows) / average
launch duration (which includes the dispatch gap, so it is an upper bound on the
kernel's own duration, which rocprofv3's kernel trace reports).

Comparators in the same run: dense decode on the same GPU and the same rotation (every
SDPA backend that runs, and this library's split-K read over the whole causal list; the
fastest is the comparator), the 32k chunked prefill as tok/s beside dense causal SDPA, a
plain device copy (achievable HBM bandwidth), and the torch CPU restatement of the step
(oracle/cpu_step.py) on every host core and on one, for the 32k decode and the 2k fp32
decode (a bounded sample; its lists are checked bit-exact against the GPU's). The numpy
oracle checks the timed step's lists (bit-exact) and read (bf16 bar).

One GPU only: ``--gpus N`` with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT / "latent-sparse-attention-rocm_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "32k bf16 decode select+read µs/step + HBM GB/s; prefill select+read tok/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
T_CTX, HQ, HKV, D = 32768, 32, 8, 128
N_BUCKETS = 512
CHUNK = 64


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class select_impl:
    """Sets LSA_SELECT_IMPL for a block and restores the caller's value after it."""

    def __init__(self, impl: str):
        self.impl, self.prev = impl, None

    def __enter__(self):
        self.prev = os.environ.get("LSA_SELECT_IMPL")
        os.environ["LSA_SELECT_IMPL"] = self.impl

    def __exit__(self, *exc):
        if self.prev is None:
            os.environ.pop("LSA_SELECT_IMPL", None)
        else:
            os.environ["LSA_SELECT_IMPL"] = self.prev


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=256, help="untimed decode steps first")
    ap.add_argument("--rotate", type=int, default=64, help="resident cache copies cycled through")
    ap.add_argument("--kernel-launches", type=int, default=512, help="event-timed read launches")
    ap.add_argument("--prefill-steps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-tree", action="store_true", help="skip the B=32 x 131k tree decode leg")
    ap.add_argument("--tree-steps", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-build", action="store_true", help="skip the bucket-table build leg")
    ap.add_argument("--no-paged", action="store_true", help="skip the paged-cache decode leg")
    ap.add_argument("--no-refcfg-prefill", action="store_true",
                    help="skip the reference-knob prefill leg (32768 per-row selections)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run 3 plain device copies of this many MiB (calibrates HBM byte counters)")
    return ap.parse_args()


# ----------------------------------------------------------------------------- workload


class DecodeCache:
    """One resident copy of everything a decode step reads."""

    def __init__(self, q_last, k, v, buckets, pos):
        self.q = q_last
        self.k = k
        self.v = v
        self.buckets = buckets
        self.pos = pos


def copy_cache(c: DecodeCache):
    from lsa_rocm_lab.port.pipeline import Buckets

    b = c.buckets
    nb = Buckets(b.centroids.clone(), b.members.clone(), b.sizes.clone(),
                 centroids_f32=None if b.centroids_f32 is None else b.centroids_f32.clone(),
                 ends=None if b.ends is None else b.ends.clone(), spans=b.spans, block_visible=b.block_visible)
    return DecodeCache(c.q.clone(), c.k.clone(), c.v.clone(), nb, c.pos.clone())


def decode_step(c: DecodeCache, config):
    """The decode step as one launch: group-mean index queries, flat select, sparse read."""
    from lsa_rocm_lab.port import pipeline

    out, lists, lengths = pipeline.flat_decode(c.q, c.k, c.v, c.pos, c.buckets, config, scale=D ** -0.5)
    return lists, lengths, out


def unfused_step(c: DecodeCache, config):
    """The same step as the reference composes it: index queries, flat select, sparse read
    (three launches)."""
    from lsa_rocm_lab.port import pipeline
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    idx = pipeline.index_queries(c.q, HKV)[0]  # [1, Hkv, D] fp32
    lists, lengths = pipeline.flat_select(idx, c.pos, c.buckets, config)
    out = sparse_read_auto(c.q, c.k, c.v, lists.unsqueeze(0), lengths.unsqueeze(0), D ** -0.5)
    return lists, lengths, out


def capture(fn, n: int, torch):
    """A HIP graph of fn(0..n-1); warm-up runs on a side stream first (torch's recipe)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


def run_steps(graphs, n_steps: int, per_graph: int, torch):
    """Replays exactly n_steps steps: full-rotation graphs, then the remainder graph."""
    full, rem = divmod(n_steps, per_graph)
    for _ in range(full):
        graphs["full"].replay()
    if rem:
        graphs[rem].replay()


def event_launch_times(fn, n: int, torch) -> list[float]:
    """Milliseconds between HIP events recorded right before and after each launch."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(evs):
        a.record()
        fn(i)
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


def profiled_traffic(kernel: str) -> int | None:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (profiles/decode_flat32k_pmc.md); None when it is absent."""
    path = ROOT / "profiles" / "decode_flat32k_pmc.md"
    if not path.is_file():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
            return int(line.split(":")[1])
    return None


def graph_launch_us(fn, n: int, replays: int, torch) -> float:
    """Average µs per launch of fn(0..n-1) replayed back to back from one HIP graph, timed
    with HIP events on the stream the graph runs on (kernel time plus the dispatch gap)."""
    g = capture(fn, n, torch)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (n * replays)


def dense_decode_fns(torch):
    """Dense SDPA decode over the whole cache, one per fused backend torch offers here (the
    math path is left out: it materializes the scores and is no attention kernel)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def make(backend, gqa):
        def fn(q, k, v):
            qq = q.permute(0, 2, 1, 3)
            if gqa:
                kk, vv = k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)
            else:
                kk = k.permute(0, 2, 1, 3).repeat_interleave(HQ // HKV, dim=1)
                vv = v.permute(0, 2, 1, 3).repeat_interleave(HQ // HKV, dim=1)
            with sdpa_kernel([backend]):
                return F.scaled_dot_product_attention(qq, kk, vv, scale=D ** -0.5, enable_gqa=gqa)
        return fn

    return [("sdpa_flash+gqa", make(SDPBackend.FLASH_ATTENTION, True)),
            ("sdpa_efficient+gqa", make(SDPBackend.EFFICIENT_ATTENTION, True)),
            ("sdpa_flash+expanded_kv", make(SDPBackend.FLASH_ATTENTION, False)),
            ("sdpa_efficient+expanded_kv", make(SDPBackend.EFFICIENT_ATTENTION, False))]


def dense_leg(caches, R, us_step, torch):
    """Dense decode comparators on the same rotation: every SDPA backend that runs, and
    this library's own split-K read over the whole causal list (ids 0..T-1 per kv-head,
    the dense attention this GPU can do with the same kernel). Each is a HIP graph of R
    steps over the resident copies, wall-clock timed; the fastest is the comparator."""
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    rows = {}
    for name, fn in dense_decode_fns(torch):
        try:
            fn(caches[0].q, caches[0].k, caches[0].v)
            torch.cuda.synchronize()
        except RuntimeError as exc:
            log(f"dense {name} unavailable: {str(exc).splitlines()[0][:120]}")
            continue
        rows[name] = lambda i, fn=fn: fn(caches[i % R].q, caches[i % R].k, caches[i % R].v)
    ids = torch.arange(T_CTX, device="cuda", dtype=torch.int32).view(1, 1, T_CTX)
    full = torch.full((1, 1), T_CTX, device="cuda", dtype=torch.int32)
    rows["lsa_read_dense"] = lambda i: sparse_read_auto(caches[i % R].q, caches[i % R].k, caches[i % R].v, ids,
                                                        full, D ** -0.5)
    out = {}
    for name, dfn in rows.items():
        event_launch_times(dfn, 8, torch)
        try:
            g = capture(dfn, R, torch)
            n_rep = max(1, 256 // R)
            g.replay()
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            for _ in range(n_rep):
                g.replay()
            torch.cuda.synchronize()
            us = (time.perf_counter() - w0) / (n_rep * R) * 1e6
            how = "graph"
        except RuntimeError as exc:
            log(f"dense {name}: graph capture failed ({str(exc).splitlines()[0][:80]}); event-timed launches")
            us = statistics.mean(event_launch_times(dfn, 128, torch)) * 1e3
            how = "events"
        out[name] = {"us_per_step": round(us, 3), "timing": how,
                     "gbps": round(2 * T_CTX * HKV * D * 2 / (us * 1e-6) / 1e9, 1)}
    best = min(out, key=lambda n: out[n]["us_per_step"])
    log(f"dense decode: {out}")
    return {"backends": out, "fastest": best, "us_per_step": out[best]["us_per_step"],
            "kv_bytes": 2 * T_CTX * HKV * D * 2,
            "speedup_vs_fastest": round(out[best]["us_per_step"] / us_step, 3),
            "meets_3x": bool(out[best]["us_per_step"] / us_step >= 3.0)}


def copy_leg(torch, mib: int = 1024):
    """Achievable HBM bandwidth on this box: a device-to-device copy of `mib` MiB (read +
    write bytes / time), median of event-timed copies."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    times = event_launch_times(lambda i: dst.copy_(src), 9, torch)
    ms = statistics.median(times)
    del src, dst
    return {"bytes_moved": 2 * (mib << 20), "ms": round(ms, 4), "gbps": round(2 * (mib << 20) / (ms * 1e-3) / 1e9, 1)}


# ----------------------------------------------------------------------------- block-sparse decode


def block_sparse_leg(args, torch, np):
    """The positional block-sparse arm (context 32768, 512 blocks of 64 with block-mean
    centroids, top-33 blocks + a 128-token window + 64 sink tokens: 34 blocks a kv-head)
    through the fused decode kernel, rotating 16 resident cache copies."""
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline

    q, k, v = workloads.geometry(T_CTX, HQ, HKV, D, dtype=torch.bfloat16, seed=0, device="cuda")
    config = workloads.BLOCK_SPARSE_32K
    buckets = pipeline.position_buckets(k, config, centroid="mean")
    pos = torch.tensor([T_CTX - 1], device="cuda", dtype=torch.int32)
    base = DecodeCache(q[:, -1:].contiguous(), k, v, buckets, pos)
    R = 16
    caches = [base] + [copy_cache(base) for _ in range(R - 1)]
    _, lengths, _ = decode_step(base, config)
    torch.cuda.synchronize()
    gathered = int(lengths.to(torch.int64).sum().item()) * D * 2 * 2
    us = graph_launch_us(lambda i: decode_step(caches[i % R], config), R, max(1, args.kernel_launches // R), torch)
    gbps = gathered / (us * 1e-6) / 1e9
    log(f"block-sparse decode {us:.2f} us per step ({gbps:.0f} GB/s on {gathered} gathered bytes)")
    return {"workload": "block_sparse_decode_32k", "blocks_per_kv_head": 34,
            "tokens_read": lengths.cpu().numpy().tolist(), "us_per_step": round(us, 3),
            "gathered_bytes": gathered, "gbps": round(gbps, 1), "roofline_frac": round(gbps / HBM_PEAK_GBS, 4)}


# ----------------------------------------------------------------------------- batched flat decode


def batched_flat_leg(args, torch, np):
    """The fused decode kernel in its bandwidth regime: B=32 sequences x 32768 tokens, Hq 32
    / Hkv 8, D 128 bf16, 512 clustered Ward buckets per (sequence, kv-head), top-32 buckets:
    one launch a step, rotating over 4 query tokens (the 4.3 GB cache is far beyond the MALL).
    Reports gathered bytes / launch time against the 8 TB/s peak; lists checked bit-exact
    against the unfused select on every (sequence, kv-head)."""
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline

    B, T, NQ = 32, 32768, 4
    data = workloads.clustered(T, HQ, HKV, D, n_clusters=512, seed=3, B=B, device="cuda", gen_device="cuda",
                               q_tokens=NQ)
    buckets = workloads.cluster_buckets(data, target=N_BUCKETS, workers=16)
    config = workloads.FLAT_32K
    pos = torch.full((B,), T - 1, device="cuda", dtype=torch.int32)
    qs = [data.q[:, i:i + 1].contiguous() for i in range(NQ)]

    def step(i):
        out, lists, lengths = pipeline.flat_decode(qs[i % NQ], data.k, data.v, pos, buckets, config, scale=D ** -0.5)
        return lists, lengths, out

    res = [step(i) for i in range(NQ)]
    torch.cuda.synchronize()
    toks = [int(r[1].to(torch.int64).sum().item()) for r in res]
    gathered = statistics.mean(toks) * D * 2 * 2
    us = graph_launch_us(step, NQ, max(1, args.tree_steps // NQ), torch)
    gbps = gathered / (us * 1e-6) / 1e9
    idx = pipeline.index_queries(qs[0], HKV)[:, 0]
    with select_impl("fused"):
        l2, n2 = pipeline.flat_select(idx, pos, buckets, config)
    same = bool(torch.equal(l2, res[0][0]) and torch.equal(n2, res[0][1]))
    log(f"batched flat decode B={B}: {us:.1f} us/step, {gbps:.0f} GB/s on {gathered / 1e6:.1f} MB gathered")
    del data
    return {"workload": "flat_decode_32k_b32", "batch": B, "context": T, "us_per_step": round(us, 2),
            "gathered_bytes": int(gathered), "gbps": round(gbps, 1), "roofline_frac": round(gbps / HBM_PEAK_GBS, 4),
            "lists_equal_unfused_select": same}


# ----------------------------------------------------------------------------- tree decode


def tree_decode_leg(args, torch, np):
    """Batched tree decode (B=32, context 131072, 2048 buckets = 128 nodes x 16 per
    sequence and kv-head, top-8 nodes then top-32 of their children): index queries + tree
    select + split read per step, rotating over 4 query tokens so that consecutive steps
    gather different rows (the 17 GB cache is far beyond the 256 MB MALL anyway)."""
    import oracle
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    B, T, NQ = 32, 131072, 4
    t0 = time.perf_counter()
    data = workloads.clustered(T, HQ, HKV, D, n_clusters=2048, seed=0, B=B, device="cuda", gen_device="cuda",
                               q_tokens=NQ)
    buckets = workloads.cluster_buckets(data, target=2048, workers=16)
    tree = workloads.node_tree(buckets, node_size=16)
    config = workloads.TREE_131K
    torch.cuda.synchronize()
    log(f"tree workload built in {time.perf_counter() - t0:.1f}s "
        f"(K/V {2 * data.k.numel() * 2 / 1e9:.1f} GB)")
    pos = torch.full((B,), T - 1, device="cuda", dtype=torch.int32)
    qs = [data.q[:, i:i + 1].contiguous() for i in range(NQ)]

    def step(i):
        q = qs[i % NQ]
        idx = pipeline.index_queries(q, HKV)[:, 0]  # [B, Hkv, D]
        lists, lengths = pipeline.tree_select(idx, pos, buckets, tree, config, score_dtype="bf16")
        out = sparse_read_auto(q, data.k, data.v, lists.unsqueeze(1), lengths.unsqueeze(1), D ** -0.5)
        return lists, lengths, out

    res = [step(i) for i in range(NQ)]
    torch.cuda.synchronize()
    toks = [int(r[1].to(torch.int64).sum().item()) for r in res]
    gathered = statistics.mean(toks) * D * 2 * 2
    g = capture(step, NQ, torch)
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, args.tree_steps // NQ)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = (time.perf_counter() - w0) / (reps * NQ) * 1e6
    dev_us = e0.elapsed_time(e1) * 1e3 / (reps * NQ)
    # the kernels alone
    idxs = [pipeline.index_queries(q, HKV)[:, 0] for q in qs]
    sel_us = graph_launch_us(lambda i: pipeline.tree_select(idxs[i % NQ], pos, buckets, tree, config,
                                                            score_dtype="bf16"), NQ, reps, torch)
    read_us = graph_launch_us(lambda i: sparse_read_auto(qs[i % NQ], data.k, data.v, res[i % NQ][0].unsqueeze(1),
                                                         res[i % NQ][1].unsqueeze(1), D ** -0.5), NQ, reps, torch)
    read_gbps = gathered / (read_us * 1e-6) / 1e9
    log(f"tree decode {us:.1f} us/step (select {sel_us:.1f} + read {read_us:.1f} us); read {read_gbps:.0f} GB/s "
        f"on {gathered / 1e6:.1f} MB gathered")
    # the same step in one launch (the tree select role in the fused decode kernel)
    fused = lambda i: pipeline.tree_decode(qs[i % NQ], data.k, data.v, pos, buckets, tree, config)
    f0 = fused(0)
    torch.cuda.synchronize()
    fused_same = bool(torch.equal(f0[1], res[0][0]) and torch.equal(f0[2], res[0][1]))
    fused_err = float((f0[0].float() - res[0][2].float()).abs().max().item())
    fused_us = graph_launch_us(fused, NQ, reps, torch)
    log(f"fused tree decode {fused_us:.1f} us/step ({gathered / (fused_us * 1e-6) / 1e9:.0f} GB/s); lists equal: "
        f"{fused_same}")
    # dense SDPA decode over the whole 17 GB cache
    dense_us = None
    try:
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel

        kk, vv = data.k.permute(0, 2, 1, 3), data.v.permute(0, 2, 1, 3)

        def dfn(i):
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                return F.scaled_dot_product_attention(qs[i % NQ].permute(0, 2, 1, 3), kk, vv, scale=D ** -0.5,
                                                      enable_gqa=True)

        dfn(0)
        torch.cuda.synchronize()
        dense_us = statistics.median(event_launch_times(dfn, 5, torch)) * 1e3
    except RuntimeError as exc:
        log(f"dense tree decode unavailable: {str(exc).splitlines()[0][:120]}")
    # parity sample: two (sequence, kv-head) selections and sequence 0's read vs the oracle
    lists0, lengths0, out0 = res[0]
    lvl = tree.levels[0]
    idx0 = idxs[0]
    exact = True
    for b, gg in ((0, 0), (B - 1, HKV - 1)):
        l, n, _ = oracle.tree_select_row(
            idx0[b, gg].float().cpu().numpy(), lvl.centroids_bf16[b, gg].float().cpu().numpy(),
            lvl.children[b, gg].cpu().numpy(), buckets.centroids[b, gg].float().cpu().numpy(),
            buckets.members[b, gg].cpu().numpy(), T - 1, visible=buckets.rows,
            node_block=config.node_cluster_block_size,
            beam_width=config.beam_width, top_p=config.top_p, top_k=config.top_k, window=0, sink=0, mode="bf16")
        exact &= bool(np.array_equal(lists0[b, gg].cpu().numpy(), l)) and int(lengths0[b, gg]) == n
    k0, v0 = data.k[:1].float().cpu().numpy(), data.v[:1].float().cpu().numpy()
    want = oracle.sparse_read(qs[0][:1].float().cpu().numpy(), k0, v0, lists0[:1, None].cpu().numpy(),
                              lengths0[:1, None].cpu().numpy(), D ** -0.5)
    err = np.abs(out0[:1].float().cpu().numpy() - want)
    del k0, v0, data
    return {"workload": "tree_decode_131k_b32", "batch": B, "context": T, "buckets": 2048, "nodes": 128,
            "beam": config.beam_width, "top_buckets": config.top_p, "us_per_step": round(us, 2),
            "device_us_per_step": round(dev_us, 2), "select_us": round(sel_us, 2), "read_us": round(read_us, 2),
            "gathered_bytes": int(gathered), "read_gbps": round(read_gbps, 1),
            "read_roofline_frac": round(read_gbps / HBM_PEAK_GBS, 4),
            "step_gbps": round(gathered / (us * 1e-6) / 1e9, 1),
            "fused_us_per_step": round(fused_us, 2),
            "fused_gbps": round(gathered / (fused_us * 1e-6) / 1e9, 1),
            "fused_roofline_frac": round(gathered / (fused_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "fused_lists_equal": fused_same, "fused_vs_unfused_read_max_abs": fused_err,
            "dense_us": None if dense_us is None else round(dense_us, 1),
            "speedup_vs_dense": None if dense_us is None else round(dense_us / us, 2),
            "parity": {"lists_bit_exact_sampled": exact, "read_max_abs": float(err.max()),
                       "read_mean_abs": float(err.mean())}}


# ----------------------------------------------------------------------------- reference knobs


def refcfg_decode_leg(args, torch, np, dense_us):
    """The reference's own decode arms at its default knobs (pipeline.py:32-54: blocks of
    512 keys, buckets of 8 keys cap 16 (64 a block), top_p 1024, top_k 4096, window 512,
    sink 4; tree: node size 4, node blocks of 64, 3 levels, beam 64) on its benchmark
    geometry (port/bench.py:75-81, :113-153: B=1, 32k, Hq 32 / Hkv 8, D 128 bf16, q/k/v ~
    0.2 N(0,1); one index-space table shared by every head). Index keys / queries: the
    mean over the key / query heads (a stand-in for upstream's regroup). Flat: the fused
    select (bf16 scores) + the split-K read; tree: the hierarchy of 1024/256/64 nodes, the
    multi-level beam (fp32 scores) + the same read. Each step rotates over the last 4 query
    tokens (positions T-4 .. T-1). Each arm's step is one fused launch with the selection
    shared by every kv-head (flat_decode_shared / tree_decode_shared); the select kernel
    followed by the read is timed beside it (two_launch). Lists of both bit-exact against
    the numpy oracle on all 4 tokens, reads within the bf16 bar on one."""
    import oracle
    from lsa_rocm_lab.port import pipeline
    from lsa_rocm_lab.port.pipeline import PortConfig
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    config = PortConfig()
    T, NQ = T_CTX, 4
    gen = torch.Generator(device="cuda").manual_seed(20261105)
    q, k, v = ((torch.randn(1, T, h, D, device="cuda", generator=gen) * 0.2).to(torch.bfloat16)
               for h in (HQ, HKV, HKV))
    idx_k = pipeline.index_queries(k, 1)[0, :, 0].contiguous()          # [T, D]
    idx_q = pipeline.index_queries(q[:, -NQ:], 1)[0, :, 0].contiguous()  # [NQ, D]
    buckets = pipeline.build_buckets(idx_k, config)
    tree = pipeline.build_hierarchy_gpu(idx_k, buckets, config)
    pos = torch.arange(T - NQ, T, device="cuda", dtype=torch.int32)
    qs = [q[:, T - NQ + i:T - NQ + i + 1].contiguous() for i in range(NQ)]
    sel = {"flat": lambda i: pipeline.flat_select(idx_q[i:i + 1], pos[i:i + 1], buckets, config),
           "tree": lambda i: pipeline.tree_select(idx_q[i:i + 1], pos[i:i + 1], buckets, tree, config)}
    out = {}
    reps = max(1, args.tree_steps // NQ)
    for name, fn in sel.items():
        res = [fn(i) for i in range(NQ)]
        torch.cuda.synchronize()

        def step(i, fn=fn):
            lists, lengths = fn(i % NQ)
            return sparse_read_auto(qs[i % NQ], k, v, lists[None], lengths[None], D ** -0.5)

        read = lambda i, res=res: sparse_read_auto(qs[i % NQ], k, v, res[i % NQ][0][None], res[i % NQ][1][None],
                                                   D ** -0.5)
        sel_us = graph_launch_us(lambda i, fn=fn: fn(i % NQ), NQ, reps, torch)
        read_us = graph_launch_us(read, NQ, reps, torch)
        step_us = graph_launch_us(step, NQ, reps, torch)
        toks = statistics.mean(int(r[1][0]) for r in res)
        gathered = toks * HKV * D * 2 * 2
        # parity: the four rows' lists against the oracle, row 0's read against the fp64 read
        lists_np = np.stack([r[0][0].cpu().numpy() for r in res])
        lengths_np = np.array([int(r[1][0]) for r in res])
        members = buckets.members.cpu().numpy()
        if name == "flat":
            want_l, want_n = oracle.flat_select(idx_q.cpu().numpy(), pos.cpu().numpy(),
                                                buckets.centroids.float().cpu().numpy(), members,
                                                cluster_block_size=config.cluster_block_size,
                                                block_buckets=config.block_bucket_count, top_p=config.top_p,
                                                top_k=config.top_k, window=config.window_size,
                                                sink=config.sink_size, mode="bf16")
        else:
            levels = [(lv.centroids.cpu().numpy(), lv.children.cpu().numpy()) for lv in tree.levels]
            vis = oracle.visible_counts(pos.cpu().numpy(), buckets.rows, config.cluster_block_size,
                                        config.block_bucket_count)
            rows = [oracle.beam_select_row(idx_q[i].cpu().numpy(), levels, buckets.centroids_f32.cpu().numpy(),
                                           members, int(pos[i]), int(vis[i]), config.node_bucket_size,
                                           config.node_cluster_block_size, config.top_level, config.beam_width,
                                           config.top_p, config.top_k, config.window_size, config.sink_size,
                                           mode="fp32") for i in range(NQ)]
            want_l, want_n = np.stack([r[0] for r in rows]), np.array([r[1] for r in rows])
        o0 = step(0)
        want = oracle.sparse_read(qs[0].float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                  lists_np[None, :1], lengths_np[None, :1], D ** -0.5)
        err = np.abs(o0.float().cpu().numpy() - want)
        two = {"select_us": round(sel_us, 2), "read_us": round(read_us, 2), "us_per_step": round(step_us, 2),
               "read_gbps": round(gathered / (read_us * 1e-6) / 1e9, 1),
               "speedup_vs_dense": None if dense_us is None else round(dense_us / step_us, 2),
               "lists_bit_exact": bool(np.array_equal(lists_np, want_l) and np.array_equal(lengths_np, want_n)),
               "read_max_abs": float(err.max()), "read_mean_abs": float(err.mean())}
        # the production step: one launch, select workgroups + readers sharing the selection
        if name == "flat":
            fused = lambda i: pipeline.flat_decode_shared(qs[i % NQ], k, v, idx_q[i % NQ:i % NQ + 1],
                                                          pos[i % NQ:i % NQ + 1], buckets, config)
        else:
            fused = lambda i: pipeline.tree_decode_shared(qs[i % NQ], k, v, idx_q[i % NQ:i % NQ + 1],
                                                          pos[i % NQ:i % NQ + 1], buckets, tree, config)
        fres = [fused(i) for i in range(NQ)]
        torch.cuda.synchronize()
        fused_us = graph_launch_us(fused, NQ, reps, torch)
        f_lists = np.stack([r[1][0].cpu().numpy() for r in fres])
        f_lengths = np.array([int(r[2][0]) for r in fres])
        ferr = np.abs(fres[0][0].float().cpu().numpy() - want)
        out[name] = {"us_per_step": round(fused_us, 2), "tokens_read": round(toks, 1),
                     "gbps": round(gathered / (fused_us * 1e-6) / 1e9, 1),
                     "speedup_vs_dense": None if dense_us is None else round(dense_us / fused_us, 2),
                     "lists_bit_exact": bool(np.array_equal(f_lists, want_l) and np.array_equal(f_lengths, want_n)),
                     "read_max_abs": float(ferr.max()), "read_mean_abs": float(ferr.mean()),
                     "two_launch": two}
        log(f"refcfg {name} decode {out[name]}")
    return {"workload": "refcfg_decode_32k", "batch": 1, "context": T, "buckets": buckets.rows,
            "nodes": [lv.centroids.shape[0] for lv in tree.levels], "knobs": "reference PortConfig defaults",
            "timing": "hip graphs of back-to-back steps over 4 query tokens, HIP events",
            "step": "one launch, the selection shared by every kv-head (lsa_decode_shared / "
                    "lsa_decode_tree_shared); two_launch: the select kernel then the split-K read", **out}


def refcfg_prefill_leg(args, torch, np, dense_ms):
    """The reference's own prefill arm at its default knobs (port/bench.py:113-154 with
    phase="prefill": every query row selects its own keys, then the per-row read; PortConfig
    defaults, pipeline.py:32-54: 512-key blocks of 64 buckets of at most 16 keys, top_p 1024
    of up to 4096 visible buckets, top_k 4096, window 512, sink 4, one index-space table
    shared by every head) on its benchmark geometry at 32k with Hq 32 / Hkv 8, D 128 bf16.
    A step is the fused select of all 32768 rows (lists [32768, 4612]) and the split-K
    read of every row's list for every head (the lists are shared by the heads). Timed by
    HIP events around whole steps (median of --prefill-steps) and each stage alone; the
    dense comparator is causal flash SDPA on the same tensors. Lists of 16 sampled rows
    bit-exact against the oracle, two rows' read within the bf16 bar."""
    import oracle
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline
    from lsa_rocm_lab.port.pipeline import PortConfig
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    cfg = PortConfig()
    T = T_CTX
    ws = workloads.index_space(T)
    pos = torch.arange(T, device="cuda", dtype=torch.int32)
    scale = D ** -0.5

    def select():
        return pipeline.flat_select(ws.idx_q, pos, ws.buckets, cfg)

    def step():
        lists, lengths = select()
        return sparse_read_auto(ws.q, ws.k, ws.v, lists[None], lengths[None], scale), lists, lengths

    out, lists, lengths = step()
    torch.cuda.synchronize()
    n = max(1, args.prefill_steps)
    step_ms = statistics.median(event_launch_times(lambda i: step(), n, torch))
    sel_ms = statistics.median(event_launch_times(lambda i: select(), n, torch))
    read_ms = statistics.median(event_launch_times(
        lambda i: sparse_read_auto(ws.q, ws.k, ws.v, lists[None], lengths[None], scale), n, torch))
    keys = float(lengths.to(torch.float64).sum().item())
    gathered = keys * HKV * D * 2 * 2  # K and V rows of every kv-head, bf16
    flops = 4.0 * D * keys * HQ
    rows = [0, 511, 512, 1024, 4096, 8191, 12345, 16384, 20000, 24576, 28000, 30000, 32255, 32256, 32700, 32767]
    want_l, want_n = oracle.flat_select(ws.idx_q[rows].cpu().numpy(), np.array(rows),
                                        ws.buckets.centroids.float().cpu().numpy(), ws.buckets.members.cpu().numpy(),
                                        cluster_block_size=cfg.cluster_block_size,
                                        block_buckets=cfg.block_bucket_count, top_p=cfg.top_p, top_k=cfg.top_k,
                                        window=cfg.window_size, sink=cfg.sink_size, mode="bf16")
    exact = bool(np.array_equal(lists[rows].cpu().numpy(), want_l)
                 and np.array_equal(lengths[rows].cpu().numpy(), want_n))
    two = [4096, 32767]
    want = oracle.sparse_read(ws.q[:, two].float().cpu().numpy(), ws.k.float().cpu().numpy(),
                              ws.v.float().cpu().numpy(), lists[two].cpu().numpy()[None],
                              lengths[two].cpu().numpy()[None], scale)
    err = np.abs(out[:, two].float().cpu().numpy() - want)
    res = {"workload": "refcfg_prefill_32k", "batch": 1, "context": T, "heads_q": HQ, "heads_kv": HKV, "head_dim": D,
           "knobs": "reference PortConfig defaults", "buckets": ws.buckets.rows, "list_width": int(lists.shape[1]),
           "ms_per_step": round(step_ms, 3), "tok_per_s": round(T / (step_ms * 1e-3), 1),
           "select_ms": round(sel_ms, 3), "read_ms": round(read_ms, 3),
           "keys_per_row": round(keys / T, 1), "read_gathered_bytes": gathered,
           "read_gbps": round(gathered / (read_ms * 1e-3) / 1e9, 1),
           "read_tflops": round(flops / (read_ms * 1e-3) / 1e12, 2),
           "dense_sdpa_ms": None if dense_ms is None else round(dense_ms, 3),
           "speedup_vs_dense": None if dense_ms is None else round(dense_ms / step_ms, 3),
           "reference_gfx1151_ms": 347.086,
           "timing": f"HIP events around whole steps, median of {n}",
           "parity": {"lists_bit_exact_sampled": exact, "rows_checked": len(rows), "read_max_abs": float(err.max()),
                      "read_mean_abs": float(err.mean())}}
    log(f"refcfg prefill {res}")
    del ws
    return res


def paged_decode_leg(args, torch, np, caches, R, config, lists0, lengths0, out0):
    """The headline decode over a paged cache: every rotation copy's K/V moved into one pool
    of 16-token pages in shuffled order (and of single tokens: page 1), the slot table
    handed to the same fused kernel (the expansion maps every listed id once; the gather
    reads pool rows). A/B against the unpaged step in the same process, each a HIP graph of
    back-to-back steps over the rotation; lists checked against the unpaged lists mapped
    through the table, outputs equal to the unpaged step's."""
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline

    reps = max(1, args.kernel_launches // R)
    base_us = graph_launch_us(lambda i: decode_step(caches[i % R], config), R, reps, torch)
    res = {"workload": "flat_decode_32k_paged", "unpaged_us_per_step": round(base_us, 3)}
    t = lists0[0].cpu().numpy()
    for page in (16, 1):
        pools = [workloads.paged(c.k, c.v, page=page, seed=page) for c in caches]

        def step(i, pools=pools):
            c, pc = caches[i % R], pools[i % R]
            return pipeline.flat_decode(c.q, pc.k, pc.v, c.pos, c.buckets, config, scale=D ** -0.5,
                                        slot_table=pc.slot_table)

        out1, l1, n1 = step(0)
        torch.cuda.synchronize()
        table = pools[0].slot_table[0].cpu().numpy()
        n = lengths0[0].cpu().numpy()
        want = np.full_like(t, -1)
        for g in range(t.shape[0]):
            want[g, : n[g]] = table[t[g, : n[g]]]
        same = bool(np.array_equal(l1[0].cpu().numpy(), want) and torch.equal(n1, lengths0)
                    and torch.equal(out1, out0))
        us = graph_launch_us(step, R, reps, torch)
        res[f"page{page}"] = {"us_per_step": round(us, 3), "vs_unpaged": round(us / base_us, 4),
                              "lists_are_mapped_unpaged_lists_and_outputs_equal": same}
        log(f"paged decode page {page}: {us:.2f} us/step against {base_us:.2f} unpaged; exact {same}")
        del pools
    return res


# ----------------------------------------------------------------------------- config 1 and the CPU


def decode_2k_leg(args, torch, np):
    """The CPU-runnable decode config on the GPU: B=1, context 2048, Hq 8 / Hkv 2, D 64, fp32,
    q/k/v ~ N(0, 1) seed 0, positional blocks of 64 with block-mean centroids, top-7 blocks
    + the last block as the window + block 0 as the sinks (8 blocks, 512 tokens a kv-head).
    One fused decode launch a step, graph-replayed over 16 resident copies; lists checked
    bit-exact and the read within the fp32 bar (1e-4) against the numpy oracle."""
    import oracle
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline

    T, Hq, Hkv, Dh = 2048, 8, 2, 64
    q, k, v = workloads.geometry(T, Hq, Hkv, Dh, dtype=torch.float32, seed=0, device="cuda")
    config = workloads.DECODE_2K
    buckets = pipeline.position_buckets(k, config, centroid="mean")
    pos = torch.tensor([T - 1], device="cuda", dtype=torch.int32)
    base = DecodeCache(q[:, -1:].contiguous(), k, v, buckets, pos)
    R = 16
    caches = [base] + [copy_cache(base) for _ in range(R - 1)]

    def step(i):
        c = caches[i % R]
        out, lists, lengths = pipeline.flat_decode(c.q, c.k, c.v, c.pos, c.buckets, config, scale=Dh ** -0.5,
                                                   score_dtype="fp32")
        return lists, lengths, out

    lists, lengths, out = step(0)
    torch.cuda.synchronize()
    us = graph_launch_us(step, R, max(1, args.kernel_launches // R), torch)
    q_np, k_np, v_np = base.q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    idx = oracle.index_queries(q_np, Hkv)[0, 0]
    cents, mem = buckets.centroids_f32.cpu().numpy(), buckets.members.cpu().numpy()
    ls, ns = [], []
    for g in range(Hkv):
        l, n = oracle.flat_select(idx[g][None], np.array([T - 1]), cents[g], mem[g],
                                  cluster_block_size=config.cluster_block_size, block_buckets=config.block_bucket_count,
                                  top_p=config.top_p, top_k=config.top_k, window=config.window_size,
                                  sink=config.sink_size, mode="fp32")
        ls.append(l[0])
        ns.append(n[0])
    ls, ns = np.stack(ls), np.array(ns)
    want = oracle.sparse_read(q_np, k_np, v_np, ls[None, None], ns[None, None], Dh ** -0.5)
    err = np.abs(out.cpu().numpy() - want)
    return {"workload": "decode_2k_fp32", "context": T, "heads_q": Hq, "heads_kv": Hkv, "head_dim": Dh,
            "dtype": "fp32", "tokens_read": lengths.cpu().numpy().tolist(), "gpu_us_per_step": round(us, 3),
            "parity": {"lists_bit_exact": bool(np.array_equal(lists[0].cpu().numpy(), ls)),
                       "lengths_bit_exact": bool(np.array_equal(lengths[0].cpu().numpy(), ns)),
                       "read_max_abs": float(err.max()), "read_mean_abs": float(err.mean())},
            "_inputs": (base, config)}


def cpu_model() -> str:
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def time_cpu(fn, budget_s: float, min_reps: int = 3, warmup: int = 1) -> tuple[float, float, int]:
    """(p50, p95) seconds and the count of fn() calls that fit in budget_s, after warmup."""
    for _ in range(warmup):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_reps:
        c0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - c0)
    times.sort()
    return times[len(times) // 2], times[min(len(times) - 1, int(0.95 * len(times)))], len(times)


def cpu_leg(args, torch, base, data, buckets, config, lists0, lengths0, c1):
    """The pure-torch CPU restatement of the decode step (oracle/cpu_step.py: index queries,
    canonical scores, top-k, rank-order expansion, gather attention, whole-tensor ops) on
    the host: every core the process may use (torch.set_num_threads), then one thread, for
    the 32k flat decode and the 2k fp32 decode. Its lists are checked bit-exact against the
    GPU's. A bounded sample: about args.cpu_seconds of CPU work in all."""
    import os

    from oracle import cpu_step

    cores = len(os.sched_getaffinity(0))
    budget = args.cpu_seconds / 4.0
    k_cpu, v_cpu = data.k.cpu(), data.v.cpu()
    q_cpu = base.q[:, 0].cpu()
    cent, mem, ends = buckets.centroids.cpu(), buckets.members.cpu(), buckets.ends.cpu()
    pos = torch.tensor([T_CTX - 1])

    def flat():
        return cpu_step.decode_step(q_cpu, k_cpu, v_cpu, cent, mem, ends, pos,
                                    cluster_block_size=config.cluster_block_size,
                                    block_buckets=config.block_bucket_count, top_p=config.top_p, top_k=config.top_k,
                                    window=config.window_size, sink=config.sink_size, scale=D ** -0.5, mode="bf16")

    b1, cfg1 = c1["_inputs"]
    q1, k1, v1 = b1.q[:, 0].cpu(), b1.k.cpu(), b1.v.cpu()
    cent1, mem1 = b1.buckets.centroids_f32.cpu(), b1.buckets.members.cpu()
    pos1 = torch.tensor([b1.k.shape[1] - 1])

    def small():
        return cpu_step.decode_step(q1, k1, v1, cent1, mem1, None, pos1, cluster_block_size=cfg1.cluster_block_size,
                                    block_buckets=cfg1.block_bucket_count, top_p=cfg1.top_p, top_k=cfg1.top_k,
                                    window=cfg1.window_size, sink=cfg1.sink_size, scale=64 ** -0.5, mode="fp32")

    prev = torch.get_num_threads()
    res = {}
    try:
        for threads in (cores, 1):
            torch.set_num_threads(threads)
            res[threads] = (time_cpu(flat, budget), time_cpu(small, budget))
    finally:
        torch.set_num_threads(prev)
    ls, ns, _ = flat()
    same = bool(torch.equal(ls[0], lists0[0].cpu()) and torch.equal(ns[0], lengths0[0].cpu()))
    (f50, f95, fn), (s50, s95, sn) = res[cores]
    (f50_1, _, _), (s50_1, _, _) = res[1]
    c1["cpu_us_per_step"] = round(s50 * 1e6, 1)
    c1["cpu_cores"] = cores
    return {"value": round(f50 * 1e6, 1), "unit": "us/step", "cores": cores, "kind": "port",
            "model": cpu_model(), "p95_us": round(f95 * 1e6, 1), "one_thread_us": round(f50_1 * 1e6, 1),
            "lists_bit_exact_vs_gpu": same,
            "decode_2k_fp32": {"us_per_step": round(s50 * 1e6, 1), "p95_us": round(s95 * 1e6, 1),
                               "one_thread_us": round(s50_1 * 1e6, 1), "steps": sn},
            "sample": f"{fn} flat_decode_32k steps and {sn} decode_2k_fp32 steps of the torch CPU restatement "
                      f"(oracle/cpu_step.py) at {cores} threads, the same at 1 thread; median (p50)"}


# ----------------------------------------------------------------------------- main


def bucket_build_leg(args, torch):
    """The index build before the path: contiguous Ward-style segments of the 32k cache's
    keys (8 kv-heads, pools of 16 -> 512 buckets of at most 256 positions each), the pool
    sums and the greedy merge on the GPU (build.hip). One workgroup per table runs the
    1536 dependent merges, so the leg is latency-bound; it reports time per merge step."""
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline

    T, POOL, TARGET, CAP = 32768, 16, 512, 256
    data = workloads.clustered(T, HQ, HKV, D, n_clusters=512, seed=1, device="cuda")
    first = pipeline.segment_starts(data.k, TARGET, POOL, CAP)
    times = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        again = pipeline.segment_starts(data.k, TARGET, POOL, CAP)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    ms = sorted(times)[len(times) // 2]
    merges = T // POOL - TARGET
    # in-place growth during decode: reference-knob block tables (512-key blocks of 64
    # buckets of at most 16 keys, 8 kv-heads) reserved for 64k keys; the step that closes
    # the last block of the 32k cache builds its 64 rows a table into the reserved rows
    cfg = pipeline.PortConfig()
    tabs = pipeline.reserve_buckets(pipeline.build_buckets(data.k[:, :T - 256], cfg), 2 * T // cfg.bucket_size)
    start = tabs.built_rows
    grow = []
    for _ in range(7):
        tabs.built_rows = start
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        pipeline.grow_buckets_(tabs, data.k, cfg)
        torch.cuda.synchronize()
        grow.append((time.perf_counter() - w0) * 1e3)
    return {"workload": "segment_starts_32k", "tables": HKV, "positions": T, "pool": POOL, "buckets": TARGET,
            "max_size": CAP, "ms": round(ms, 3), "merges_per_table": merges,
            "us_per_merge": round(ms * 1e3 / merges, 3), "deterministic": bool(torch.equal(first, again)),
            "grow_one_block_ms": round(sorted(grow)[len(grow) // 2], 3),
            "grow": "one closed 512-key block x 8 kv-heads into reserved rows (wall, synchronized)"}


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the select+read path shards by kv-head with no exchange "
              "inside the step, and this benchmark runs on a single MI355X; use --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from lsa_rocm_lab import _abi

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    _abi.load()  # fails loudly without the HIP library
    torch.cuda.set_device(0)
    dev = "cuda"
    # every select in this run is the fused HIP kernel; the caller's setting is restored after
    with select_impl("fused"):
        return run(args, np, torch, dev)


def run(args, np, torch, dev) -> int:
    """Every leg of the benchmark, in one process; prints the JSON line."""
    from lsa_rocm_lab import workloads
    from lsa_rocm_lab.port import pipeline
    from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto

    config = workloads.FLAT_32K

    # ---- workload (seeded CPU draw, identical on every machine)
    t0 = time.perf_counter()
    data = workloads.clustered(T_CTX, HQ, HKV, D, n_clusters=512, seed=0, device=dev)
    buckets = workloads.cluster_buckets(data, target=N_BUCKETS)
    log(f"workload built in {time.perf_counter() - t0:.1f}s")
    pos = torch.tensor([T_CTX - 1], device=dev, dtype=torch.int32)
    base = DecodeCache(data.q[:, -1:].contiguous(), data.k, data.v, buckets, pos)
    lists0, lengths0, out0 = decode_step(base, config)
    torch.cuda.synchronize()
    n_tok = lengths0.cpu().numpy().astype(np.int64)  # tokens read per kv-head
    gathered = int(n_tok.sum()) * D * 2 * 2          # K and V rows, bf16
    cand_bytes = HKV * N_BUCKETS * D * 2             # centroid scan, bf16
    cap = buckets.members.shape[-1]
    # the picks' member rows, or with span tables the two span ends a pick
    ids_bytes = HKV * config.top_p * (8 if buckets.spans else cap * 4)
    list_bytes = lists0.numel() * 4 + lengths0.numel() * 4  # the lists handed back
    qo_bytes = 2 * HQ * D * 2
    total_bytes = gathered + cand_bytes + ids_bytes + list_bytes + qo_bytes

    # ---- rotation copies
    R = max(1, args.rotate)
    caches = [base] + [copy_cache(base) for _ in range(R - 1)]
    torch.cuda.synchronize()
    log(f"{R} resident cache copies ({R * 2 * data.k.numel() * 2 / 2**30:.1f} GiB of K/V)")

    step = lambda i: decode_step(caches[i % R], config)
    graphs = {"full": capture(step, R, torch)}
    rem = args.steps % R
    if rem:
        graphs[rem] = capture(step, rem, torch)
    wrem = args.warmup % R
    if wrem and wrem not in graphs:
        graphs[wrem] = capture(step, wrem, torch)

    # ---- warmup + timed region
    run_steps(graphs, args.warmup, R, torch)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record()
    run_steps(graphs, args.steps, R, torch)
    ev1.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - w0
    us_step = wall_s / args.steps * 1e6
    dev_us_step = ev0.elapsed_time(ev1) * 1e3 / args.steps
    log(f"decode step {us_step:.2f} us (device {dev_us_step:.2f} us)")

    # warm (MALL-resident) variant: the same graph recipe on one copy
    warm_graph = capture(lambda i: decode_step(base, config), R, torch)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for _ in range(max(1, args.steps // R)):
        warm_graph.replay()
    torch.cuda.synchronize()
    warm_us = (time.perf_counter() - w0) / (max(1, args.steps // R) * R) * 1e6

    # ---- kernels alone: each replayed back to back from a HIP graph over the rotation, HIP
    # events around the replays on the stream they run on. The fused decode kernel is the
    # step's only kernel; the unfused path's select and read kernels are timed beside it.
    reps = max(1, args.kernel_launches // R)
    fused_us = graph_launch_us(step, R, reps, torch)
    achieved = gathered / (fused_us * 1e-6) / 1e9
    sel = [pipeline.flat_select(pipeline.index_queries(c.q, HKV)[0], c.pos, c.buckets, config) for c in caches]
    idxs = [pipeline.index_queries(c.q, HKV)[0] for c in caches]
    torch.cuda.synchronize()
    read_fn = lambda i: sparse_read_auto(caches[i % R].q, caches[i % R].k, caches[i % R].v,
                                         sel[i % R][0].unsqueeze(0), sel[i % R][1].unsqueeze(0), D ** -0.5)
    sel_fn = lambda i: pipeline.flat_select(idxs[i % R], caches[i % R].pos, caches[i % R].buckets, config)
    read_us = graph_launch_us(read_fn, R, reps, torch)
    sel_us = graph_launch_us(sel_fn, R, reps, torch)
    unfused_us = graph_launch_us(lambda i: unfused_step(caches[i % R], config), R, reps, torch)
    u_lists, u_lengths, u_out = unfused_step(base, config)
    torch.cuda.synchronize()
    unfused_same = bool(torch.equal(u_lists, lists0) and torch.equal(u_lengths, lengths0))
    log(f"fused decode kernel {fused_us:.2f} us per launch: {achieved:.0f} GB/s on gathered bytes; "
        f"unfused step {unfused_us:.2f} us (select {sel_us:.2f} + read {read_us:.2f} + index queries); "
        f"unfused lists identical: {unfused_same}")

    # ---- the same decode over a paged cache (slot table), A/B against the unpaged step
    paged = None if args.no_paged else paged_decode_leg(args, torch, np, caches, R, config, lists0, lengths0, out0)

    # ---- dense comparators on the same rotation
    dense = dense_leg(caches, R, us_step, torch)
    speedup = dense["speedup_vs_fastest"]
    copy = copy_leg(torch)
    log(f"copy {copy}")

    # ---- prefill (chunked, shared selection per 64-token chunk)
    prefill = None
    if not args.no_prefill:
        C = T_CTX // CHUNK
        ppos = torch.arange(C, device=dev, dtype=torch.int32) * CHUNK - 1

        def prefill_step():
            idx = pipeline.index_queries(data.q, HKV, CHUNK)[0]  # [C, Hkv, D]
            pl, pn = pipeline.flat_select(idx, ppos, buckets, config)
            return pipeline.lsa_read_chunked(data.q, data.k, data.v, pl.unsqueeze(0), pn.unsqueeze(0), D ** -0.5,
                                             CHUNK), pn

        _, pn = prefill_step()
        torch.cuda.synchronize()
        keys_per_row = pn.float().mean().item()
        ms = event_launch_times(lambda i: prefill_step(), args.prefill_steps, torch)
        p_ms = statistics.median(ms)
        # the stages alone: chunk index queries + select, and the read kernel
        pidx = pipeline.index_queries(data.q, HKV, CHUNK)[0]
        plists, plens = pipeline.flat_select(pidx, ppos, buckets, config)
        torch.cuda.synchronize()
        sel_ms = statistics.median(event_launch_times(
            lambda i: pipeline.flat_select(pipeline.index_queries(data.q, HKV, CHUNK)[0], ppos, buckets, config),
            args.prefill_steps, torch))
        read_ms = statistics.median(event_launch_times(
            lambda i: pipeline.lsa_read_chunked(data.q, data.k, data.v, plists.unsqueeze(0), plens.unsqueeze(0),
                                                D ** -0.5, CHUNK), args.prefill_steps, torch))
        # flops: 4*D per (q-head row, key); shared list + the causal local triangle
        list_pairs = float(pn.to(torch.float64).sum().item()) * CHUNK * (HQ // HKV)
        local_pairs = C * HQ * CHUNK * (CHUNK + 1) / 2
        flops = 4.0 * D * (list_pairs + local_pairs)
        dense_p = None
        try:
            import torch.nn.functional as F
            from torch.nn.attention import SDPBackend, sdpa_kernel

            qq, kk, vv = (t.permute(0, 2, 1, 3) for t in (data.q, data.k, data.v))

            def dfn(i):
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                    return F.scaled_dot_product_attention(qq, kk, vv, is_causal=True, scale=D ** -0.5,
                                                          enable_gqa=True)

            dfn(0)
            torch.cuda.synchronize()
            dense_p = statistics.median(event_launch_times(dfn, args.prefill_steps, torch))
        except RuntimeError as exc:
            log(f"dense prefill unavailable: {str(exc).splitlines()[0][:120]}")
        prefill = {"workload": "flat_prefill_32k", "chunk": CHUNK, "ms_per_step": round(p_ms, 3),
                   "tok_per_s": round(T_CTX / (p_ms * 1e-3), 1), "keys_per_row": round(keys_per_row + CHUNK / 2, 1),
                   "flops": flops, "tflops": round(flops / (p_ms * 1e-3) / 1e12, 2),
                   "mfma_frac": round(flops / (p_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                   "select_ms": round(sel_ms, 3), "read_ms": round(read_ms, 3),
                   "read_tflops": round(flops / (read_ms * 1e-3) / 1e12, 2),
                   "read_mfma_frac": round(flops / (read_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                   "read": "MFMA tile kernel (bf16 v_mfma_f32_32x32x16, fp32 accumulate)",
                   "dense_sdpa_ms": None if dense_p is None else round(dense_p, 3),
                   "speedup_vs_dense": None if dense_p is None else round(dense_p / p_ms, 3)}
        log(f"prefill {prefill}")

    # ---- the positional block-sparse arm through the same fused kernel
    block_sparse = block_sparse_leg(args, torch, np)

    # ---- batched flat decode (B=32 x 32k): the fused kernel's bandwidth regime
    batched = None if args.no_tree else batched_flat_leg(args, torch, np)

    # ---- batched tree decode (B=32 x 131k): the bandwidth-bound regime of the read
    tree = None
    if not args.no_tree:
        tree = tree_decode_leg(args, torch, np)
        log(f"tree {tree}")

    # ---- the reference's decode arms at its default knobs (flat and the 3-level tree)
    refcfg = None
    if not args.no_tree:
        refcfg = refcfg_decode_leg(args, torch, np, dense.get("us_per_step") if dense else None)

    # ---- the reference's prefill arm at its default knobs (per-row selection, per-row read)
    refcfg_p = None
    if not args.no_refcfg_prefill:
        refcfg_p = refcfg_prefill_leg(args, torch, np, prefill.get("dense_sdpa_ms") if prefill else None)

    # ---- the bucket-table build (the index build before the path)
    build = None
    if not args.no_build:
        build = bucket_build_leg(args, torch)
        log(f"bucket build {build}")

    # ---- parity of the timed step against the numpy oracle (lists bit-exact, read in the bar)
    parity = None
    if not args.no_cpu:
        import oracle

        q_np = base.q.float().cpu().numpy()
        cents = buckets.centroids.float().cpu().numpy()
        members_np, ends_np = buckets.members.cpu().numpy(), buckets.ends.cpu().numpy()
        idx_np = oracle.index_queries(q_np, HKV)[0, 0]
        ls, ns = [], []
        for g in range(HKV):
            lst, n = oracle.flat_select(idx_np[g][None], np.array([T_CTX - 1]), cents[g], members_np[g],
                                        cluster_block_size=config.cluster_block_size,
                                        block_buckets=config.block_bucket_count, top_p=config.top_p,
                                        top_k=config.top_k, window=config.window_size, sink=config.sink_size,
                                        mode="bf16", ends=ends_np[g])
            ls.append(lst[0])
            ns.append(n[0])
        ls, ns = np.stack(ls), np.array(ns)
        want = oracle.sparse_read(q_np, data.k.float().cpu().numpy(), data.v.float().cpu().numpy(),
                                  ls[None, None], ns[None, None], D ** -0.5)
        err = np.abs(out0.float().cpu().numpy() - want)
        parity = {"lists_bit_exact": bool(np.array_equal(lists0[0].cpu().numpy(), ls)),
                  "lengths_bit_exact": bool(np.array_equal(lengths0[0].cpu().numpy(), ns)),
                  "read_max_abs": float(err.max()), "read_mean_abs": float(err.mean())}
        log(f"parity {parity}")

    # ---- the 2k fp32 decode (CPU-runnable config): GPU step and parity
    c1 = decode_2k_leg(args, torch, np)
    log(f"decode_2k_fp32 {c1}")

    # ---- CPU baseline: the torch CPU restatement of the same step on the host cores
    cpu = None
    if not args.no_cpu:
        cpu = cpu_leg(args, torch, base, data, buckets, config, lists0, lengths0, c1)
        log(f"cpu {cpu}")

    if args.copy_mib:  # a plain copy of known size, for scaling FETCH_SIZE / WRITE_SIZE counters
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {args.copy_mib} MiB three times")

    line = {
        "metric": METRIC,
        "value": round(us_step, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded clustered keys (512 clusters/kv-head, sigma 0.3), q/v ~ N(0,1)",
        "config": {"workload": "flat_decode_32k", "batch": 1, "context": T_CTX, "heads_q": HQ, "heads_kv": HKV,
                   "head_dim": D, "buckets_per_kv_head": N_BUCKETS, "top_buckets": config.top_p,
                   "tokens_read": n_tok.tolist(), "rotated_copies": R, "timing": "hip graphs, wall clock"},
        "gbps": round(gathered / (us_step * 1e-6) / 1e9, 1),
        "gbps_total": round(total_bytes / (us_step * 1e-6) / 1e9, 1),
        "device_us_per_step": round(dev_us_step, 3),
        "warm_us_per_step": round(warm_us, 3),
        "fused_kernel_us": round(fused_us, 3),
        "unfused": {"us_per_step": round(unfused_us, 3), "select_us": round(sel_us, 3), "read_us": round(read_us, 3),
                    "lists_identical": unfused_same},
        "kernel_timing": "per launch, HIP graph of back-to-back launches over the rotation, HIP events",
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("decode_flat_kernel"),
                     "traffic_source": "not measured in this run: the rocprofv3 FETCH_SIZE + WRITE_SIZE figure "
                                       "of this kernel committed in profiles/decode_flat32k_pmc.md",
                     "kernel": "decode_flat_kernel<bf16,bf16,128,4>", "bytes_per_launch": gathered,
                     "all_bytes_per_launch": total_bytes},
        "dense": dense,
        "speedup_vs_dense": None if speedup is None else round(speedup, 3),
        "hbm_copy": copy,
        "decode_2k_fp32": {k: v for k, v in c1.items() if not k.startswith("_")},
        "prefill": prefill,
        "block_sparse_decode": block_sparse,
        "batched_flat_decode": batched,
        "tree_decode": tree,
        "refcfg_decode": refcfg,
        "refcfg_prefill": refcfg_p,
        "paged_decode": paged,
        "bucket_build": build,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
