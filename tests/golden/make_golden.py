"""Writes the golden fixtures of the select+read path from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no tensor fixtures for this path, so these are written here, from the
oracle (itself pinned by tests/test_oracle.py). Inputs are not stored: each case names a
seeded CPU generator recipe (lsa_rocm_lab.workloads) that every machine reproduces bit for
bit, and the fixture keeps the sha256 of the generated inputs to detect drift. Stored per
case: the expected read lists, lengths and fp32 read output.
"""

from __future__ import annotations

import hashlib
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT / "latent-sparse-attention-rocm_amd", ROOT):
    sys.path.insert(0, str(p))

import oracle  # noqa: E402
from lsa_rocm_lab import workloads  # noqa: E402


def sha(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def positional_case(name, T, Hq, Hkv, D, dtype, config):
    q, k, v = workloads.geometry(T, Hq, Hkv, D, dtype=dtype, seed=0, device="cpu")
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    blocks = T // config.cluster_block_size
    members = oracle.position_members(blocks, config.cluster_block_size, config.bucket_size, config.bucket_cap)
    mode = "fp32" if dtype == torch.float32 else "bf16"
    idx = oracle.index_queries(qn[:, -1:], Hkv)[0, 0]
    lists, lengths = [], []
    for g in range(Hkv):
        cent = oracle.bucket_centroids(kn[0, :, g], members, "mean")
        cent = cent if mode == "fp32" else oracle.bf16_round(cent)
        l, n = oracle.flat_select(idx[g][None], np.array([T - 1]), cent, members,
                                  cluster_block_size=config.cluster_block_size, block_buckets=config.block_bucket_count,
                                  top_p=config.top_p, top_k=config.top_k, window=config.window_size,
                                  sink=config.sink_size, mode=mode)
        lists.append(l[0])
        lengths.append(n[0])
    lists, lengths = np.stack(lists), np.array(lengths, np.int32)
    out = oracle.sparse_read(qn[:, -1:], kn, vn, lists[None, None], lengths[None, None])
    return dict(name=name, recipe=f"geometry(T={T}, Hq={Hq}, Hkv={Hkv}, D={D}, {dtype}, seed=0)",
                input_sha256=sha(qn, kn, vn), lists=lists, lengths=lengths, out=out)


def clustered_case(name, T, Hq, Hkv, D, n_clusters, seed, target):
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=n_clusters, seed=seed, device="cpu")
    qn, kn, vn = (t.float().numpy() for t in (data.q, data.k, data.v))
    config = workloads.FLAT_32K
    idx = oracle.index_queries(qn[:, -1:], Hkv)[0, 0]
    lists, lengths, starts_all = [], [], []
    for g in range(Hkv):
        starts = workloads.ward_segments(data.run_lengths[0, g].numpy(), data.run_clusters[0, g].numpy(),
                                         data.centers[0, g].numpy(), T, target)
        members, _, ends = (t.numpy() for t in workloads.segment_tables(starts, config.bucket_cap, "cpu"))
        cent = oracle.bf16_round(oracle.bucket_centroids(kn[0, :, g], members, "mean"))
        l, n = oracle.flat_select(idx[g][None], np.array([T - 1]), cent, members,
                                  cluster_block_size=config.cluster_block_size, block_buckets=config.block_bucket_count,
                                  top_p=config.top_p, top_k=config.top_k, window=config.window_size,
                                  sink=config.sink_size, mode="bf16", ends=ends)
        lists.append(l[0])
        lengths.append(n[0])
        starts_all.append(starts)
    lists, lengths = np.stack(lists), np.array(lengths, np.int32)
    out = oracle.sparse_read(qn[:, -1:], kn, vn, lists[None, None], lengths[None, None])
    return dict(name=name, recipe=f"clustered(T={T}, Hq={Hq}, Hkv={Hkv}, D={D}, n_clusters={n_clusters}, "
                f"seed={seed}); ward_segments(target={target})", input_sha256=sha(qn, kn, vn),
                starts=np.stack(starts_all), lists=lists, lengths=lengths, out=out)


def cases():
    yield positional_case("decode_2k_fp32", 2048, 8, 2, 64, torch.float32, workloads.DECODE_2K)
    yield positional_case("block_sparse_4k_bf16", 4096, 8, 2, 128, torch.bfloat16, workloads.BLOCK_SPARSE_32K)
    yield clustered_case("flat_clustered_4k_bf16", 4096, 8, 2, 128, 64, 5, 64)


def main() -> None:
    for case in cases():
        name = case.pop("name")
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **{k: (np.asarray(v) if not isinstance(v, str) else np.array(v)) for k, v in case.items()})
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
