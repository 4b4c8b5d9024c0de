"""The bucket-table build on the GPU (contiguous Ward-style segments from the keys) vs the
CPU oracle.

Segment starts must equal the oracle's bit for bit (the merge order depends on exact fp64
costs). Cases: fp32 / bf16 / fp16 keys, head dims 32 / 64 / 128, pool sizes 4 / 8 / 16, a
shorter last pool, several (batch, kv-head) tables with strided cache views, the 32k
table of the benchmark geometry, ties (identical keys merge leftmost first), a target no
merge can reach under max_size (ValueError), and the tables feeding the fused decode
(lists equal the oracle's flat select over the same tables).
"""

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline

pytestmark = pytest.mark.gpu
DEV = "cuda"


def oracle_starts(keys, pool, target, max_size):
    B, T, H, D = keys.shape
    kf = keys.float().cpu().numpy()
    return np.stack([np.stack([oracle.ward_segments_keys(kf[b, :, g], pool, target, max_size) for g in range(H)])
                     for b in range(B)])


def clustered_keys(B, T, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    centers = torch.randn(B, H, 16, D, generator=g)
    runs = torch.randint(0, 16, (B, H, T // 24 + 1), generator=g).repeat_interleave(24, dim=-1)[..., :T]
    k = torch.gather(centers, 2, runs[..., None].expand(B, H, T, D)) + 0.3 * torch.randn(B, H, T, D, generator=g)
    return k.permute(0, 2, 1, 3).contiguous().to(dtype)


@pytest.mark.parametrize("dtype,D,pool,T,target,max_size", [
    (torch.bfloat16, 128, 16, 2048, 32, 256),
    (torch.float32, 64, 8, 1000, 40, 96),
    (torch.float16, 32, 4, 777, 50, 64),
    (torch.bfloat16, 128, 16, 4096, 64, 128),
])
def test_segment_starts_equal_oracle(dtype, D, pool, T, target, max_size):
    keys = clustered_keys(2, T, 2, D, dtype, seed=T + D)
    print(f"case {dtype} D={D} pool={pool} T={T} target={target} max={max_size}", flush=True)
    got = pipeline.segment_starts(keys.to(DEV), target, pool, max_size).cpu().numpy()
    assert np.array_equal(got, oracle_starts(keys, pool, target, max_size))


def test_segment_starts_on_a_strided_cache_view():
    """K rows read in place from a view of a wider cache (token stride 3 Hkv D)."""
    base = clustered_keys(1, 1536, 6, 64, torch.bfloat16, seed=8)
    view = base.to(DEV)[:, :, 2:4]  # kv-heads 2 and 3 of 6
    got = pipeline.segment_starts(view, 24, 16, 256).cpu().numpy()
    assert np.array_equal(got, oracle_starts(base[:, :, 2:4], 16, 24, 256))


def test_segment_starts_32k_table():
    """The benchmark geometry's table size: 32768 positions, 2048 pools -> 512 segments."""
    data = workloads.clustered(32768, 8, 2, 128, n_clusters=512, seed=3, device=DEV)
    got = pipeline.segment_starts(data.k, 512, 16, 256).cpu().numpy()
    assert np.array_equal(got, oracle_starts(data.k, 16, 512, 256))


def test_ties_merge_leftmost_and_unreachable_target_raises():
    keys = torch.ones(1, 64, 1, 64, dtype=torch.float32, device=DEV)
    assert pipeline.segment_starts(keys, 3, 8, 64).cpu().tolist() == [[[0, 48, 56, 64]]]
    with pytest.raises(ValueError, match="cannot reach"):
        pipeline.segment_starts(keys, 3, 8, 8)


def test_built_tables_drive_the_fused_decode():
    """Tables built on the GPU feed the fused decode (span tables); its lists equal the
    oracle's flat select over the same tables and its output the oracle read."""
    from test_gpu_decode import check_decode

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=21, device=DEV)
    buckets = pipeline.segment_buckets(data.k, T // 64, 16, 256)
    assert buckets.spans and buckets.members.shape == (Hkv, T // 64, 256)
    ends = buckets.ends.cpu().numpy()
    starts = oracle_starts(data.k, 16, T // 64, 256)[0]
    assert np.array_equal(ends, starts[:, 1:])
    members = buckets.members.cpu().numpy()
    for g in range(Hkv):
        want = oracle.bucket_centroids(data.k[0, :, g].float().cpu().numpy(), members[g], "mean")
        assert np.abs(buckets.centroids_f32[g].cpu().numpy() - want).max() <= 1e-5
    pos = torch.tensor([T - 1], dtype=torch.int32)
    check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K, label="built tables")
