"""lsa_decode_flat_noalloc (the decode entry point that allocates nothing, its counters and
scratch in a file-scope device array) against lsa_decode_flat with caller buffers, through
the C ABI: lists, lengths and outputs bit-identical (the same kernels), on two calls in a
row, the second with a smaller input, and a size beyond the array rejected."""

import ctypes

import pytest
import torch

from lsa_rocm_lab import _abi, workloads
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.read_kernel_tiled import _kv_layout

pytestmark = pytest.mark.gpu
DEV = "cuda"


def noalloc_decode(q, k, v, pos, buckets, config, reset=0):
    """The flat_decode argument set, passed to lsa_decode_flat_noalloc."""
    B, _, Hq, D = q.shape
    Tk, Hkv = k.shape[1], k.shape[2]
    q = q.contiguous()
    k, v, sb, st, sh = _kv_layout(k, v)
    members = buckets.members.to(torch.int32).contiguous()
    ends = buckets.ends.to(torch.int32).contiguous()
    table = buckets.centroids.to(torch.bfloat16).contiguous()
    lead = table.dim() - 2
    row_tables, group_tables = (0, 1) if lead == 1 else (Hkv, 1)
    width = config.top_k + config.window_size + config.sink_size
    lists = torch.empty(B, Hkv, width, dtype=torch.int32, device=DEV)
    lengths = torch.empty(B, Hkv, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    splits = pipeline._select_splits(B, Hkv, table.shape[-2], config.top_p)
    rc = _abi.load().lsa_decode_flat_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _abi.dtype_code(q.dtype), B, Tk, Hq, Hkv, D, sb, st, sh,
        table.data_ptr(), members.data_ptr(), ends.data_ptr(), _abi.TABLE_SPANS if buckets.spans else 0,
        table.shape[-2], members.shape[-1], row_tables, group_tables, _abi.SCORE_BF16, pos.data_ptr(),
        config.cluster_block_size, config.block_bucket_count, config.top_p, config.window_size, config.sink_size,
        config.top_k, ctypes.c_float(D ** -0.5), splits, 0, reset, lists.data_ptr(), lengths.data_ptr(),
        out.data_ptr(), status.data_ptr(), _abi.stream(torch.device(DEV)))
    return rc, out, lists, lengths, status


def case(T, Hq, Hkv, B, seed):
    data = workloads.clustered(T, Hq, Hkv, 128, n_clusters=T // 64, seed=seed, B=B, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    pos = torch.full((B,), T - 1, dtype=torch.int32, device=DEV)
    return data.q[:, -1:].contiguous(), data.k, data.v, pos, buckets


def test_noalloc_equals_workspace_decode_twice_then_smaller():
    config = workloads.FLAT_32K
    for label, (T, Hq, Hkv, B, seed) in (("32k B=1 Hkv=8", (32768, 32, 8, 1, 3)), ("4k B=2 Hkv=2", (4096, 8, 2, 2, 4))):
        print(f"case no-alloc {label}", flush=True)
        q, k, v, pos, buckets = case(T, Hq, Hkv, B, seed)
        want = pipeline.flat_decode(q, k, v, pos, buckets, config)
        for _ in range(2):
            rc, out, lists, lengths, status = noalloc_decode(q, k, v, pos, buckets, config)
            torch.cuda.synchronize()
            assert rc == 0, _abi.load().lsa_last_error()
            assert int(status.item()) == 0
            assert torch.equal(lists, want[1]) and torch.equal(lengths, want[2])
            assert torch.equal(out, want[0])
    # an explicit counter reset gives the same result
    rc, out, lists, lengths, _ = noalloc_decode(q, k, v, pos, buckets, config, reset=1)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(out, want[0]) and torch.equal(lists, want[1])


def test_noalloc_rejects_sizes_beyond_its_array():
    """Partials of 32 readers for 4096 (row, kv-head) units exceed the 15 MiB of scratch
    (and their counters the 1 MiB): a clear error before any launch."""
    lib = _abi.load()
    need = lib.lsa_decode_flat_scratch_bytes(_abi.LSA_BF16, 512, 32, 8, 128, 512, 32, 0, 0, 1, 32)
    assert need > 15 << 20
    rc = lib.lsa_decode_flat_noalloc(16, 16, 16, _abi.LSA_BF16, 512, 32768, 32, 8, 128, 0, 1024, 128, 16, 16, 16,
                                     1, 512, 256, 0, 1, _abi.SCORE_BF16, 16, 64, 1, 32, 0, 0, 8192,
                                     ctypes.c_float(0.088), 1, 32, 0, 16, 16, 16, None, None)
    assert rc == -5 and b"exceed" in lib.lsa_last_error()
