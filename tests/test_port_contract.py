"""Host-side contract of the port surface, on the CPU: the LSA_SELECT_IMPL switch, the
reference's error types, and no CPU fallback anywhere on the path."""

import os
import pathlib

import pytest
import torch

from lsa_rocm_lab.port import pipeline, select_fused
from lsa_rocm_lab.port.pipeline import Buckets, PortConfig
from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto


def _tiny():
    tiny = torch.randn(2, 16)
    config = PortConfig(top_p=4, top_k=8, window_size=4, sink_size=2, cluster_block_size=8, bucket_size=2,
                        bucket_cap=4, pool_size=2, node_bucket_size=2)
    buckets = Buckets(tiny.bfloat16(), torch.zeros(8, 4, dtype=torch.int32) - 1, torch.zeros(8, dtype=torch.int32),
                      centroids_f32=tiny)
    return tiny, config, buckets


def test_switch_unknown_impl_fails_loudly():
    tiny, config, buckets = _tiny()
    os.environ["LSA_SELECT_IMPL"] = "bogus"
    try:
        with pytest.raises(ValueError, match="LSA_SELECT_IMPL"):
            pipeline.flat_select(tiny, torch.tensor([7, 7]), buckets, config)
    finally:
        os.environ.pop("LSA_SELECT_IMPL", None)


def test_switch_default_is_reference_and_documented(monkeypatch):
    monkeypatch.delenv("LSA_SELECT_IMPL", raising=False)
    assert pipeline.flat_select.__doc__ and "LSA_SELECT_IMPL" in pipeline.flat_select.__doc__


@pytest.mark.parametrize("impl", ["reference", "fused", "fused_unpack"])
def test_cpu_tensors_have_no_fallback(impl, monkeypatch):
    tiny, config, buckets = _tiny()
    monkeypatch.setenv("LSA_SELECT_IMPL", impl)
    with pytest.raises(ValueError, match="ROCm kernel"):
        pipeline.flat_select(tiny, torch.tensor([7, 7]), buckets, config)


def test_position_mismatch_raises_like_the_reference():
    tiny, config, buckets = _tiny()
    with pytest.raises(ValueError, match="a position a query"):
        pipeline._production_scores(tiny, torch.tensor([7]), buckets, config, "bf16")


def test_select_topk_scores_rejects_cpu_after_wide_warning():
    scores = torch.randn(4, 64)
    with pytest.warns(UserWarning, match="sampled listing"):
        with pytest.raises(ValueError, match="ROCm kernel"):
            select_fused.select_topk_scores(scores, torch.full((4,), 64, dtype=torch.int32), 8)


def test_expand_rejects_cpu():
    with pytest.raises(ValueError, match="ROCm kernel"):
        select_fused.expand_in_order_from_keys(torch.zeros(1, 4, dtype=torch.int64), torch.zeros(4, 16,
                                               dtype=torch.int32), torch.zeros(1, dtype=torch.int32), 4, 2, 8)


def test_sparse_read_asserts_gpu():
    q = torch.randn(1, 4, 8, 64)
    k = torch.randn(1, 4, 2, 64)
    with pytest.raises(AssertionError, match="GPU kernel"):
        sparse_read_auto(q, k, k, torch.zeros(1, 4, 8, dtype=torch.int32), torch.ones(1, 4, dtype=torch.int32))


def test_dense_read_rejects_long_queries():
    q = torch.randn(1, 8, 2, 16)
    k = torch.randn(1, 4, 2, 16)
    with pytest.raises(ValueError, match="exceed the cache"):
        pipeline.dense_read(q, k, k, 0.25)


def test_config_defaults_match_the_reference():
    c = PortConfig()
    assert (c.cluster_block_size, c.pool_size, c.bucket_size, c.bucket_cap, c.top_p, c.top_k, c.window_size,
            c.sink_size, c.node_bucket_size, c.top_level, c.node_cluster_block_size, c.beam_width,
            c.start_nodes) == (512, 4, 8, 16, 1024, 4096, 512, 4, 4, 3, 64, 64, None)
    assert c.block_bucket_count == 64


def test_bucket_build_rejects_cpu_tensors():
    """The bucket build is a GPU kernel too: host tensors raise, nothing falls back."""
    keys = torch.zeros(1, 1024, 2, 64)
    with pytest.raises(ValueError, match="ROCm kernel"):
        pipeline.segment_starts(keys, 8)
    with pytest.raises(ValueError, match="ROCm kernel"):
        pipeline.build_buckets(keys[0, :, 0], pipeline.PortConfig())


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys

    root = pathlib.Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0 and "one GPU" in r.stdout + r.stderr
