"""The sparse read on the GPU vs the CPU oracle and the dense SDPA baseline.

Cases follow the reference's read tests (test_read_kernel_tiled.py, test_dense_read.py,
gates D2/G/H): real selections at fp32/fp16/bf16, full causal lists == dense SDPA,
GQA/MQA mappings, pad and boundary ids, duplicates per occurrence, zero-length rows
(tiled: zeros; v1: NaN), ragged batches, a 4620-id decode row, per-kv-head lists,
every split count, and the chunked-prefill read.
Tolerances (max-abs vs the fp64 oracle): fp32 1e-4, fp16 5e-3, bf16 2e-2 with
mean-abs 2e-3 for bf16.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.read_kernel import sparse_read
from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_auto, sparse_read_chunked, sparse_read_tiled

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: (1e-4, 1e-5), torch.float16: (5e-3, 5e-4), torch.bfloat16: (2e-2, 2e-3)}


def geometry(dtype, T=512, Hq=8, Hkv=2, D=64, seed=20261106, B=1, Tk=None):
    g = torch.Generator().manual_seed(seed)
    Tk = Tk or T
    q = (torch.randn(B, T, Hq, D, generator=g) * 0.2).to(dtype)
    k = (torch.randn(B, Tk, Hkv, D, generator=g) * 0.2).to(dtype)
    v = (torch.randn(B, Tk, Hkv, D, generator=g) * 0.2).to(dtype)
    return q, k, v


def check(out, want, dtype):
    max_abs, mean_abs = TOL[dtype]
    err = np.abs(out.float().cpu().numpy() - want)
    assert np.isfinite(err).all()
    assert err.max() <= max_abs, f"max-abs {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"mean-abs {err.mean():.3e} > {mean_abs}"


def run(fn, q, k, v, ids, lengths, **kw):
    return fn(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), **kw)


def want_of(q, k, v, ids, lengths, scale=None, empty="zero"):
    return oracle.sparse_read(q.float().numpy(), k.float().numpy(), v.float().numpy(), ids.numpy(), lengths.numpy(),
                              scale, empty)


def causal_lists(T, width=None):
    row = torch.arange(T, dtype=torch.int32)
    ids = torch.where(row[None, :] <= row[:, None], row[None, :].expand(T, T), torch.tensor(-1, dtype=torch.int32))
    if width is not None:
        ids = torch.cat([ids, torch.full((T, width - T), -1, dtype=torch.int32)], dim=1)
    return ids.view(1, T, -1).contiguous(), (row + 1).view(1, T).contiguous()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_random_lists_all_dtypes(dtype):
    q, k, v = geometry(dtype, T=256)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(-1, 256, (1, 256, 300), generator=g, dtype=torch.int32)
    lengths = torch.randint(0, 301, (1, 256), generator=g, dtype=torch.int32)
    check(run(sparse_read_auto, q, k, v, ids, lengths), want_of(q, k, v, ids, lengths), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_full_causal_matches_dense_sdpa(dtype):
    q, k, v = geometry(dtype, T=256)
    ids, lengths = causal_lists(256)
    scale = q.shape[-1] ** -0.5
    got = run(sparse_read_tiled, q, k, v, ids, lengths, scale=scale)
    dense = pipeline.dense_read(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    max_abs = TOL[dtype][0]
    assert float((got.float() - dense.float()).abs().max()) <= max_abs
    check(got, want_of(q, k, v, ids, lengths, scale), dtype)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 1), (2, 2), (16, 2)])
def test_gqa_mqa_mapping(hq, hkv):
    q, k, v = geometry(torch.bfloat16, T=384, Hq=hq, Hkv=hkv)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 384, (1, 384, 1024), generator=g, dtype=torch.int32)
    lengths = torch.full((1, 384), 1024, dtype=torch.int32)
    check(run(sparse_read_auto, q, k, v, ids, lengths), want_of(q, k, v, ids, lengths), torch.bfloat16)


def test_batch_and_ragged_rows():
    B, T = 3, 13
    q, k, v = geometry(torch.bfloat16, T=T, B=B)
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, T, (B, T, 128), generator=g, dtype=torch.int32)
    lengths = torch.randint(1, 129, (B, T), generator=g, dtype=torch.int32)
    check(run(sparse_read_auto, q, k, v, ids, lengths), want_of(q, k, v, ids, lengths), torch.bfloat16)


@pytest.mark.parametrize("splits", ["1", "3", "64", None])
def test_decode_single_row_long_list(splits):
    q, k, v = geometry(torch.bfloat16, T=512)
    g = torch.Generator().manual_seed(13)
    ids = torch.randint(0, 512, (1, 1, 4620), generator=g, dtype=torch.int32)
    lengths = torch.full((1, 1), 4620, dtype=torch.int32)
    if splits:
        os.environ["LSA_READ_SPLITS"] = splits
    try:
        got = run(sparse_read_auto, q[:, -1:], k, v, ids, lengths)
    finally:
        os.environ.pop("LSA_READ_SPLITS", None)
    check(got, want_of(q[:, -1:], k, v, ids, lengths), torch.bfloat16)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (64, 8, 2), (256, 4, 4), (32, 8, 1)])
def test_per_kv_head_lists_decode(D, Hq, Hkv):
    q, k, v = geometry(torch.bfloat16, T=2048, Hq=Hq, Hkv=Hkv, D=D)
    g = torch.Generator().manual_seed(D + Hq)
    ids = torch.randint(-1, 2048, (1, 1, Hkv, 700), generator=g, dtype=torch.int32)
    lengths = torch.randint(0, 701, (1, 1, Hkv), generator=g, dtype=torch.int32)
    got = run(sparse_read_auto, q[:, -1:], k, v, ids, lengths)
    check(got, want_of(q[:, -1:], k, v, ids, lengths), torch.bfloat16)


def test_pad_and_boundary_indices():
    q, k, v = geometry(torch.bfloat16, T=256)
    ids = torch.full((1, 256, 512), -1, dtype=torch.int32)
    ids[:, :, 0] = 0
    ids[:, :, 1] = 255
    lengths = torch.full((1, 256), 3, dtype=torch.int32)
    got = run(sparse_read_tiled, q, k, v, ids, lengths)
    check(got, want_of(q, k, v, ids, lengths), torch.bfloat16)
    assert got.float().abs().max() > 0


def test_out_of_range_ids_are_skipped():
    q, k, v = geometry(torch.float32, T=64)
    ids = torch.tensor([[[3, 64, 1000, -5, 7]]], dtype=torch.int32).expand(1, 64, 5).contiguous()
    lengths = torch.full((1, 64), 5, dtype=torch.int32)
    got = run(sparse_read_auto, q, k, v, ids, lengths)
    keep = torch.tensor([[[3, 7]]], dtype=torch.int32).expand(1, 64, 2).contiguous()
    check(got, want_of(q, k, v, keep, torch.full((1, 64), 2, dtype=torch.int32)), torch.float32)


def test_duplicate_ids_counted_per_occurrence():
    q, k, v = geometry(torch.bfloat16, T=128)
    ids = torch.full((1, 128, 8), -1, dtype=torch.int32)
    ids[:, 0, 0] = 5
    ids[:, 0, 1] = 5
    lengths = torch.full((1, 128), 2, dtype=torch.int32)
    got = run(sparse_read_tiled, q, k, v, ids, lengths)
    for h in range(8):
        assert torch.allclose(got[0, 0, h].float().cpu(), v[0, 5, h // 4].float(), atol=1e-2, rtol=1e-2), h


def test_zero_length_rows_zero_tiled_nan_v1():
    q, k, v = geometry(torch.bfloat16, T=64)
    ids = torch.full((1, 64, 128), -1, dtype=torch.int32)
    lengths = torch.zeros(1, 64, dtype=torch.int32)
    tiled = run(sparse_read_tiled, q, k, v, ids, lengths)
    assert torch.isfinite(tiled).all() and tiled.float().abs().max() == 0.0
    base = run(sparse_read, q, k, v, ids, lengths)
    assert torch.isnan(base).all()


def test_mixed_zero_and_real_rows():
    q, k, v = geometry(torch.bfloat16, T=64)
    g = torch.Generator().manual_seed(17)
    ids = torch.randint(0, 64, (1, 64, 32), generator=g, dtype=torch.int32)
    lengths = torch.full((1, 64), 32, dtype=torch.int32)
    lengths[0, 1::2] = 0
    got = run(sparse_read_tiled, q, k, v, ids, lengths)
    assert torch.isfinite(got).all()
    assert got[0, 1::2].float().abs().max() == 0.0
    assert got[0, 0::2].float().abs().max() > 0
    check(got, want_of(q, k, v, ids, lengths), torch.bfloat16)


def test_lengths_clamped_to_width():
    q, k, v = geometry(torch.float32, T=64)
    g = torch.Generator().manual_seed(19)
    ids = torch.randint(0, 64, (1, 64, 16), generator=g, dtype=torch.int32)
    lengths = torch.full((1, 64), 10_000, dtype=torch.int32)
    got = run(sparse_read_auto, q, k, v, ids, lengths)
    check(got, want_of(q, k, v, ids, torch.full((1, 64), 16, dtype=torch.int32)), torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunked_read_matches_oracle(dtype):
    T, Hq, Hkv, D, chunk = 256, 8, 2, 64, 64
    q, k, v = geometry(dtype, T=T, Hq=Hq, Hkv=Hkv, D=D)
    C = T // chunk
    g = torch.Generator().manual_seed(23)
    ids = torch.full((1, C, Hkv, 96), -1, dtype=torch.int32)
    lengths = torch.zeros(1, C, Hkv, dtype=torch.int32)
    for c in range(1, C):
        for h in range(Hkv):
            n = int(torch.randint(1, 97, (1,), generator=g))
            ids[0, c, h, :n] = torch.randint(0, c * chunk, (n,), generator=g, dtype=torch.int32)
            lengths[0, c, h] = n
    got = sparse_read_chunked(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), None, chunk)
    want = oracle.sparse_read_chunked(q.float().numpy(), k.float().numpy(), v.float().numpy(), ids.numpy(),
                                      lengths.numpy(), chunk)
    check(got, want, dtype)


def test_dense_decode_and_chunk_equal_prefill_tail():
    q, k, v = geometry(torch.bfloat16, T=512)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    scale = q.shape[-1] ** -0.5
    prefill = pipeline.dense_read(q, k, v, scale)
    decode = pipeline.dense_read(q[:, -1:], k, v, scale)
    tail = pipeline.dense_read(q[:, -16:], k, v, scale)
    assert torch.allclose(decode.float(), prefill[:, -1:].float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(tail.float(), prefill[:, -16:].float(), atol=2e-2, rtol=2e-2)
    with pytest.raises(ValueError):
        pipeline.dense_read(q, k[:, :32], v[:, :32], scale)


def test_kv_views_are_read_in_place():
    """K/V given as views into a larger cache (token stride of a longer buffer, every other
    kv-head) give the same output as their dense copies, and nothing is copied."""
    q, k, v = geometry(torch.bfloat16, T=256, Hq=8, Hkv=4, D=128)
    big_k = torch.zeros(1, 512, 4, 128, dtype=torch.bfloat16)
    big_v = torch.zeros(1, 512, 4, 128, dtype=torch.bfloat16)
    big_k[:, :256], big_v[:, :256] = k, v
    g = torch.Generator().manual_seed(29)
    ids = torch.randint(-1, 256, (1, 1, 2, 600), generator=g, dtype=torch.int32)
    lengths = torch.tensor([[[600, 333]]], dtype=torch.int32)
    bk, bv = big_k.to(DEV), big_v.to(DEV)
    kview, vview = bk[:, :256, ::2], bv[:, :256, ::2]  # 2 kv-heads, strided tokens and heads
    assert not kview.is_contiguous()
    got = sparse_read_auto(q[:, -1:].to(DEV)[:, :, :4].contiguous(), kview, vview, ids.to(DEV), lengths.to(DEV))
    want = oracle.sparse_read(q[:, -1:, :4].float().numpy(), k[:, :, ::2].float().numpy(),
                              v[:, :, ::2].float().numpy(), ids.numpy(), lengths.numpy())
    check(got, want, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (16, 4), (16, 2)])
def test_matrix_core_read_group_sizes(dtype, hq, hkv):
    """16-bit rows of D = 128 score on the matrix cores for 1, 2, 4 and 8 query heads a
    kv-head: a batch of per-token lists (one tile or two per row), then a decode row of
    per-kv-head lists long enough that every split walks several tiles (the pipelined loop
    with loads one tile ahead), at a fixed split count and at the planner's."""
    T = 1024
    q, k, v = geometry(dtype, T=T, Hq=hq, Hkv=hkv, D=128, seed=100 * hq + hkv)
    g = torch.Generator().manual_seed(hq + 7 * hkv)
    ids = torch.randint(-1, T, (1, 96, 160), generator=g, dtype=torch.int32)
    lengths = torch.randint(0, 161, (1, 96), generator=g, dtype=torch.int32)
    qs = q[:, -96:].contiguous()
    print(f"case prefill rows {dtype} hq={hq} hkv={hkv}", flush=True)
    check(run(sparse_read_auto, qs, k, v, ids, lengths), want_of(qs, k, v, ids, lengths), dtype)
    ids = torch.randint(-1, T, (1, 1, hkv, 3000), generator=g, dtype=torch.int32)
    lengths = torch.randint(2000, 3001, (1, 1, hkv), generator=g, dtype=torch.int32)
    q1 = q[:, -1:].contiguous()
    want = want_of(q1, k, v, ids, lengths)
    for splits in ("4", None):
        print(f"case decode row {dtype} hq={hq} hkv={hkv} splits={splits}", flush=True)
        if splits:
            os.environ["LSA_READ_SPLITS"] = splits
        try:
            got = run(sparse_read_auto, q1, k, v, ids, lengths)
        finally:
            os.environ.pop("LSA_READ_SPLITS", None)
        check(got, want, dtype)
