"""The torch CPU decode step (oracle/cpu_step.py, the CPU comparator bench.py times) equals
the numpy oracle: lists and lengths bit for bit, the read within the fp32 bar (CPU only)."""

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_step

RNG = np.random.default_rng(9)


def span_tables(G, T, n, cap):
    """G tables of n contiguous buckets covering [0, T) (sizes 1..cap), member rows, ends."""
    members = np.full((G, n, cap), -1, np.int32)
    ends = np.zeros((G, n), np.int32)
    step = T // n
    for g in range(G):
        cuts = np.arange(1, n) * step + RNG.integers(-(step // 2) + 1, step // 2, n - 1)
        bounds = np.concatenate([[0], cuts, [T]])
        assert np.diff(bounds).min() >= 1 and np.diff(bounds).max() <= cap
        for j in range(n):
            members[g, j, : bounds[j + 1] - bounds[j]] = np.arange(bounds[j], bounds[j + 1])
        ends[g] = bounds[1:]
    return members, ends


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
@pytest.mark.parametrize("window,sink,top_k", [(0, 0, 4096), (64, 4, 300), (200, 64, 64)])
def test_cpu_step_equals_oracle_span_tables(mode, window, sink, top_k):
    B, T, Hq, Hkv, D, n, cap = 2, 4096, 8, 2, 64, 64, 128
    q = RNG.standard_normal((B, Hq, D)).astype(np.float32)
    k = RNG.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = RNG.standard_normal((B, T, Hkv, D)).astype(np.float32)
    cent = RNG.standard_normal((Hkv, n, D)).astype(np.float32)
    members, ends = span_tables(Hkv, T, n, cap)
    positions = np.array([T - 1, 1500])
    lists, lengths, out = cpu_step.decode_step(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), torch.from_numpy(cent),
        torch.from_numpy(members), torch.from_numpy(ends), torch.from_numpy(positions), cluster_block_size=64,
        block_buckets=1, top_p=16, top_k=top_k, window=window, sink=sink, scale=D ** -0.5, mode=mode)
    idx = oracle.index_queries(q[:, None], Hkv)[:, 0]
    assert np.array_equal(cpu_step.index_queries(torch.from_numpy(q), Hkv).numpy(), idx)
    want_l = np.zeros_like(lists.numpy())
    want_n = np.zeros_like(lengths.numpy())
    for b in range(B):
        for g in range(Hkv):
            l, nn = oracle.flat_select(idx[b, g][None], positions[b:b + 1], cent[g], members[g],
                                       cluster_block_size=64, block_buckets=1, top_p=16, top_k=top_k, window=window,
                                       sink=sink, mode=mode, ends=ends[g])
            want_l[b, g], want_n[b, g] = l[0], nn[0]
    assert np.array_equal(lists.numpy(), want_l)
    assert np.array_equal(lengths.numpy(), want_n)
    want_o = oracle.sparse_read(q[:, None], k, v, want_l[:, None], want_n[:, None], D ** -0.5)[:, 0]
    assert np.abs(out.numpy() - want_o).max() <= 1e-4


def test_cpu_step_positional_tables_and_nothing_visible():
    """Fixed blocks without span ends (visibility by closed blocks), per-row tables, a row
    that sees no bucket (only its window and sinks)."""
    B, T, Hq, Hkv, D, block = 2, 2048, 8, 2, 64, 64
    q = RNG.standard_normal((B, Hq, D)).astype(np.float32)
    k = RNG.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = RNG.standard_normal((B, T, Hkv, D)).astype(np.float32)
    rows = T // block
    members = np.broadcast_to(np.arange(T, dtype=np.int32).reshape(rows, block), (B, Hkv, rows, block)).copy()
    cent = RNG.standard_normal((B, Hkv, rows, D)).astype(np.float32)
    positions = np.array([T - 1, 40])
    lists, lengths, out = cpu_step.decode_step(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), torch.from_numpy(cent),
        torch.from_numpy(members), None, torch.from_numpy(positions), cluster_block_size=block, block_buckets=1,
        top_p=7, top_k=384, window=64, sink=64, scale=D ** -0.5, mode="fp32")
    idx = oracle.index_queries(q[:, None], Hkv)[:, 0]
    for b in range(B):
        for g in range(Hkv):
            l, nn = oracle.flat_select(idx[b, g][None], positions[b:b + 1], cent[b, g], members[b, g],
                                       cluster_block_size=block, block_buckets=1, top_p=7, top_k=384, window=64,
                                       sink=64, mode="fp32")
            assert np.array_equal(lists[b, g].numpy(), l[0]) and int(lengths[b, g]) == nn[0], (b, g)
    assert int(lengths[1, 0]) == 41  # window [0, 40], no sinks past the window start
    want_o = oracle.sparse_read(q[:, None], k, v, lists.numpy()[:, None], lengths.numpy()[:, None], D ** -0.5)
    assert np.abs(out.numpy() - want_o[:, 0]).max() <= 1e-4
