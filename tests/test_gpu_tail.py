"""What the window/sink tail order leaves open, confined (GPU).

Upstream's ``_append_window_and_sink`` (absent here) fixes the element order inside the
tail of every read list; the reference states only "the expansion, the window, then the
sinks" (read_kernel.py:11-13). This build appends the window ascending, then the sinks
ascending. These tests pin what the mathematics fixes instead: the tail is exactly the
causal set (window [window_start, position], sinks [0, min(sink, window_start))), and the
sparse read's output does not depend on the tail's order (within the dtype's bar), at the
2k fp32 and 32k bf16 block-sparse decode shapes and at a position whose window starts
before the sinks end.
"""

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: (1e-4, 1e-5), torch.bfloat16: (2e-2, 2e-3)}


def _np(t):
    return t.detach().float().cpu().numpy() if t.is_floating_point() else t.detach().cpu().numpy()


CASES = {
    # name: (T, Hq, Hkv, D, dtype, config, positions)
    "decode_2k_fp32": (2048, 8, 2, 64, torch.float32, workloads.DECODE_2K, [2047, 1000]),
    "block_sparse_32k_bf16": (32768, 32, 8, 128, torch.bfloat16, workloads.BLOCK_SPARSE_32K, [32767]),
    "window_before_sinks": (2048, 8, 2, 64, torch.float32, workloads.DECODE_2K, [100, 64, 3]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_tail_is_the_causal_set_and_its_order_is_free(name):
    T, Hq, Hkv, D, dtype, config, positions = CASES[name]
    print(f"case {name}", flush=True)
    q, k, v = workloads.geometry(T, Hq, Hkv, D, dtype=dtype, seed=7, device=DEV)
    buckets = pipeline.position_buckets(k, config, centroid="mean")
    B = len(positions)
    pos = torch.tensor(positions, dtype=torch.int32, device=DEV)
    qrows = q[0, pos.long()].unsqueeze(1)  # [B, 1, Hq, D]: row b is the token at positions[b]
    kk, vv = k.expand(B, -1, -1, -1), v.expand(B, -1, -1, -1)
    idx = pipeline.index_queries(qrows, Hkv)[:, 0]  # [B, Hkv, D]
    lists, lengths = pipeline.flat_select(idx, pos, buckets, config)
    lists_np, lengths_np = _np(lists), _np(lengths)
    gen = np.random.default_rng(11)
    perm = lists_np.copy()
    for b, p in enumerate(positions):
        ws = max(0, p + 1 - config.window_size)
        n_win, n_sink = p + 1 - ws, min(config.sink_size, ws)
        for g in range(Hkv):
            n = int(lengths_np[b, g])
            tail = lists_np[b, g, n - n_win - n_sink:n]
            want = set(range(ws, p + 1)) | set(range(0, min(config.sink_size, ws)))
            assert sorted(tail.tolist()) == sorted(want) and len(tail) == len(want), (name, b, g)
            kept = lists_np[b, g, : n - n_win - n_sink]
            assert ((kept >= config.sink_size) & (kept < ws)).all()  # the kept prefix avoids the tail
            assert (lists_np[b, g, n:] == -1).all()
            perm[b, g, n - n_win - n_sink:n] = gen.permutation(tail)
    assert not np.array_equal(perm, lists_np) or all(p < 2 for p in positions)
    scale = D ** -0.5
    out = pipeline.lsa_read(qrows, kk, vv, lists.unsqueeze(1), lengths.unsqueeze(1), scale)
    out_p = pipeline.lsa_read(qrows, kk, vv, torch.from_numpy(perm).to(DEV).unsqueeze(1), lengths.unsqueeze(1),
                              scale)
    want = oracle.sparse_read(_np(qrows), _np(kk[:1]).repeat(B, 0), _np(vv[:1]).repeat(B, 0),
                              lists_np[:, None], lengths_np[:, None], scale)
    max_abs, mean_abs = TOL[dtype]
    for o in (out, out_p):
        err = np.abs(_np(o) - want)
        assert err.max() <= max_abs and err.mean() <= mean_abs, (name, err.max(), err.mean())
    diff = np.abs(_np(out) - _np(out_p))
    assert diff.max() <= max_abs and diff.mean() <= mean_abs, (name, diff.max())
