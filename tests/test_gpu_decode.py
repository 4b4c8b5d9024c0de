"""The fused decode step (index queries + flat select + sparse read in one launch) on the GPU.

Lists and lengths must equal, bit for bit, the oracle's flat select on the group-mean index
queries (and so the unfused HIP select's); the output must match the oracle's sparse read of
those lists within the dtype's bar (max-abs / mean-abs vs fp64: fp32 1e-4 / 1e-5, bf16
2e-2 / 2e-3). Cases: the clustered decode geometry up to 32k, positional buckets with
window and sink tails, top_k cutting a bucket short, fewer visible buckets than picks,
nothing visible (zeros), batch rows with their own tables and positions, every select
split count, reader counts from 1 to 256, both hand-off forms (the rank form, span and member tables: every reader ranks the
splits' published keys; with one split, the select's record), both
scoring dtypes, and repeated launches (the record or published keys, counters and
partials are reused and must come back clean).
"""

import dataclasses

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.pipeline import PortConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: (1e-4, 1e-5), torch.bfloat16: (2e-2, 2e-3), torch.float16: (5e-3, 5e-4)}


def _np(t):
    return t.detach().cpu().numpy()


def oracle_decode(q, k, v, positions, buckets, config, score_dtype, top_k=None):
    """Oracle lists/lengths [B, Hkv, W] / [B, Hkv] and output [B, 1, Hq, D]."""
    top_k = config.top_k if top_k is None else top_k
    B, _, Hq, D = q.shape
    Hkv = k.shape[2]
    idx = oracle.index_queries(q.float().cpu().numpy(), Hkv)[:, 0]  # [B, Hkv, D]
    per_row = buckets.members.dim() == 4
    cents = buckets.centroids_f32 if score_dtype == "fp32" else buckets.centroids.float()
    lists, lengths = [], []
    for b in range(B):
        lb, nb = [], []
        for g in range(Hkv):
            sel = (b, g) if per_row else (g,)
            ve = pipeline.visible_ends(buckets)
            ends = None if ve is None else _np(ve[sel])
            l, n = oracle.flat_select(idx[b, g][None], np.array([int(positions[b])]), _np(cents[sel]),
                                      _np(buckets.members[sel]), cluster_block_size=config.cluster_block_size,
                                      block_buckets=config.block_bucket_count, top_p=config.top_p, top_k=top_k,
                                      window=config.window_size, sink=config.sink_size, mode=score_dtype, ends=ends)
            lb.append(l[0])
            nb.append(n[0])
        lists.append(np.stack(lb))
        lengths.append(np.array(nb))
    lists, lengths = np.stack(lists), np.stack(lengths)
    out = oracle.sparse_read(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                             lists[:, None], lengths[:, None], D ** -0.5)
    return lists, lengths, out


def check_decode(q, k, v, positions, buckets, config, score_dtype="bf16", top_k=None, splits=None, label="",
                 readers=None):
    print(f"case {label} B={q.shape[0]} Hq={q.shape[2]} D={q.shape[3]} {q.dtype} {score_dtype} splits={splits} "
          f"readers={readers}", flush=True)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    out, lists, lengths = pipeline.flat_decode(q, k, v, positions.to(DEV), buckets, config, top_k=top_k,
                                               score_dtype=score_dtype, splits=splits, readers=readers,
                                               status=status)
    want_l, want_n, want_o = oracle_decode(q, k, v, positions, buckets, config, score_dtype, top_k)
    assert int(status.item()) == 0
    assert np.array_equal(_np(lengths), want_n), label
    assert np.array_equal(_np(lists), want_l), label
    max_abs, mean_abs = TOL[q.dtype]
    err = np.abs(_np(out.float()) - want_o)
    assert np.isfinite(err).all(), label
    assert err.max() <= max_abs and err.mean() <= mean_abs, (label, err.max(), err.mean())
    return out, lists, lengths


@pytest.mark.parametrize("splits", [1, 3, 16, None])
def test_clustered_decode_matches_oracle(splits):
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=4, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    pos = torch.tensor([T - 1], dtype=torch.int32)
    check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K, splits=splits,
                 label=f"clustered splits={splits}")


@pytest.mark.parametrize("form", ["spans", "members"])
@pytest.mark.parametrize("splits", [48, 100])
def test_select_splits_past_the_table(form, splits):
    """More select splits than the table's columns fill: with 128 buckets, 48 splits take 3
    columns each and splits 43..47 start past the table (100 splits: 2 columns, 64..99
    empty). An empty split scores nothing and still publishes; its loads stay inside the
    table. Span tables and member tables (the rank form counts the picks' members from
    their rows). Lists bit-exact vs the oracle."""
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=5, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    rows = buckets.rows
    assert buckets.spans and (splits - 1) * -(-rows // splits) >= rows  # the last split is empty
    if form == "members":
        buckets = dataclasses.replace(buckets, spans=False)
    pos = torch.tensor([T - 1], dtype=torch.int32)
    check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K, splits=splits,
                 label=f"{form} splits={splits} rows=128")


@pytest.mark.parametrize("form", ["rank", "record"])
@pytest.mark.parametrize("readers", [1, 2, 5, 40, 256])
def test_reader_counts_match_oracle(form, readers):
    """Any reader count splits a unit's list the same way. The list here holds 44 tiles of
    64 slots (32 buckets' keys below the window, then a 1024-key window and 4 sinks: 2782 and
    2764 slots): one reader writes
    the output itself (no partials); 2 and 5 leave a remainder of tiles; 40 publish more
    partials than the combine's first batch of loads covers; 256 (the most the host accepts)
    leave readers without a tile, which still write their share of the list's padding and
    arrive. Both hand-off forms (the rank form: 8 select splits publish keys; the record: one
    split). Lists bit-exact vs the oracle, output within the bf16 bar."""
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=6, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    config = dataclasses.replace(workloads.FLAT_32K, window_size=1024, sink_size=4)
    pos = torch.tensor([T - 1], dtype=torch.int32)
    _, _, lengths = check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, config,
                                 splits=8 if form == "rank" else 1, readers=readers, label=f"{form} readers={readers}")
    assert _np(lengths).min() > 40 * 64  # more tiles than 40 readers take one each


@pytest.mark.parametrize("dtype,hq,hkv", [(torch.bfloat16, 8, 8), (torch.bfloat16, 8, 4), (torch.bfloat16, 16, 2),
                                          (torch.float16, 8, 2), (torch.float16, 16, 2), (torch.float16, 4, 4)])
def test_matrix_core_decode_group_sizes(dtype, hq, hkv):
    """The fused decode on 16-bit rows of D = 128 reads on the matrix cores for 1, 2, 4 and
    8 query heads a kv-head, in bf16 and fp16; lists bit-exact, outputs within the dtype's
    bar."""
    T, D = 8192, 128
    data = workloads.clustered(T, hq, hkv, D, n_clusters=128, seed=hq + hkv, dtype=dtype, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    pos = torch.tensor([T - 1], dtype=torch.int32)
    check_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K,
                 label=f"mfma decode {dtype} hq={hq} hkv={hkv}")


def test_decode_32k_geometry_matches_unfused_path(monkeypatch):
    """The benchmark geometry: 32k context, Hq 32 / Hkv 8, 512 buckets per kv-head."""
    T, Hq, Hkv, D = 32768, 32, 8, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=512, seed=1, device=DEV)
    buckets = workloads.cluster_buckets(data, target=512)
    config = workloads.FLAT_32K
    pos = torch.tensor([T - 1], dtype=torch.int32)
    q = data.q[:, -1:]
    out, lists, lengths = check_decode(q, data.k, data.v, pos, buckets, config, label="32k")
    monkeypatch.setenv("LSA_SELECT_IMPL", "fused")
    idx = pipeline.index_queries(q, Hkv)[0]
    l2, n2 = pipeline.flat_select(idx, pos.to(DEV), buckets, config)
    assert torch.equal(lists, l2) and torch.equal(lengths, n2)  # [1, Hkv, W], [1, Hkv]
    o2 = pipeline.lsa_read(q, data.k, data.v, l2.unsqueeze(0), n2.unsqueeze(0), D ** -0.5)
    assert (out.float() - o2.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("top_k", [100, 2000])
@pytest.mark.parametrize("score_dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_positional_window_sink_and_truncation(score_dtype, dtype, top_k):
    """Window + sink tails, top_k cutting the expansion inside a bucket (100), positions that
    see fewer buckets than picks (32 per closed block, 48 picks) or none (only the window) -
    one launch over batch rows with their own tables."""
    T, Hq, Hkv, D = 4096, 8, 2, 64
    g = torch.Generator().manual_seed(20261201)
    B = 3
    q = (torch.randn(B, 1, Hq, D, generator=g) * 0.5).to(dtype).to(DEV)
    k = (torch.randn(B, T, Hkv, D, generator=g) * 0.5).to(dtype).to(DEV)
    v = torch.randn(B, T, Hkv, D, generator=g).to(dtype).to(DEV)
    config = PortConfig(cluster_block_size=512, bucket_size=16, bucket_cap=16, top_p=48, top_k=top_k,
                        window_size=128, sink_size=4)
    buckets = pipeline.position_buckets(k, config, centroid="mean")  # [B, Hkv, rows, ...]
    for positions in ([T - 1, 1500, 700], [5, 513, 4000]):
        pos = torch.tensor(positions, dtype=torch.int32)
        check_decode(q, k, v, pos, buckets, config, score_dtype=score_dtype,
                     label=f"positional {positions} top_k={top_k}")


def test_nothing_visible_gives_zeros_and_empty_lists():
    T, Hq, Hkv, D = 2048, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=32, seed=6, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    pos = torch.tensor([3], dtype=torch.int32)  # no bucket ends at or before position 4
    out, lists, lengths = check_decode(data.q[:, :1], data.k, data.v, pos, buckets, workloads.FLAT_32K,
                                       label="nothing visible")
    assert int(lengths.max().item()) == 0 and torch.all(lists == -1)
    assert torch.all(out == 0)


def test_repeated_launches_reuse_workspace():
    """Three launches in a row on one stream with different queries and positions: the
    record, the arrival counters and the partials left by one launch serve the next."""
    T, Hq, Hkv, D = 8192, 16, 4, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=64, seed=7, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    for step, p in enumerate((T - 1, T - 300, 5000)):
        pos = torch.tensor([p], dtype=torch.int32)
        check_decode(data.q[:, p:p + 1], data.k, data.v, pos, buckets, workloads.FLAT_32K, label=f"repeat {step}")


def test_decode_deterministic():
    T, Hq, Hkv, D = 4096, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=64, seed=8, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    first = pipeline.flat_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K)
    for _ in range(3):
        again = pipeline.flat_decode(data.q[:, -1:], data.k, data.v, pos, buckets, workloads.FLAT_32K)
        assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_rejects_cpu_tensors_and_bad_shapes():
    data = workloads.clustered(1024, 8, 2, 128, n_clusters=16, seed=9, device=DEV)
    buckets = workloads.cluster_buckets(data, target=16)
    pos = torch.tensor([1023], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        pipeline.flat_decode(data.q[:, -1:].cpu(), data.k, data.v, pos, buckets, workloads.FLAT_32K)
    with pytest.raises(ValueError):
        pipeline.flat_decode(data.q[:, -2:], data.k, data.v, pos, buckets, workloads.FLAT_32K)


@pytest.mark.parametrize("window,sink", [(0, 0), (100, 4)])
def test_span_tables_match_member_tables(window, sink):
    """Contiguous-segment tables decoded through their spans (LSA_TABLE_SPANS: counts and
    ids from the ends, no member rows) and through their member rows give the same lists,
    lengths and outputs, and both match the oracle; the window and sink clip some picks'
    spans at both ends."""
    import dataclasses

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=11, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    assert buckets.spans
    config = dataclasses.replace(workloads.FLAT_32K, window_size=window, sink_size=sink)
    for p in (T - 1, 3000):
        pos = torch.tensor([p], dtype=torch.int32)
        q = data.q[:, p:p + 1]
        got = check_decode(q, data.k, data.v, pos, buckets, config, label=f"spans p={p}")
        ref = check_decode(q, data.k, data.v, pos, dataclasses.replace(buckets, spans=False), config,
                           label=f"members p={p}")
        assert all(torch.equal(a, b) for a, b in zip(got, ref))


def test_tied_scores_take_the_block_top_k():
    """Every centroid equal: all scores tie, the one-wave histogram cut is not selective
    (every key in one bin) and the block's radix top-k decides; ties go to the lower
    bucket, so the picks are buckets 0..31 in order."""
    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=64, seed=12, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    import dataclasses

    same = buckets.centroids[..., :1, :].expand_as(buckets.centroids).contiguous()
    tied = dataclasses.replace(buckets, centroids=same, centroids_f32=same.float())
    pos = torch.tensor([T - 1], dtype=torch.int32)
    out, lists, lengths = check_decode(data.q[:, -1:], data.k, data.v, pos, tied, workloads.FLAT_32K,
                                       label="tied scores")
    ends = tied.ends.cpu()
    for g in range(Hkv):
        n = int(ends[g, 31])  # buckets 0..31 are the spans [0, ends[31])
        assert int(lengths[0, g]) == n
        assert torch.equal(lists[0, g, :n].cpu(), torch.arange(n, dtype=torch.int32))


@pytest.mark.parametrize("case", ["pos-inf", "neg-inf", "half-tied", "half-tied-32k", "top1", "top17", "early"])
def test_rank_form_register_top_k_edges(case):
    """The rank form's readers rank up to 32 picks in registers: the K-th best lane maximum's
    16-bit score prefix bounds the candidates, a 64-lane bitonic sort ranks them, and more
    than 64 candidates fall back to the binned ranking. Lists must still equal the oracle's
    at the edges of that scheme: infinite scores (ranked by their packed keys like any
    other), half the buckets tied (ties go to the lower bucket; the tied keys share every
    prefix), one and 17 picks, and a position with fewer visible buckets than picks."""
    T = 32768 if case.endswith("32k") else 8192
    Hq, Hkv, D = 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=21, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    config = workloads.FLAT_32K
    pos = torch.tensor([T - 1], dtype=torch.int32)
    cent = buckets.centroids.clone()
    if case == "pos-inf":
        cent[0, 5, 3] = float("inf")
        cent[1, 9, 7] = float("inf")
    elif case == "neg-inf":
        cent[0, 5, 3] = float("-inf")
        cent[1, 100, 7] = float("-inf")
    elif case.startswith("half-tied"):
        n = cent.shape[1]
        cent[:, n // 2:] = cent[:, :1]  # the upper half all score like bucket 0
    elif case == "top1":
        config = dataclasses.replace(config, top_p=1)
    elif case == "top17":
        config = dataclasses.replace(config, top_p=17)
    elif case == "early":
        pos = torch.tensor([700], dtype=torch.int32)
    odd = dataclasses.replace(buckets, centroids=cent, centroids_f32=cent.float())
    check_decode(data.q[:, -1:], data.k, data.v, pos, odd, config, label=f"register top-k {case}")


@pytest.mark.parametrize("form", ["rank-spans", "rank-members", "record"])
def test_give_up_is_reported_and_the_next_launch_is_clean(form):
    """The host makes every reader's bounded wait give up (select workgroups skip
    publishing, a 64-poll limit): all workgroups exit normally, the status word reads 1,
    the next flat_decode call zeroes the counters and raises, and the launch after it is
    bit-identical to one before the failure. Both hand-offs: with two splits the readers
    wait for the splits' published keys (rank form; span and member tables), with one
    split for the select's record."""
    from lsa_rocm_lab import _abi

    T, Hq, Hkv, D = 4096, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=64, seed=31, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    assert buckets.spans
    if form == "rank-members":
        buckets = dataclasses.replace(buckets, spans=False)
    config = PortConfig(cluster_block_size=64, bucket_size=64, bucket_cap=256, top_p=16, top_k=4096,
                        window_size=64, sink_size=4)
    q = data.q[:, -1:].contiguous()
    pos = torch.tensor([T - 1], dtype=torch.int32, device=DEV)
    splits = 1 if form == "record" else 2
    run = lambda: pipeline.flat_decode(q, data.k, data.v, pos, buckets, config, splits=splits)
    good = run()
    torch.cuda.synchronize()
    word = _abi.StatusWord.get(torch.device(DEV))
    assert int(word[0]) == 0
    lib = _abi.load()
    print(f"case give-up ({form} form): skip_publish=1 spin_limit=64", flush=True)
    lib.lsa_debug_decode(1, 64)
    try:
        run()
        torch.cuda.synchronize()
    finally:
        lib.lsa_debug_decode(0, 0)
    assert int(word[0]) == 1
    with pytest.raises(_abi.LsaError, match="gave up"):
        run()
    assert int(word[0]) == 0
    again = run()
    torch.cuda.synchronize()
    for a, b in zip(good, again):
        assert torch.equal(a, b)
    pipeline.check_decode()  # nothing pending


REP_CASES = {
    # label: (T, Hq, Hkv, D, dtype, B, positions, window, sink, top_p)
    "8k bf16 hq8 hkv2": (8192, 8, 2, 128, torch.bfloat16, 1, [8191], 0, 0, 32),
    "32k bf16 hq32 hkv8": (32768, 32, 8, 128, torch.bfloat16, 1, [32767], 0, 0, 32),
    "8k fp16 hq16 hkv2": (8192, 16, 2, 128, torch.float16, 1, [8191], 0, 0, 32),
    "4k fp32 hq8 hkv2": (4096, 8, 2, 128, torch.float32, 1, [4095], 0, 0, 32),
    "4k bf16 d64 hq8 hkv8": (4096, 8, 8, 64, torch.bfloat16, 1, [4095], 0, 0, 16),
    "8k bf16 window sink": (8192, 8, 2, 128, torch.bfloat16, 1, [8191], 300, 4, 32),
    "8k bf16 ragged rows": (8192, 8, 2, 128, torch.bfloat16, 3, [8191, 3000, 40], 64, 4, 48),
    "8k bf16 one pick": (8192, 8, 2, 128, torch.bfloat16, 1, [8191], 0, 0, 1),
}


@pytest.mark.parametrize("label", list(REP_CASES))
def test_replicated_select_equals_exchange_and_oracle(label):
    """The replicated form (every reader selects for itself: matrix-core screen, exact
    re-score of the rows near the cut) against the oracle, and bit-identical to the
    exchange form (select workgroups publishing the picks): lists, lengths and outputs."""
    import dataclasses

    T, Hq, Hkv, D, dtype, B, positions, window, sink, top_p = REP_CASES[label]
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=T // 64, seed=13, dtype=dtype, B=B, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    assert buckets.spans
    config = dataclasses.replace(workloads.FLAT_32K, window_size=window, sink_size=sink, top_p=top_p)
    pos = torch.tensor(positions, dtype=torch.int32)
    q = torch.stack([data.q[b, p] for b, p in enumerate(positions)])[:, None]  # [B, 1, Hq, D]
    rep = check_decode(q, data.k, data.v, pos, buckets, config, splits=0, label=f"rep {label}")
    exch = pipeline.flat_decode(q, data.k, data.v, pos.to(DEV), buckets, config, splits=2)
    for a, b in zip(rep, exch):
        assert torch.equal(a, b), label


def test_replicated_select_non_finite_takes_the_exact_path():
    """A centroid holding +inf: its screen and bound are not finite, so the readers score
    every row exactly (the bucket lands first or last by the sign of its score); lists
    equal the oracle's and the exchange form's."""
    import dataclasses

    T, Hq, Hkv, D = 8192, 8, 2, 128
    data = workloads.clustered(T, Hq, Hkv, D, n_clusters=128, seed=14, device=DEV)
    buckets = workloads.cluster_buckets(data, target=T // 64)
    cent = buckets.centroids.clone()
    cent[0, 5, 3] = float("inf")
    cent[1, 9, 7] = float("inf")
    odd = dataclasses.replace(buckets, centroids=cent, centroids_f32=cent.float())
    pos = torch.tensor([T - 1], dtype=torch.int32)
    rep = check_decode(data.q[:, -1:], data.k, data.v, pos, odd, workloads.FLAT_32K, splits=0, label="rep inf")
    exch = pipeline.flat_decode(data.q[:, -1:], data.k, data.v, pos.to(DEV), odd, workloads.FLAT_32K, splits=2)
    for a, b in zip(rep, exch):
        assert torch.equal(a, b)
