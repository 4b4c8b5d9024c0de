"""Golden fixtures of the select+read path (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle still reproduces every fixture from its seeded inputs (the inputs'
sha256 is checked first, so a change of the torch generator shows up as a skip, not as a
false failure). GPU: the HIP path - fused select, per-kv-head lists, split read - gives
the fixture's lists and lengths bit for bit and its output within the dtype's bar.
"""

import hashlib
import pathlib

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import workloads
from lsa_rocm_lab.port import pipeline
from lsa_rocm_lab.port.pipeline import Buckets

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
CASES = {
    "decode_2k_fp32": dict(kind="positional", T=2048, Hq=8, Hkv=2, D=64, dtype=torch.float32,
                           config=workloads.DECODE_2K, tol=(1e-4, 1e-5)),
    "block_sparse_4k_bf16": dict(kind="positional", T=4096, Hq=8, Hkv=2, D=128, dtype=torch.bfloat16,
                                 config=workloads.BLOCK_SPARSE_32K, tol=(2e-2, 2e-3)),
    "flat_clustered_4k_bf16": dict(kind="clustered", T=4096, Hq=8, Hkv=2, D=128, n_clusters=64, seed=5,
                                   config=workloads.FLAT_32K, tol=(2e-2, 2e-3)),
}


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def fixture(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def inputs(name, device="cpu"):
    c = CASES[name]
    if c["kind"] == "positional":
        q, k, v = workloads.geometry(c["T"], c["Hq"], c["Hkv"], c["D"], dtype=c["dtype"], seed=0, device=device)
        return q, k, v, None
    data = workloads.clustered(c["T"], c["Hq"], c["Hkv"], c["D"], n_clusters=c["n_clusters"], seed=c["seed"],
                               device=device)
    return data.q, data.k, data.v, data


def checked_inputs(name, device="cpu"):
    q, k, v, data = inputs(name, device)
    fx = fixture(name)
    if sha(*(t.float().cpu().numpy() for t in (q, k, v))) != str(fx["input_sha256"]):
        pytest.skip(f"{name}: the seeded generator no longer reproduces the fixture inputs (torch changed)")
    return q, k, v, data, fx


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_golden(name):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    make_golden = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(make_golden)
    checked_inputs(name)
    case = next(c for c in make_golden.cases() if c["name"] == name)
    fx = fixture(name)
    assert np.array_equal(case["lists"], fx["lists"]) and np.array_equal(case["lengths"], fx["lengths"])
    assert np.array_equal(case["out"], fx["out"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_path_matches_golden(name, monkeypatch):
    c = CASES[name]
    q, k, v, data, fx = checked_inputs(name, device="cuda")
    config = c["config"]
    if c["kind"] == "positional":
        buckets = pipeline.position_buckets(k, config, centroid="mean")
        score_dtype = "fp32" if c["dtype"] == torch.float32 else "bf16"
    else:
        members, sizes, ends = workloads.segment_tables(fx["starts"], config.bucket_cap, "cuda")
        c32, c16 = pipeline.bucket_centroids(k, members, "mean")
        buckets = Buckets(c16, members, sizes, centroids_f32=c32, ends=ends)
        score_dtype = "bf16"
    monkeypatch.setenv("LSA_SELECT_IMPL", "fused")
    idx = pipeline.index_queries(q[:, -1:], c["Hkv"])[0]
    pos = torch.tensor([c["T"] - 1], device="cuda", dtype=torch.int32)
    lists, lengths = pipeline.flat_select(idx, pos, buckets, config, score_dtype=score_dtype)
    out = pipeline.lsa_read(q[:, -1:], k, v, lists.unsqueeze(0), lengths.unsqueeze(0), c["D"] ** -0.5)
    assert np.array_equal(lists[0].cpu().numpy(), fx["lists"])
    assert np.array_equal(lengths[0].cpu().numpy(), fx["lengths"])
    err = np.abs(out.float().cpu().numpy() - fx["out"])
    max_abs, mean_abs = c["tol"]
    assert err.max() <= max_abs and err.mean() <= mean_abs, (err.max(), err.mean())
