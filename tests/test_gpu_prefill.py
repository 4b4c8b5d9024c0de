"""The MFMA tile kernel of the chunked prefill read on the GPU vs the CPU oracle.

Every query row t reads its chunk's shared per-kv-head list (first lengths slots) and the
chunk's causal block [chunk start, t]. Cases: both 16-bit types, head dims 64 and 128,
chunks 16 / 32 / 64 / 128, groups 1 / 2 / 4 / 8 (several workgroups per kv-head when the
group does not fit 256 rows), ragged and empty lists, -1 and out-of-range ids (skipped),
duplicate ids (counted per occurrence), a partial last chunk, two batch rows, a long list
with large score spreads (the lazy rescale), K/V views whose rows lie more than 4 GiB
apart (64-bit gather offsets), and agreement with the gather kernel.
Tolerances (max-abs / mean-abs vs the fp64 oracle): bf16 2e-2 / 2e-3, fp16 5e-3 / 5e-4.
"""

import numpy as np
import pytest
import torch

import oracle
from lsa_rocm_lab import _abi
from lsa_rocm_lab.port.read_kernel_tiled import sparse_read_chunked

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (5e-3, 5e-4)}


def make_case(dtype, B=1, T=256, Tk=None, Hq=8, Hkv=2, D=128, chunk=64, W=160, seed=0, scale=0.5,
              bad_ids=False, empty_every=0):
    g = torch.Generator().manual_seed(seed)
    Tk = Tk or T
    q = (torch.randn(B, T, Hq, D, generator=g) * scale).to(dtype)
    k = (torch.randn(B, Tk, Hkv, D, generator=g) * scale).to(dtype)
    v = torch.randn(B, Tk, Hkv, D, generator=g).to(dtype)
    C = -(-T // chunk)
    ids = torch.full((B, C, Hkv, W), -1, dtype=torch.int32)
    lengths = torch.zeros(B, C, Hkv, dtype=torch.int32)
    for b in range(B):
        for c in range(C):
            for h in range(Hkv):
                if c == 0 or (empty_every and (c + h) % empty_every == 0):
                    continue
                n = int(torch.randint(1, W + 1, (1,), generator=g))
                row = torch.randint(0, c * chunk, (n,), generator=g, dtype=torch.int32)
                if bad_ids:
                    row[::7] = -1
                    row[3::11] = Tk + 5
                ids[b, c, h, :n] = row
                lengths[b, c, h] = n
    return q, k, v, ids, lengths


def run_and_check(q, k, v, ids, lengths, chunk, path="mfma", label=""):
    print(f"case {label} q={tuple(q.shape)} {q.dtype} chunk={chunk} path={path}", flush=True)
    got = sparse_read_chunked(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), None, chunk, path=path)
    ids_np = ids.numpy().copy()
    ids_np[ids_np >= k.shape[1]] = -1  # the oracle indexes rows; out-of-range ids are skipped like -1
    want = oracle.sparse_read_chunked(q.float().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), ids_np,
                                      lengths.numpy(), chunk)
    max_abs, mean_abs = TOL[q.dtype]
    err = np.abs(got.float().cpu().numpy() - want)
    assert np.isfinite(err).all(), label
    assert err.max() <= max_abs and err.mean() <= mean_abs, (label, err.max(), err.mean())
    return got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_mfma_prefill_dtypes_and_dims(dtype, D):
    q, k, v, ids, lengths = make_case(dtype, D=D, seed=D)
    run_and_check(q, k, v, ids, lengths, 64, label=f"D={D}")


@pytest.mark.parametrize("chunk,Hq,Hkv", [(64, 32, 8), (32, 16, 2), (16, 8, 2), (128, 8, 4), (64, 16, 2),
                                          (64, 8, 8)])
def test_mfma_prefill_chunks_and_groups(chunk, Hq, Hkv):
    q, k, v, ids, lengths = make_case(torch.bfloat16, T=512, Hq=Hq, Hkv=Hkv, chunk=chunk, W=200, seed=chunk + Hq)
    run_and_check(q, k, v, ids, lengths, chunk, label=f"chunk={chunk} group={Hq // Hkv}")


def test_mfma_prefill_bad_ids_empty_lists_partial_chunk_batch():
    q, k, v, ids, lengths = make_case(torch.bfloat16, B=2, T=300, Tk=320, W=150, seed=5, bad_ids=True,
                                      empty_every=3)
    run_and_check(q, k, v, ids, lengths, 64, label="ragged")


def test_mfma_prefill_duplicates_and_long_lists():
    """A long list (many tiles) of repeated ids with a wide score spread: the running max
    grows in steps, exercising the lazy rescale, and duplicates count per occurrence."""
    q, k, v, ids, lengths = make_case(torch.bfloat16, T=1024, W=900, seed=9, scale=2.0)
    ids[..., 1::2] = ids[..., 0::2]  # every id twice
    run_and_check(q, k, v, ids, lengths, 64, label="long")


def test_mfma_prefill_wide_token_stride():
    """K/V rows 9.4 M elements apart (views into a 4.8 GB cache, read in place): byte
    offsets past 4 GiB take the kernel's 64-bit gather addresses."""
    q, k, v, ids, lengths = make_case(torch.bfloat16, T=256, Hq=8, Hkv=2, W=160, seed=21)
    Tk, Hkv, D = k.shape[1], k.shape[2], k.shape[3]
    stride = (1 << 23) + (1 << 20)
    assert (Tk - 1) * stride * 2 >= 1 << 32
    base = torch.empty(Tk, stride, dtype=torch.bfloat16, device=DEV)
    kd = torch.as_strided(base, (1, Tk, Hkv, D), (Tk * stride, stride, D, 1))
    vd = torch.as_strided(base, (1, Tk, Hkv, D), (Tk * stride, stride, D, 1), Hkv * D)
    kd.copy_(k.to(DEV))
    vd.copy_(v.to(DEV))
    run_and_check(q, kd, vd, ids, lengths, 64, label="wide stride")
    del kd, vd, base


def test_mfma_and_gather_paths_agree():
    q, k, v, ids, lengths = make_case(torch.bfloat16, T=512, Hq=32, Hkv=8, W=300, seed=11)
    a = sparse_read_chunked(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), None, 64, path="mfma")
    b = sparse_read_chunked(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), None, 64, path="gather")
    assert (a.float() - b.float()).abs().max().item() <= 2e-2


def test_mfma_path_rejects_unsupported_shapes():
    q, k, v, ids, lengths = make_case(torch.float32, T=128, D=64, W=16)
    with pytest.raises(ValueError, match="MFMA path"):
        sparse_read_chunked(q.to(DEV), k.to(DEV), v.to(DEV), ids.to(DEV), lengths.to(DEV), None, 64, path="mfma")
    assert _abi.load().lsa_read_chunked_mfma_ok(_abi.LSA_BF16, 128, 64) == 1
    assert _abi.load().lsa_read_chunked_mfma_ok(_abi.LSA_F32, 128, 64) == 0
