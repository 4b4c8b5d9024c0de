"""Bucket tables on disk (CSR member lists + centroids, safetensors): round trips and the
rejection of malformed files. CPU only; the GPU tests drive the fused select from a loaded
table."""

import dataclasses

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from lsa_rocm_lab.port import tables
from lsa_rocm_lab.port.pipeline import Buckets


def member_table(lead, rows, cap, dim, seed):
    g = torch.Generator().manual_seed(seed)
    sizes = torch.randint(0, cap + 1, (*lead, rows), generator=g, dtype=torch.int32)
    sizes.view(-1)[0] = cap  # a full row
    sizes.view(-1)[1] = 0  # an empty row
    ids = torch.randint(0, 1 << 20, (*lead, rows, cap), generator=g, dtype=torch.int32)
    members = torch.where(torch.arange(cap) < sizes[..., None], ids, -1)
    cent = torch.randn(*lead, rows, dim, generator=g)
    return Buckets(centroids=cent.bfloat16(), members=members, sizes=sizes, centroids_f32=cent)


def span_table(G, lengths, cap, dim):
    ends = torch.tensor(np.cumsum(lengths), dtype=torch.int32).repeat(G, 1)
    begin = torch.cat([torch.zeros(G, 1, dtype=torch.int32), ends[:, :-1]], 1)
    sizes = ends - begin
    members = torch.where(torch.arange(cap) < sizes[..., None], begin[..., None] + torch.arange(cap), -1).int()
    cent = torch.randn(G, len(lengths), dim, generator=torch.Generator().manual_seed(1))
    return Buckets(centroids=cent.bfloat16(), members=members, sizes=sizes, centroids_f32=None, ends=ends, spans=True)


def same(a, b):
    for f in ("centroids", "members", "sizes", "centroids_f32", "ends"):
        x, y = getattr(a, f), getattr(b, f)
        assert (x is None and y is None) or (x.dtype == y.dtype and torch.equal(x, y)), f
    assert a.spans == b.spans
    assert a.block_visible == b.block_visible


@pytest.mark.parametrize("lead,rows,cap,dim", [((), 37, 16, 64), ((8,), 64, 256, 128), ((2, 3), 5, 4, 32)])
def test_member_tables_round_trip(tmp_path, lead, rows, cap, dim):
    b = member_table(lead, rows, cap, dim, seed=rows)
    tables.save_buckets(tmp_path / "t.safetensors", b)
    got = tables.load_buckets(tmp_path / "t.safetensors")
    same(b, got)
    # the CSR layout itself: row r of the flattened tables is member_ids[offsets[r]:offsets[r+1]]
    from safetensors import safe_open
    with safe_open(str(tmp_path / "t.safetensors"), framework="pt") as f:
        off, ids = f.get_tensor("offsets"), f.get_tensor("member_ids")
    flat_m, flat_s = b.members.reshape(-1, cap), b.sizes.reshape(-1)
    r = flat_s.numel() // 2
    assert torch.equal(ids[off[r]:off[r + 1]], flat_m[r, :flat_s[r]])
    assert int(off[-1]) == int(flat_s.sum())


def test_span_tables_round_trip(tmp_path):
    b = span_table(4, [3, 16, 1, 7, 16, 9], 16, 64)
    tables.save_buckets(tmp_path / "s.safetensors", b)
    got = tables.load_buckets(tmp_path / "s.safetensors")
    same(b, got)
    assert got.spans


def test_block_visible_flag_round_trips(tmp_path):
    """Positional tables: span ends with visibility by closed blocks; the flag survives a
    save and load, and a file written before the flag existed reads as span visibility."""
    import dataclasses

    b = dataclasses.replace(span_table(2, [8] * 12, 8, 32), block_visible=True)
    tables.save_buckets(tmp_path / "p.safetensors", b)
    got = tables.load_buckets(tmp_path / "p.safetensors")
    same(b, got)
    assert got.block_visible and got.spans
    plain = span_table(2, [8] * 12, 8, 32)
    tables.save_buckets(tmp_path / "q.safetensors", plain)
    assert not tables.load_buckets(tmp_path / "q.safetensors").block_visible


def test_save_rejects_holes_and_bad_ids(tmp_path):
    b = member_table((2,), 6, 8, 16, seed=4)
    holed = b.members.clone()
    holed[0, 0, 0] = -1  # a hole before real ids of the row
    with pytest.raises(ValueError, match="real ids"):
        tables.save_buckets(tmp_path / "h.safetensors", dataclasses.replace(b, members=holed))
    low = b.members.clone()
    low[1, 2, -1] = -5  # below the padding value
    with pytest.raises(ValueError, match="real ids"):
        tables.save_buckets(tmp_path / "l.safetensors", dataclasses.replace(b, members=low))


def _write(path, tensors, meta):
    save_file(tensors, str(path), metadata=meta)


def test_malformed_files_raise(tmp_path):
    b = member_table((2,), 6, 8, 16, seed=3)
    tables.save_buckets(tmp_path / "ok.safetensors", b)
    from safetensors import safe_open
    with safe_open(str(tmp_path / "ok.safetensors"), framework="pt") as f:
        good = {n: f.get_tensor(n) for n in f.keys()}
        meta = f.metadata()
    cases = {
        "format": ({}, {**meta, "format": "other/1"}),
        "starting at 0": ({"offsets": good["offsets"] + 1}, meta),
        "decrease or exceed": ({"offsets": torch.cat([good["offsets"][:1], good["offsets"][2:3] + 1, good["offsets"][2:]])}, meta),
        "member ids": ({"member_ids": good["member_ids"][:-1]}, meta),
        "exceed bucket_cap": ({}, {**meta, "bucket_cap": "1"}),
        "int64": ({"offsets": good["offsets"].int()}, meta),
        "ends": ({"ends": torch.zeros(2, 5, dtype=torch.int32)}, meta),
        "needs its ends": ({}, {**meta, "spans": "1"}),
        "must be >= 0": ({"member_ids": torch.cat([good["member_ids"][:1] * 0 - 1, good["member_ids"][1:]])}, meta),
        "ends decrease": ({"ends": torch.tensor([[5, 4, 6, 7, 8, 9], [1, 2, 3, 4, 5, 6]], dtype=torch.int32)}, meta),
    }
    for i, (match, (change, m)) in enumerate(cases.items()):
        p = tmp_path / f"bad{i}.safetensors"
        _write(p, {**good, **change}, m)
        with pytest.raises(ValueError, match=match):
            tables.load_buckets(p)
    # a span flag on tables whose rows are not their spans
    s = span_table(1, [2, 3], 4, 8)
    tables.save_buckets(tmp_path / "s.safetensors", s)
    with safe_open(str(tmp_path / "s.safetensors"), framework="pt") as f:
        st = {n: f.get_tensor(n) for n in f.keys()}
        sm = f.metadata()
    st["member_ids"] = st["member_ids"].flip(0).contiguous()
    _write(tmp_path / "s2.safetensors", st, sm)
    with pytest.raises(ValueError, match="spans"):
        tables.load_buckets(tmp_path / "s2.safetensors")
