"""The C ABI without a GPU: the library loads, exports every symbol the headers under
include/ declare (the interface, lsa_rocm.h, and the test hooks, lsa_rocm_testing.h), and its
host-side validation rejects bad arguments before any HIP call."""

import ctypes
import pathlib
import re

import pytest

from lsa_rocm_lab import _abi

HEADERS = sorted((pathlib.Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared() -> list[str]:
    text = "".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(lsa_\w+)\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _abi.load()
    names = declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
        assert name in _abi.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_abi.SIGNATURES) == set(names)


def test_version_and_error_string():
    lib = _abi.load()
    assert lib.lsa_abi_version() == 3
    assert isinstance(lib.lsa_last_error(), bytes)


def test_null_pointers_rejected_before_launch():
    with pytest.raises(ValueError, match="NULL"):
        _abi.call("lsa_read", None, None, None, 1, 1, 1, 8, 8, 2, 64, 1024, 128, 64, None, None, 4, 0, 0.1, 0, 1, None,
                  None, 0, None, None)
    with pytest.raises(ValueError, match="NULL"):
        _abi.call("lsa_select_flat", None, 1, 1, 8, 128, None, None, None, 0, 512, 256, 0, 1, 0, None, None, 64, 1, 32,
                  0, 0, 8192, 8, None, None, 0, None, None, None)


@pytest.mark.parametrize("dim", [8, 100, 512])
def test_bad_index_dim_rejected(dim):
    with pytest.raises(ValueError, match="index dim"):
        _abi.call("lsa_score_rows", 1, 1, 1, 1, dim, 1, 4, 0, 0, 0, 1, None)


def test_bad_head_dim_group_and_alignment_rejected():
    with pytest.raises(ValueError, match="head dim"):
        _abi.call("lsa_read", 16, 16, 16, 1, 1, 1, 8, 8, 2, 48, 768, 96, 48, 16, 16, 4, 0, 0.1, 0, 1, None, None, 0, 16, None)
    with pytest.raises(ValueError, match="group"):
        _abi.call("lsa_read", 16, 16, 16, 1, 1, 1, 8, 6, 4, 64, 2048, 256, 64, 16, 16, 4, 0, 0.1, 0, 1, None, None, 0, 16, None)
    with pytest.raises(ValueError, match="aligned"):
        _abi.call("lsa_read", 18, 16, 16, 1, 1, 1, 8, 8, 2, 64, 1024, 128, 64, 16, 16, 4, 0, 0.1, 0, 1, None, None, 0, 16, None)


def test_workspace_required_for_split_reads():
    need = _abi.size("lsa_read_scratch_bytes", 1, 32, 8, 128, 32)
    assert need == 8 * 32 * 4 * 130 * 4
    with pytest.raises(_abi.LsaError, match="WORKSPACE"):
        _abi.call("lsa_read", 16, 16, 16, 1, 1, 1, 8, 32, 8, 128, 8192, 1024, 128, 16, 16, 4, 1, 0.1, 0, 32, None, None, 0, 16, None)
    with pytest.raises(_abi.LsaError, match="WORKSPACE"):  # scratch without counters
        _abi.call("lsa_read", 16, 16, 16, 1, 1, 1, 8, 32, 8, 128, 8192, 1024, 128, 16, 16, 4, 1, 0.1, 0, 32, None, 16, need, 16, None)
    assert _abi.size("lsa_select_flat_scratch_bytes", 1, 8, 32, 512, 8) == 8 * 512 * 8  # every column key
    assert _abi.size("lsa_select_flat_scratch_bytes", 1, 8, 32, 512, 1) == 0


def test_select_limits_rejected():
    # 8192 columns in one split exceed the LDS key budget
    with pytest.raises(ValueError, match="exceed"):
        _abi.call("lsa_select_flat", 16, 1, 1, 1, 128, 16, 16, None, 0, 8192, 16, 0, 0, 0, 16, None, 512, 64, 32, 0, 0,
                  64, 1, None, None, 0, 16, 16, None)


def _beam_args(levels=3, n_nodes=(1024, 256, 64), **kw):
    """lsa_select_beam arguments at the reference defaults (4096 buckets of cap 16, node
    size 4, block 64, beam 64, top_p 1024) with fake (never dereferenced) pointers."""
    ptrs = (ctypes.c_void_p * max(levels, 1))(*([16] * max(levels, 1)))
    counts = (ctypes.c_int32 * max(levels, 1))(*(list(n_nodes) + [64] * levels)[: max(levels, 1)])
    args = dict(q=16, q_dtype=_abi.LSA_F32, R=1, G=1, D=128, n_levels=levels, cents=ctypes.addressof(ptrs),
                kids=ctypes.addressof(ptrs), n_nodes=ctypes.addressof(counts), node_size=4, node_block=64,
                top_level=3, centroids=16, members=16, ends=None, flags=0, rows=4096, cap=16, row_tables=0,
                group_tables=0, mode=_abi.SCORE_F32, pos=16, slots=None, cbs=512, bb=64, beam=64, top_p=1024, window=512,
                sink=4, top_k=4096, lists=16, lengths=16, stream=None)
    args.update(kw)
    return [ptrs, counts], list(args.values())


def test_beam_arguments_rejected_before_launch():
    keep, args = _beam_args(levels=5, n_nodes=(1024, 256, 64, 16, 4))
    with pytest.raises(ValueError, match="node levels"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(node_block=6)
    with pytest.raises(ValueError, match="multiple of node_size"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(beam=2048)  # 8192 carried children exceed a level's LDS keys
    with pytest.raises(ValueError, match="candidates"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(n_nodes=(1024, 256, 64), rows=16384)  # too many buckets for the dedup bitmap
    with pytest.raises(ValueError, match="buckets"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(n_nodes=(1024, 0, 64))
    with pytest.raises(ValueError, match="level 2"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(cents=None)
    with pytest.raises(ValueError, match="NULL"):
        _abi.call("lsa_select_beam", *args)
    keep, args = _beam_args(flags=_abi.TABLE_SPANS)
    with pytest.raises(ValueError, match="span ends"):
        _abi.call("lsa_select_beam", *args)


def _decode_args(**kw):
    """lsa_decode_flat arguments for a flat 32k decode shape with fake (never dereferenced)
    pointers; kw overrides by name."""
    args = dict(q=16, k=16, v=16, dtype=_abi.LSA_BF16, R=1, Tk=32768, Hq=32, Hkv=8, D=128, sb=0, st=1024, sh=128,
                cent=16, members=16, ends=None, flags=0, rows=512, cap=256, row_tables=0, group_tables=1,
                mode=_abi.SCORE_BF16, pos=16, slots=None, cbs=64, bb=1, top_p=32, window=0, sink=0, top_k=8192,
                scale=0.088,
                splits=16, readers=0, counters=16, n_counters=1 << 20, scratch=16, scratch_bytes=1 << 30, lists=16,
                lengths=16, out=16, status=None, stream=None)
    args.update(kw)
    return list(args.values())


def test_decode_workspace_sizes():
    n = _abi.size("lsa_decode_flat_counters", 1, 8, 512, 32)
    units, K, rows = 8, 32, 512
    stride = ((units * 2 * K + 1023) // 1024) * 1024 + 64
    record = 2 * units + 8 * stride  # arrival counters + 8 record copies
    # then, 256-byte aligned, the rank form's published keys: one u64 per (unit, bucket)
    assert n == (record + 63) // 64 * 64 + 2 * units * rows
    # past 65536 key slots (B=32: 256 units x 512 buckets) the counters hold no keys
    big = _abi.size("lsa_decode_flat_counters", 32, 8, 512, 32)
    assert big == 2 * 256 + 8 * (((256 * 2 * K + 1023) // 1024) * 1024 + 64)
    keys = 8 * 512 * 8  # every column key of 16 select splits
    parts = 8 * 24 * 4 * 130 * 4  # 24 readers' partials per unit (one a pick, at most 24 by default)
    got = _abi.size("lsa_decode_flat_scratch_bytes", _abi.LSA_BF16, 1, 32, 8, 128, 512, 32, 0, 0, 16, 0)
    assert got == ((keys + 255) // 256) * 256 + parts
    assert _abi.size("lsa_decode_flat_counters", 1, 8, 512, 65) == 0  # more than 64 picks is not served


def test_rank_form_limits_match_the_library():
    """pipeline's rank-form limits (the split planner's) are the library's: the counters hold
    the published keys exactly when rows <= _RANK_MAX_ROWS and (row, kv-head, bucket) slots
    <= _RANK_MAX_SLOTS."""
    from lsa_rocm_lab.port import pipeline

    def record_only(R, Hkv, K):
        units = R * Hkv
        return 2 * units + 8 * (((units * 2 * K + 1023) // 1024) * 1024 + 64)

    K = 32
    for R, Hkv, rows in ((16, 8, 512), (17, 8, 512), (1, 8, pipeline._RANK_MAX_ROWS),
                         (1, 8, pipeline._RANK_MAX_ROWS + 4), (1, 2, 2048)):
        fits = rows <= pipeline._RANK_MAX_ROWS and R * Hkv * rows <= pipeline._RANK_MAX_SLOTS
        n = _abi.size("lsa_decode_flat_counters", R, Hkv, rows, K)
        assert (n > record_only(R, Hkv, K)) == fits, (R, Hkv, rows, n)


def test_decode_arguments_rejected_before_launch():
    with pytest.raises(ValueError, match="NULL"):
        _abi.call("lsa_decode_flat", *_decode_args(q=None))
    with pytest.raises(ValueError, match="picks exceed"):
        _abi.call("lsa_decode_flat", *_decode_args(top_p=65))
    with pytest.raises(ValueError, match="group size"):
        _abi.call("lsa_decode_flat", *_decode_args(Hq=24, Hkv=8))
    with pytest.raises(ValueError, match="aligned"):
        _abi.call("lsa_decode_flat", *_decode_args(q=18))
    with pytest.raises(ValueError, match="select splits"):
        _abi.call("lsa_decode_flat", *_decode_args(splits=513))
    with pytest.raises(ValueError, match="readers"):
        _abi.call("lsa_decode_flat", *_decode_args(readers=257))
    with pytest.raises(_abi.LsaError, match="WORKSPACE"):
        _abi.call("lsa_decode_flat", *_decode_args(n_counters=10))
    with pytest.raises(_abi.LsaError, match="WORKSPACE"):
        _abi.call("lsa_decode_flat", *_decode_args(scratch_bytes=1024))
    with pytest.raises(ValueError, match="table flags"):
        _abi.call("lsa_decode_flat", *_decode_args(flags=4))
    with pytest.raises(ValueError, match="span ends"):  # span tables need their ends
        _abi.call("lsa_decode_flat", *_decode_args(flags=_abi.TABLE_SPANS))


def test_chunked_read_paths():
    lib = _abi.load()
    assert lib.lsa_read_chunked_mfma_ok(_abi.LSA_BF16, 128, 64) == 1
    assert lib.lsa_read_chunked_mfma_ok(_abi.LSA_F16, 64, 16) == 1
    assert lib.lsa_read_chunked_mfma_ok(_abi.LSA_F32, 128, 64) == 0
    assert lib.lsa_read_chunked_mfma_ok(_abi.LSA_BF16, 256, 64) == 0
    assert lib.lsa_read_chunked_mfma_ok(_abi.LSA_BF16, 128, 48) == 0
    base = [16, 16, 16, _abi.LSA_F32, 1, 128, 128, 8, 2, 64, 0, 128, 64, 16, 16, 8, 64, None, 0.125]
    with pytest.raises(ValueError, match="MFMA path"):
        _abi.call("lsa_read_chunked", *base, _abi.CHUNKED_MFMA, 16, None)
    with pytest.raises(ValueError, match="path"):
        _abi.call("lsa_read_chunked", *base, 7, 16, None)


def test_segment_build_arguments_rejected_before_launch():
    lib = _abi.load()
    assert lib.lsa_ward_segments_scratch_bytes(8, 32768, 128, 16) == 8 * 2048 * 128 * 8
    assert lib.lsa_ward_segments_scratch_bytes(1, 100, 64, 16) == 7 * 64 * 8  # a shorter last pool
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails its checks first

    def call(**kw):
        a = dict(B=1, T=32768, H=8, D=128, pool=16, target=512, max_size=256, scratch_bytes=1 << 30)
        a.update(kw)
        _abi.call("lsa_ward_segments", p, _abi.LSA_BF16, a["B"], a["T"], a["H"], a["D"], a["T"] * a["H"] * a["D"],
                  a["H"] * a["D"], a["D"], a["pool"], a["target"], a["max_size"], p, a["scratch_bytes"], p, p, None,
                  None)

    with pytest.raises(ValueError, match="NULL"):
        _abi.call("lsa_ward_segments", None, _abi.LSA_BF16, 1, 64, 1, 64, 0, 64, 0, 16, 2, 64, p, 1 << 20, p, p, None,
                  None)
    with pytest.raises(ValueError, match="pools exceed"):
        call(pool=4)  # 8192 pools
    with pytest.raises(ValueError, match="target"):
        call(T=1024, target=65)
    with pytest.raises(ValueError, match="max_size"):
        call(max_size=8)
    with pytest.raises(ValueError, match="scratch"):
        call(scratch_bytes=1024)
    with pytest.raises(ValueError, match="dtype"):
        _abi.call("lsa_ward_segments", p, 9, 1, 64, 1, 64, 0, 64, 0, 16, 2, 64, p, 1 << 20, p, p, None, None)


def _slots(table=16, rows=16, stride=32768, width=32768, n_rows=1):
    return ctypes.pointer(_abi.SlotMap(table, rows, stride, width, n_rows))


def test_slot_maps_rejected_before_launch():
    """A paged cache's slot map (lsa_slot_map) is checked on the host by every entry that
    takes one: a NULL table or rows, no rows, a width below 1 or a stride below the width."""
    for bad, what in ((_slots(table=None), "NULL"), (_slots(rows=None), "NULL"), (_slots(n_rows=0), "n_rows"),
                      (_slots(width=0), "width"), (_slots(stride=100, width=200), "stride")):
        with pytest.raises(ValueError, match=what):
            _abi.call("lsa_decode_flat", *_decode_args(slots=bad))
        with pytest.raises(ValueError, match=what):
            _abi.call("lsa_expand", 16, 0, 1, 1, 32, 16, 512, 16, 0, 0, 16, bad, 0, 0, 64, 16, 16, None)
        with pytest.raises(ValueError, match=what):
            _abi.call("lsa_select_flat", 16, 1, 1, 1, 128, 16, 16, None, 0, 512, 16, 0, 0, 0, 16, bad, 512, 64, 32,
                      0, 0, 64, 1, None, None, 0, 16, 16, None)
        keep, args = _beam_args(slots=bad)
        with pytest.raises(ValueError, match=what):
            _abi.call("lsa_select_beam", *args)
        with pytest.raises(ValueError, match=what):
            _abi.call("lsa_read_chunked", 16, 16, 16, _abi.LSA_BF16, 1, 128, 128, 8, 2, 64, 0, 128, 64, 16, 16, 8, 64,
                      bad, 0.125, _abi.CHUNKED_AUTO, 16, None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_abi, "_lib", None)
    monkeypatch.setattr(_abi, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(_abi.ExtensionMissing):
        _abi.load()
