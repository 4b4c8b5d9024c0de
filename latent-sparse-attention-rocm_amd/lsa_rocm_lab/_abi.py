"""ctypes binding of liblsa_rocm.so (the C ABI in include/lsa_rocm.h).

The library is loaded after ``torch`` so that it shares torch's HIP runtime (one
device context, one set of streams). Every call passes raw device pointers and
``torch.cuda.current_stream().cuda_stream``; nothing here computes on the host.
If the library is missing the first call raises ``ExtensionMissing`` - there is
no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(os.environ.get("LSA_ROCM_LIB", pathlib.Path(__file__).parent / "_lib" / "liblsa_rocm.so"))

LSA_F32, LSA_BF16, LSA_F16 = 0, 1, 2
CHUNKED_AUTO, CHUNKED_GATHER, CHUNKED_MFMA = 0, 1, 2
SCORE_BF16, SCORE_F32 = 0, 1
TABLE_SPANS = 1  # LSA_TABLE_SPANS: every bucket row holds exactly its span of `ends`
TABLE_BLOCK_VISIBLE = 2  # LSA_TABLE_BLOCK_VISIBLE: visibility by closed blocks, ends for spans only
BEAM_MAX_LEVELS = 4  # LSA_BEAM_MAX_LEVELS: node levels lsa_select_beam walks
CENTROID_MEAN, CENTROID_NORMALIZED, CENTROID_SUM = 0, 1, 2

_ERRORS = {
    -1: "LSA_ERR_NULL",
    -2: "LSA_ERR_SHAPE",
    -3: "LSA_ERR_DTYPE",
    -4: "LSA_ERR_POW2",
    -5: "LSA_ERR_WORKSPACE",
    -6: "LSA_ERR_LAUNCH",
    -7: "LSA_ERR_ALIGN",
}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/lsa_rocm.h
SIGNATURES = {
    "lsa_abi_version": (_int, []),
    "lsa_last_error": (ctypes.c_char_p, []),
    "lsa_debug_decode": (None, [_i32, _i32]),
    "lsa_visible_counts": (_int, [_p, _i64, _i32, _i32, _i32, _i32, _p, _i64, _i64, _p, _p]),
    "lsa_score_rows": (_int, [_p, _int, _i64, _i32, _i32, _p, _i32, _i64, _i64, _int, _p, _p]),
    "lsa_pack_listing": (_int, [_p, _p, _i64, _i32, _p, _p]),
    "lsa_topk_keys": (_int, [_p, _p, _i64, _i32, _i32, _p, _p]),
    "lsa_select_topk_scores": (_int, [_p, _p, _i64, _i32, _i32, _p, _p]),
    "lsa_unpack_ids": (_int, [_p, _i64, _p, _p]),
    "lsa_expand": (_int, [_p, _int, _i64, _i32, _i32, _p, _i32, _i32, _i64, _i64, _p, _p, _i32, _i32, _i32, _p, _p,
                          _p]),
    "lsa_select_flat_scratch_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "lsa_select_flat": (_int, [_p, _int, _i64, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i64, _i64, _int, _p, _p, _i32,
                               _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _sz, _p, _p, _p]),
    "lsa_select_tree": (_int, [_p, _int, _i64, _i32, _i32, _p, _p, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i64, _i64,
                               _int, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "lsa_select_beam": (_int, [_p, _int, _i64, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _p, _p, _p, _i32, _i32,
                               _i32, _i64, _i64, _int, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p,
                               _p]),
    "lsa_index_queries": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p]),
    "lsa_bucket_centroids": (_int, [_p, _int, _i64, _i64, _i64, _i32, _i32, _p, _i64, _i32, _i32, _int, _p, _p, _p]),
    "lsa_ward_segments_scratch_bytes": (_sz, [_i64, _i64, _i32, _i32]),
    "lsa_ward_segments": (_int, [_p, _int, _i64, _i64, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _p, _sz, _p,
                                 _p, _p, _p]),
    "lsa_read_scratch_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "lsa_read_tile_tokens": (_i32, [_int, _i32, _i32]),
    "lsa_read": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _i32, _int,
                        _f32, _int, _i32, _p, _p, _sz, _p, _p]),
    "lsa_read_chunked": (_int, [_p, _p, _p, _int, _i64, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _i32,
                                _i32, _p, _f32, _i32, _p, _p]),
    "lsa_read_chunked_mfma_ok": (_int, [_int, _i32, _i32]),
    "lsa_decode_flat_counters": (_i64, [_i64, _i32, _i32, _i32]),
    "lsa_decode_flat_rep_ok": (_int, [_int, _i32, _i32, _i32, _i32, _int, _i32]),
    "lsa_decode_flat_scratch_bytes": (_sz, [_int, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "lsa_decode_flat": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _p, _i32, _i32,
                               _i32, _i64, _i64, _int, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32,
                               _p, _i64, _p, _sz, _p, _p, _p, _p, _p]),
    "lsa_decode_tree": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _i32, _i32,
                               _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i64, _i64, _int, _p, _p, _i32, _i32, _i32,
                               _i32, _i32, _i32, _f32, _i32, _p, _i64, _p, _sz, _p, _p, _p, _p, _p]),
    "lsa_decode_shared_counters": (_i64, [_i64, _i32, _i32]),
    "lsa_decode_shared_scratch_bytes": (_sz, [_int, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "lsa_decode_shared": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _p, _i32,
                                 _i32, _i64, _int, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p,
                                 _i64, _p, _sz, _p, _p, _p, _p, _p]),
    "lsa_decode_tree_shared_counters": (_i64, [_i64, _i32, _i32, _p, _i32]),
    "lsa_decode_tree_shared": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _i32, _p,
                                      _p, _p, _i32, _i32, _i32, _p, _p, _i32, _i32, _i64, _int, _p, _p, _i32, _i32,
                                      _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _i64, _p, _sz, _p, _p, _p,
                                      _p, _p]),
    "lsa_decode_flat_noalloc": (_int, [_p, _p, _p, _int, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _p, _p, _p,
                                       _i32, _i32, _i32, _i64, _i64, _int, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                                       _f32, _i32, _i32, _i32, _p, _p, _p, _p, _p]),
}


class ExtensionMissing(RuntimeError):
    """liblsa_rocm.so is not built or cannot be loaded: the HIP path cannot run."""


class LsaError(RuntimeError):
    """A launch-level failure reported by the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{_ERRORS.get(code, code)}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads the library once (after torch) and binds every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.is_file():
                raise ExtensionMissing(
                    f"{LIB_PATH} is missing - build it with __graft_entry__.build() "
                    "(hipcc --offload-arch=gfx950); the select+read path has no CPU fallback")
            try:
                lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            except OSError as exc:
                raise ExtensionMissing(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args):
    """Calls an entry point; a nonzero status raises (ValueError for argument errors)."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = load().lsa_last_error().decode(errors="replace")
        if rc in (-1, -2, -3, -4, -7):
            raise ValueError(f"{name}: {_ERRORS.get(rc, rc)}: {msg}")
        raise LsaError(rc, f"{name}: {msg}")
    return rc


def size(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


class SlotMap(ctypes.Structure):
    """``lsa_slot_map`` (include/lsa_rocm.h): a paged cache's slot table."""

    _fields_ = [("table", _p), ("rows", _p), ("stride", _i64), ("width", _i32), ("n_rows", _i32)]


def slot_map(table: torch.Tensor | None, rows: torch.Tensor | None):
    """``const lsa_slot_map*`` for a call (None: no paging): table [n_rows, width] int32 with
    contiguous rows, rows [R] int32. The caller keeps both tensors alive for the call."""
    if table is None:
        return None
    return ctypes.pointer(SlotMap(table.data_ptr(), rows.data_ptr(), table.stride(0), table.shape[1],
                                  table.shape[0]))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def device_index(device: torch.device | int | str | None) -> int:
    """The ordinal of a CUDA device (``cuda`` alone is the current device)."""
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    device = torch.device(device)
    return torch.cuda.current_device() if device.index is None else device.index


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return LSA_F32
    if dtype == torch.bfloat16:
        return LSA_BF16
    if dtype == torch.float16:
        return LSA_F16
    raise ValueError(f"unsupported dtype {dtype} (fp32, bf16, fp16)")


class Workspace:
    """Scratch per (device, stream, purpose), grown on demand; kernels fully write the
    part they read, so it needs no initialisation. Calls sharing it are stream-ordered.
    A buffer that is outgrown is retired, never freed: a HIP graph captured earlier may
    still replay against it."""

    _buffers: dict[tuple, torch.Tensor] = {}
    _retired: list[torch.Tensor] = []

    @classmethod
    def get(cls, device: torch.device, purpose: str, nbytes: int) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        key = (device_index(device), stream(device), purpose)
        buf = cls._buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                cls._retired.append(buf)
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            cls._buffers[key] = buf
        return buf


class Counters:
    """Split-arrival counters per (device, stream): int32 that every kernel finds zero at
    launch and leaves zero, so the buffer is zero-filled only when it is (re)allocated.
    Outgrown buffers are retired, never freed (a captured graph may hold them)."""

    _buffers: dict[tuple, torch.Tensor] = {}
    _retired: list[torch.Tensor] = []

    @classmethod
    def get(cls, device: torch.device, n: int) -> torch.Tensor:
        key = (device_index(device), stream(device))
        buf = cls._buffers.get(key)
        if buf is None or buf.numel() < n:
            if buf is not None:
                cls._retired.append(buf)
            buf = torch.zeros(max(n, 4096), dtype=torch.int32, device=device)
            cls._buffers[key] = buf
        return buf

    @classmethod
    def reset(cls, device: torch.device) -> None:
        """Zeroes every counter buffer of the device (after a decode gave up waiting)."""
        index = device_index(device)
        for (dev, _), buf in cls._buffers.items():
            if dev == index:
                buf.zero_()


class StatusWord:
    """One int32 per (device, purpose) in pinned host memory that a kernel sets with a
    system-scope store - the fused decode when a reader gives up waiting ("decode"), the
    bucket-table build when a table cannot reach its segment count ("build") - and the host
    reads without a device sync."""

    _words: dict[tuple[int, str], torch.Tensor] = {}

    @classmethod
    def get(cls, device: torch.device, purpose: str = "decode") -> torch.Tensor:
        key = (device_index(device), purpose)
        word = cls._words.get(key)
        if word is None:
            word = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            cls._words[key] = word
        return word
