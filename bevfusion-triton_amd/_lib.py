"""ctypes binding of ``libbevpool_amd.so`` (the C ABI declared in
``include/bevpool.h``).

The library is built in-tree by ``csrc/Makefile`` next to this file.  There is
no fallback: when the library is missing or fails to load, every entry point
raises :class:`LibraryNotBuilt`.

torch is imported before the library is loaded so that the HIP runtime the
library links against (``libamdhip64.so.7``) resolves to the instance torch
already loaded; device pointers and streams are then shared with torch.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first; see module docstring)

LIB_PATH = Path(__file__).resolve().parent / 'libbevpool_amd.so'
ABI_VERSION = 4

F32, F16, BF16 = 0, 1, 2
META_N_KEPT, META_N_INTERVALS, META_N_BAD, META_FIRST_BAD = 0, 1, 2, 3
META_LEN = 8
REPORT_LEN = META_LEN + 1  # the counters, then a done flag

DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


class LibraryNotBuilt(RuntimeError):
    """libbevpool_amd.so is missing or unloadable (run ``__graft_entry__.build()``)."""


class BevPoolError(RuntimeError):
    """A C ABI call returned a non-zero status."""


_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f3 = ctypes.c_float * 3
_i3 = ctypes.c_int32 * 3

_SIGNATURES = {
    'bevpool_abi_version': ([], ctypes.c_int),
    'bevpool_last_error': ([], ctypes.c_char_p),
    'bevpool_index_workspace_bytes': ([_i64, _i64], _sz),
    'bevpool_quantize_geom': (
        [_vp, _i64, _i64, _i64, _i32, _f3, _f3, _i3, _vp, _vp, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_quantize_cameras': (
        [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f3, _f3, _i3,
         _vp, _vp, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_coord_ranks': (
        [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_sort': ([_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
    'bevpool_intervals': ([_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
    'bevpool_meta_report': ([_vp, _vp, _vp], ctypes.c_int),
    'bevpool_forward_scratch_bytes': ([_i64, _i32], _sz),
    'bevpool_forward': (
        [_vp, _i32, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64, _i64,
         _vp, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_backward_scratch_bytes': ([_i64, _i32, _i32], _sz),
    'bevpool_backward': (
        [_vp, _i32, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i64, _vp, _i64,
         _i32, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_op_index_bytes': ([_i64, _i64], _sz),
    'bevpool_op_scratch_bytes': ([_i64, _i64, _i32], _sz),
    'bevpool_op_workspace_bytes': ([_i64, _i64, _i32], _sz),
    'bevpool_op_forward': (
        [_vp, _i32, _i64, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _sz,
         _vp, _sz, _vp, _vp],
        ctypes.c_int,
    ),
    'bevpool_op_forward_noalloc': (
        [_vp, _i32, _i64, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp],
        ctypes.c_int,
    ),
    'bevpool_op_backward': (
        [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp,
         _sz, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_legacy_forward': (
        [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
        ctypes.c_int,
    ),
    'bevpool_legacy_backward': (
        [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
        ctypes.c_int,
    ),
    'bevpool_runs_workspace_bytes': ([_i64], _sz),
    'bevpool_runs': ([_vp, _i32, _i64, _vp, _vp, _vp, _vp, _sz, _vp], ctypes.c_int),
    'bevpool_context_rows': ([_vp, _i64, _i64, _i32, _i32, _i64, _vp, _vp], ctypes.c_int),
    'bevpool_planar_rows': ([_vp, _i64, _i64, _i32, _i32, _i64, _vp, _vp], ctypes.c_int),
    'bevpool_backward_planar': (
        [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i64, _i64, _vp, _i64,
         _i64, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_forward_depth': (
        [_vp, _vp, _i32, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64,
         _i64, _vp, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_backward_depth': (
        [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _i32,
         _i64, _vp, _vp, _i64, _i64, _vp, _sz, _vp],
        ctypes.c_int,
    ),
    'bevpool_timing_enable': ([ctypes.c_int], ctypes.c_int),
    'bevpool_timing_reset': ([], ctypes.c_int),
    'bevpool_timing_read': (
        [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
         ctypes.POINTER(ctypes.c_int64), ctypes.c_int],
        ctypes.c_int,
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None


def library():
    """The loaded ctypes library (loaded once)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryNotBuilt(
            f'{LIB_PATH} is missing: build it with `python -c "import __graft_entry__ as g; '
            f'g.build()"` (or `make -C bevfusion-triton_amd/csrc`)'
        )
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the runtime image
        raise LibraryNotBuilt(f'cannot load {LIB_PATH}: {exc}') from exc
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    version = lib.bevpool_abi_version()
    if version != ABI_VERSION:
        raise LibraryNotBuilt(f'{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}')
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = library().bevpool_last_error().decode(errors='replace')
        raise BevPoolError(f'{what} failed (status {status}): {msg}')


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def timing_enable(on: bool) -> None:
    check(library().bevpool_timing_enable(1 if on else 0), 'bevpool_timing_enable')


def timing_reset() -> None:
    check(library().bevpool_timing_reset(), 'bevpool_timing_reset')


def timing_read(max_entries: int = 64) -> dict:
    """{kernel name: (total ms, launches)} since the last reset (synchronises)."""
    stride = 64
    names = ctypes.create_string_buffer(stride * max_entries)
    ms = (ctypes.c_double * max_entries)()
    launches = (ctypes.c_int64 * max_entries)()
    n = library().bevpool_timing_read(names, stride, ms, launches, max_entries)
    if n < 0:
        check(n, 'bevpool_timing_read')
    out = {}
    for i in range(n):
        raw = names.raw[i * stride:(i + 1) * stride]
        out[raw.split(b'\0', 1)[0].decode()] = (ms[i], int(launches[i]))
    return out
