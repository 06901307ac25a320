"""ctypes binding of libgdn2_hip.so (declared in include/gdn2.h).

Loading never falls back to anything: if the shared library is missing or does
not export a symbol, ``lib()`` raises ``GDN2LibraryError``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

# torch first: its bundled HIP runtime carries the soname libamdhip64.so.7, so
# the library below binds to that same runtime instead of loading a second one.
import torch  # noqa: F401

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("GDN2_LIB", _HERE / "libgdn2_hip.so"))

GDN2_F32 = 0
GDN2_BF16 = 1
GDN2_BF16_F32 = 2   # bfloat16 inputs and gradients, float32 arithmetic and residuals
FWD_SAVE_A = 1
FWD_RAW_INPUTS = 2
FWD_PARTIAL_CHUNK = 4
# gdn2_bwd_stage_workspace_bytes: which backward stage
STAGE_DHU = 1
STAGE_DAV = 2
STAGE_WY = 3
STAGE_INTRA = 4


def FWD_SEGMENTS(n: int) -> int:
    """gdn2_fwd flag forcing n segments of the state scan (include/gdn2.h)."""
    return (int(n) & 0xFF) << 8

OK = 0
ERR_HEAD_DIM = -1
ERR_SEQ_LEN = -2
ERR_CHUNK = -3
ERR_DTYPE = -4
ERR_NULL = -5
ERR_ALIGN = -6
ERR_WORKSPACE = -7
ERR_SHAPE = -8
ERR_LAUNCH = -9
ERR_FLAGS = -10
ERR_SCRATCH = -11
NOALLOC_SCRATCH_BYTES = 128 << 20

_c_int, _c_float, _c_size, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); exactly the entry points of include/gdn2.h
SIGNATURES = {
    "gdn2_version": (ctypes.c_char_p, []),
    "gdn2_strerror": (ctypes.c_char_p, [_c_int]),
    "gdn2_validate": (_c_int, [_c_int] * 7),
    "gdn2_fwd_workspace_bytes": (_c_size, [_c_int] * 6),
    "gdn2_fwd_workspace_bytes_ex": (_c_size, [_c_int] * 7),
    "gdn2_bwd_workspace_bytes": (_c_size, [_c_int] * 6),
    "gdn2_fwd": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 7
                 + [_c_float, _vp, _vp, _vp, _c_size, _c_int]),
    "gdn2_fwd_debug": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 7
                       + [_c_float, _vp, _vp, _vp, _c_size, _vp]),
    "gdn2_set_launch_events": (_c_int, [_vp, _c_int]),
    "gdn2_set_clip": (_c_int, [_c_float]),
    "gdn2_bwd": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 7
                 + [_c_float, _vp, _vp] + [_vp] * 7 + [_vp, _c_size, _vp, _c_size]),
    "gdn2_decode": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 6 + [_c_float, _vp, _vp, _vp]),
    "gdn2_fwd_noalloc": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 7
                         + [_c_float, _vp, _vp, _c_int]),
    "gdn2_fwd_varlen_workspace_bytes": (_c_size, [_c_int] * 5),
    "gdn2_fwd_varlen": (_c_int, [_vp, _c_int, _vp, _vp] + [_c_int] * 7 + [_vp] * 7
                        + [_c_float, _vp, _vp, _vp, _c_size, _c_int]),
    "gdn2_bwd_varlen_workspace_bytes": (_c_size, [_c_int] * 5),
    "gdn2_bwd_varlen": (_c_int, [_vp, _c_int, _vp] + [_c_int] * 6 + [_vp] * 7
                        + [_c_float, _vp, _vp] + [_vp] * 7 + [_vp, _c_size, _vp, _c_size]),
    "gdn2_chunk_scores": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 4 + [_c_float, _vp, _vp]),
    "gdn2_wy_solve": (_c_int, [_vp, ctypes.c_longlong, _c_int, _vp, _vp]),
    "gdn2_recompute_wy": (_c_int, [_vp] + [_c_int] * 7 + [_vp] * 7 + [_vp] * 5),
    "gdn2_chunk_combine_workspace_bytes": (_c_size, [_c_int] * 5),
    "gdn2_chunk_combine": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 7
                           + [_c_float, _vp, _vp, _vp, _vp, _vp, _c_size]),
    "gdn2_bwd_stage_workspace_bytes": (_c_size, [_c_int] * 6),
    "gdn2_bwd_dhu": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 6
                     + [_c_float, _vp, _vp, _vp, _vp, _vp, _c_size]),
    "gdn2_bwd_dav": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 6 + [_c_size]),
    "gdn2_bwd_wy_dqkg": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 12 + [_c_float]
                         + [_vp] * 8 + [_c_size]),
    "gdn2_bwd_intra": (_c_int, [_vp] + [_c_int] * 5 + [_vp] * 6 + [_c_float]
                       + [_vp] * 5 + [_c_size]),
    "gdn2_bwd_reverse_cumsum": (_c_int, [_vp, ctypes.c_longlong, _c_int, _c_int, _vp, _vp]),
}


class GDN2LibraryError(RuntimeError):
    """libgdn2_hip.so could not be loaded (build it with __graft_entry__.build())."""


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise GDN2LibraryError(
                f"{LIB_PATH} not found: build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (gfx950 HIP library; there is no CPU fallback)")
        try:
            L = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise GDN2LibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(L, name)
            except AttributeError as e:
                raise GDN2LibraryError(f"{LIB_PATH} does not export {name}") from e
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def strerror(code: int) -> str:
    return lib().gdn2_strerror(code).decode()
