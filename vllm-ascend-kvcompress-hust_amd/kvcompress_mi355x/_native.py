"""ctypes binding of the C ABI in include/kvcompress_mi355x.h.

The shared library is built in-tree (``csrc/build.py``) next to this file.  A
missing library is an error: the compression path has no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIBRARY_NAME = "libkvcompress_mi355x.so"
LIBRARY_PATH = Path(__file__).resolve().parent / LIBRARY_NAME

ABI_VERSION = 2
EINVAL = -22
DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2
ROPE_HALF = 0
ROPE_INTERLEAVED = 1
POLICY_GLOBAL = 0
POLICY_V3 = 1
LAYER_MEAN = 0
LAYER_MAX = 1
AGG_ACCUMULATE = 1
AGG_FINALIZE = 2
AGG_RSQRT = 4
RAW_TOKEN_MAJOR = 0
RAW_HEAD_MAJOR = 1
COMPACT_LAYER_MAJOR = 0
COMPACT_LAYERS_INTERLEAVED = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the order of declaration follows the header.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "kvc_abi_version": (_i32, []),
    "kvc_last_error": (ctypes.c_char_p, []),
    "kvc_mean_phases": (_i32, [_p, _i32, _i32, _i32, _p, _p, _i32, _p, _p, _p]),
    "kvc_shift_mean_phases": (_i32, [_p, _i32, _i64, _p, _p, _p, _p, _p]),
    "kvc_score_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "kvc_score_raw_layout": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "kvc_score_paged": (
        _i32,
        [
            _p, _i32, _i32, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
            _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _p, _sz,
        ],
    ),
    "kvc_offset_phases": (_i32, [_p, _i32, _i32, _i32, _p, _p, _i32, _p, _p, _p]),
    "kvc_score_max_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "kvc_score_paged_max": (
        _i32,
        [
            _p, _i32, _i32, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
            _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i64, _p, _i64, _i64, _i64, _p, _sz,
        ],
    ),
    "kvc_head_stats": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _sz, _p, _p]),
    "kvc_score_paged_noalloc": (
        _i32,
        [
            _p, _i32, _i32, _p, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
            _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _p, _p,
        ],
    ),
    "kvc_aggregate": (
        _i32,
        [_p, _i32, _i32, _i32, _i32, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i32, _u32, _p],
    ),
    "kvc_layer_head_max": (
        _i32,
        [_p, _i32, _i32, _i32, _i32, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _u32, _p, _i64],
    ),
    "kvc_combine_layer_scores": (_i32, [_p, _i32, _i64, _p, _i64, _i32, _u32, _p]),
    "kvc_select_keep": (_i32, [_p, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _i64]),
    "kvc_select_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "kvc_select_keep_split": (_i32, [_p, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _sz]),
    "kvc_compact_workspace_bytes": (_sz, [_i32, _i32]),
    "kvc_compact": (
        _i32,
        [_p, _i32, _p, _p, _i64, _i64, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _sz, _i32],
    ),
    "kvc_rewrite_block_tables": (_i32, [_p, _i32, _i32, _p, _p, _p, _p, _p, _p, _p]),
    "kvc_token_slots": (_i32, [_p, _p, _i64, _p, _i64, _i32, _p]),
    "kvc_expand_block_ids": (_i32, [_p, _p, _i64, _i32, _p]),
    "kvc_materialize_slots": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i32, _p, _p, _i64, _p, _p]),
    "kvc_shift_positions": (_i32, [_p, _p, _p, _i32, _p, _i64, _p]),
    "kvc_physical_slot_mapping": (_i32, [_p, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i64, _p, _p]),
    "kvc_shift_lengths": (_i32, [_p, _p, _i32, _p, _i32]),
    "kvc_qstats_state_bytes": (_sz, [_i32, _i32, _i32]),
    "kvc_qstats_accumulate": (_i32, [_p, _i32, _p, _i64, _i64, _i32, _i32, _i32, _p, _sz]),
    "kvc_qstats_finish": (_i32, [_p, _i32, _i32, _i32, _p, _p, _p, _p, _p]),
}

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


class NativeLibraryError(RuntimeError):
    """The HIP extension is missing or does not match this binding."""


def library_path() -> Path:
    override = os.environ.get("KVCOMPRESS_MI355X_LIBRARY")
    return Path(override) if override else LIBRARY_PATH


def load() -> ctypes.CDLL:
    """Load the shared library once and bind every exported symbol."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.is_file():
            raise NativeLibraryError(
                f"HIP extension {path} is not built; run __graft_entry__.build() "
                "or vllm-ascend-kvcompress-hust_amd/csrc/build.py"
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as error:
                raise NativeLibraryError(f"{path} does not export {name}") from error
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.kvc_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"{path} has ABI {version}, binding expects {ABI_VERSION}")
        _LIB = lib
        return lib


def check(code: int, what: str) -> None:
    """Raise the reference's fail-closed error types for a nonzero return."""
    if code == 0:
        return
    message = (load().kvc_last_error() or b"").decode(errors="replace")
    if code == EINVAL:
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what} failed with HIP error {code}: {message}")


def call(name: str, *args: object) -> None:
    check(getattr(load(), name)(*args), name)
