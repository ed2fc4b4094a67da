"""ctypes binding of the HIP C-ABI library (``include/mogt_scan.h``).

This is the only place Python touches the native library.  Loading fails
loudly: there is no CPU or PyTorch fallback behind any public operator.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

from . import _build

MOGT_F32 = 0
MOGT_BF16 = 1
MOGT_F64 = 2
MOGT_F16 = 3
MOGT_CONN_EXP = 0
MOGT_CONN_CAYLEY = 1
ABI_VERSION = 11

_c_void_p = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes); must match include/mogt_scan.h
SIGNATURES: dict[str, tuple] = {
    "mogt_last_error": (ctypes.c_char_p, []),
    "mogt_abi_version": (_c_int, []),
    "mogt_build_manifest": (ctypes.c_char_p, []),
    "mogt_workspace_faults": (_c_int, [_c_void_p, _c_size, ctypes.POINTER(ctypes.c_uint32), _c_void_p]),
    "mogt_diag_scan_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int]),
    "mogt_diag_scan_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
         _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_diag_scan_rev_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p]),
    "mogt_diag_scan_workspace_bytes_cfg": (
        _c_size, [_c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int]),
    "mogt_diag_scan_fwd_cfg": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_diag_scan_tiles": (_c_int, [_c_int, ctypes.POINTER(_c_int), _c_int]),
    "mogt_diag_scan_fwd_noalloc": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_void_p],
    ),
    "mogt_coupled_rank_scan_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "mogt_coupled_rank_scan_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int,
         _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_coupled_rank_scan_stats_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_int,
         _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_coupled_rank_scan_proj_fwd": (
        _c_int,
        [_c_void_p, _c_i64, _c_i64, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_float, _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_coupled_rank_scan_proj_grad": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_float, _c_int, _c_void_p],
    ),
    "mogt_coupled_rank_scan_fwd_cfg": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_coupled_rank_scan_rev_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_void_p, _c_size,
         _c_void_p],
    ),
    "mogt_coupled_rank_scan_rev_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "mogt_coupled_rank_scan_rev_fwd_cfg": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_void_p, _c_size, _c_void_p]),
    "mogt_coupled_rank_scan_grad": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64,
                 _c_i64, _c_float, _c_int, _c_void_p]),
    "mogt_affine_scan_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "mogt_affine_scan_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
         _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_affine_scan_vk_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
         _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_affine_scan_rev_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p]),
    "mogt_affine_scan_grad_u": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p]),
    "mogt_affine_scan_generic_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "mogt_affine_scan_generic_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int,
         _c_int, _c_void_p, _c_size, _c_void_p]),
    "mogt_affine_local_scan_generic": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
         _c_int, _c_void_p]),
    "mogt_fused_scan_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "mogt_fused_scan_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "mogt_affine_local_scan": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_int, _c_void_p],
    ),
    "mogt_rmsnorm_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_float, _c_int, _c_int, _c_void_p]),
    "mogt_add_rmsnorm_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_float,
         _c_int, _c_int, _c_void_p]),
    "mogt_silu_mul_fwd": (_c_int, [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_int, _c_void_p]),
    "mogt_swiglu_gate_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
                 _c_void_p]),
    "mogt_swiglu_gate_fwd_cfg": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
                 _c_int, _c_void_p]),
    "mogt_swiglu_check_schedule": (_c_int, [_c_i64, _c_i64, _c_int]),
    "mogt_linear_wgrad": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
                 _c_void_p, _c_size, _c_void_p]),
    "mogt_linear_wgrad_splits": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "mogt_linear_wgrad_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "mogt_add_rmsnorm_rowscale_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_float, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_i64,
         _c_i64, _c_float, _c_int, _c_int, _c_void_p]),
    "mogt_rmsnorm_bwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_float,
                 _c_int, _c_int, _c_int, _c_void_p, _c_float, _c_int, _c_void_p]),
    "mogt_silu_mul_bwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_int, _c_void_p]),
    "mogt_embedding_bwd": (
        _c_int, [_c_void_p, _c_i64, _c_void_p, _c_i64, _c_i64, _c_int, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64,
                 _c_void_p, _c_void_p, _c_void_p]),
    "mogt_connection_map_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_float, _c_float, _c_int, _c_int, _c_void_p]),
    "mogt_lm_ce_fwd": (
        _c_int, [_c_void_p, _c_i64, _c_int, _c_void_p, _c_i64, _c_i64, _c_i64, _c_void_p, _c_void_p,
                 _c_void_p]),
    "mogt_lm_ce_bwd": (
        _c_int, [_c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_void_p,
                 _c_void_p, _c_i64, _c_int, _c_void_p]),
    "mogt_rank1_coupled_scan_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "mogt_rank1_coupled_scan_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_int, _c_int, _c_void_p, _c_size, _c_void_p]),
    "mogt_rank1_coupled_scan_fwd_cfg": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_int, _c_int, _c_void_p, _c_size, _c_int, _c_void_p]),
    "mogt_rank1_check_ranges": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MogtError(RuntimeError):
    """A native entry point returned an error code."""


def library_path() -> Path:
    override = os.environ.get("MOGT_HIP_LIB")
    return Path(override) if override else _build.lib_path()


def load() -> ctypes.CDLL:
    """Load (once) and type the native library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"MOGT HIP library not built: {path} is missing. "
                "Run `python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)."
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.mogt_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"MOGT HIP library ABI {ver} != expected {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mogt_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise MogtError(f"{what} failed ({rc}): {msg}")


def build_manifest() -> dict[str, str]:
    """``name -> hash`` of the sources and flags the loaded library was built from."""
    return _build.parse_manifest(load().mogt_build_manifest().decode())


def build_id() -> str:
    """One short id for the loaded library's build (hash of its manifest)."""
    return _build.build_id(build_manifest())


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def diag_tiles(family: int) -> list[tuple[int, int, int, int]]:
    """Compiled diag-scan tiles (vec, lanes, steps, waves) of a family:
    0 fp32 input, 1 bf16 input, 2 coupled scan."""
    lib = load()
    n = lib.mogt_diag_scan_tiles(family, None, 0)
    buf = (_c_int * (4 * n))()
    lib.mogt_diag_scan_tiles(family, buf, n)
    return [tuple(buf[4 * i:4 * i + 4]) for i in range(n)]
