"""The C-ABI library loads without a GPU, exports every function declared in
include/*.h, and rejects bad arguments before touching the device."""
import re
from pathlib import Path

import pytest

from mogt_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(mogt_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert names, "no declarations found in include/*.h"
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_covers_header(lib):
    assert declared_functions() == set(_lib.SIGNATURES)


def test_abi_version(lib):
    assert lib.mogt_abi_version() == _lib.ABI_VERSION


def test_library_built_from_these_sources(lib):
    # the manifest compiled into the library names every source and its hash;
    # a library older than any source (or built with other flags) fails here
    from mogt_amd import _build

    built = _lib.build_manifest()
    tree = _build.source_manifest()
    assert set(built) == set(tree)
    stale = sorted(k for k in tree if built[k] != tree[k])
    assert not stale, f"library built from other sources: {stale} (rebuild)"
    assert _lib.build_id() == _build.build_id(tree)


def test_workspace_queries_are_host_only(lib):
    n = lib.mogt_diag_scan_workspace_bytes(1, 32768, 768, _lib.MOGT_F32)
    assert 256 < n < 64 << 20
    assert lib.mogt_diag_scan_workspace_bytes_cfg(1, 32768, 768, 2, 32, 16, 16) == n
    assert lib.mogt_diag_scan_workspace_bytes_cfg(1, 32768, 768, 2, 24, 16, 16) == 256
    assert lib.mogt_coupled_rank_scan_workspace_bytes(1, 1024, 16, 48, _lib.MOGT_BF16) > 256
    # the coupled reverse scan's query covers its 4-channel default tile
    rev = lib.mogt_coupled_rank_scan_rev_workspace_bytes(1, 32768, 16, 48)
    assert rev >= lib.mogt_diag_scan_workspace_bytes_cfg(1, 32768, 768, 4, 16, 8, 8) > 256
    assert lib.mogt_coupled_rank_scan_rev_workspace_bytes(0, 32768, 16, 48) == 256


def test_argument_errors_without_device(lib):
    # Validation happens on the host before any HIP call.
    rc = lib.mogt_diag_scan_fwd(None, None, None, None, 1, 8, 8, 7, 0, None, 0, None)
    assert rc == -1 and b"dtype" in lib.mogt_last_error()
    rc = lib.mogt_diag_scan_fwd_cfg(1, 1, 1, None, 1, 8, 8, 0, 0, 3, 64, 8, 4, None, 0, None)
    assert rc == -1 and b"not compiled" in lib.mogt_last_error()
    rc = lib.mogt_diag_scan_fwd_cfg(1, 1, 1, None, 1, 8, 8, 0, 0, 1, 64, 8, 16, None, 0, None)
    assert rc == -2 and b"workspace" in lib.mogt_last_error()
    rc = lib.mogt_coupled_rank_scan_fwd(1, 1, 1, 1, 8, 0, 48, 1.0, 0, 0, 0, None, 0, None)
    assert rc == -1
    # zero-size problems are a no-op success
    assert lib.mogt_diag_scan_fwd(None, None, None, None, 0, 8, 8, 0, 0, None, 0, None) == 0
    # cross-entropy rows: stride shorter than the vocabulary, bad dtype, in place
    # with a different stride; zero rows are a no-op
    rc = lib.mogt_lm_ce_fwd(1, 10, 0, 1, 4, 32, -100, 1, 1, None)
    assert rc == -1 and b"stride" in lib.mogt_last_error()
    assert lib.mogt_lm_ce_fwd(1, 32, 5, 1, 4, 32, -100, 1, 1, None) == -1
    rc = lib.mogt_lm_ce_bwd(8, 32, 0, 1, 1, 4, 32, -100, 1, 8, 40, 0, None)
    assert rc == -1 and b"in place" in lib.mogt_last_error()
    assert lib.mogt_lm_ce_fwd(None, 32, 0, None, 0, 32, -100, None, None, None) == 0
    # fused SwiGLU gate: bf16 only, d_in % 32, hidden % 128, strides covering
    # the rows
    assert lib.mogt_swiglu_gate_fwd(16, 16, 16, 16, 8, 64, 128, 64, 128, 0, None) == -1
    rc = lib.mogt_swiglu_gate_fwd(16, 16, 16, 16, 8, 48, 128, 48, 128, 1, None)
    assert rc == -1 and b"multiple" in lib.mogt_last_error()
    assert lib.mogt_swiglu_gate_fwd(16, 16, 16, 16, 8, 64, 96, 64, 96, 1, None) == -1
    rc = lib.mogt_swiglu_gate_fwd(16, 16, 16, 16, 8, 64, 128, 32, 128, 1, None)
    assert rc == -1 and b"stride" in lib.mogt_last_error()
    rc = lib.mogt_swiglu_gate_fwd(8, 16, 16, 16, 8, 64, 128, 64, 128, 1, None)
    assert rc == -1 and b"align" in lib.mogt_last_error()
    assert lib.mogt_swiglu_gate_fwd(None, None, None, None, 0, 64, 128, 64, 128, 1, None) == 0
    # embedding backward: row length, stride and dtype checks before any launch
    assert lib.mogt_embedding_bwd(16, 64, None, 0, 4, 0, 16, 16, 4, 6, 10, 16, 16, None) == -1
    assert lib.mogt_embedding_bwd(16, 32, None, 0, 4, 0, 16, 16, 4, 64, 10, 16, 16, None) == -1
    assert lib.mogt_embedding_bwd(16, 64, None, 0, 4, 5, 16, 16, 4, 64, 10, 16, 16, None) == -1
    # a second gradient source: n_first within [0, n] (n without one), its stride
    rc = lib.mogt_embedding_bwd(16, 64, None, 0, 3, 0, 16, 16, 4, 64, 10, 16, 16, None)
    assert rc == -1 and b"n_first" in lib.mogt_last_error()
    assert lib.mogt_embedding_bwd(16, 64, 16, 32, 2, 0, 16, 16, 4, 64, 10, 16, 16, None) == -1
    rc = lib.mogt_embedding_bwd(8, 64, None, 0, 4, 0, 16, 16, 4, 64, 10, 16, 16, None)
    assert rc == -1 and b"align" in lib.mogt_last_error()


def test_linear_wgrad_plan_and_checks_without_device(lib):
    """The split-K weight-gradient GEMM's slice plan and argument checks are
    host-only.  Plan: enough slices to give each CU one 256 x 256 work-group
    tile (256 CUs), whole 32-token stages per slice, no empty slice."""
    plan = lib.mogt_linear_wgrad_splits
    assert plan(32768, 768, 768, 0, 256) == 28        # 9 tiles
    assert plan(32768, 800, 768, 0, 256) == 21        # 12 tiles (a partial row of tiles)
    assert plan(32768, 768, 3072, 0, 256) == 7        # 36 tiles
    assert plan(32768, 6144, 768, 0, 256) == 3        # 72 tiles
    assert plan(32768, 8192, 8192, 0, 256) == 1       # more tiles than CUs
    assert plan(200, 768, 768, 0, 256) == 1           # under two minimum slices of 128 tokens
    assert plan(0, 768, 768, 0, 256) == 0
    assert plan(4096, 16, 16, 4096, 256) == 128       # explicit: capped at one stage per slice
    assert plan(4097, 16, 16, 3, 256) == 3            # slices of 1376 tokens, the last one 1345
    assert plan(10, 8, 8, 0, 256) == 1
    assert plan(-1, 8, 8, 0, 256) == -1 and plan(8, 0, 8, 0, 256) == -1
    assert lib.mogt_linear_wgrad_workspace_bytes(32768, 768, 768, 0, 256) == 28 * 768 * 768 * 4
    assert lib.mogt_linear_wgrad_workspace_bytes(0, 768, 768, 0, 256) == 0
    N = None
    # dW dtype, feature multiples of 8, strides, alignment, workspace size:
    # all rejected before any HIP call (explicit splits: no device query)
    call = lib.mogt_linear_wgrad
    assert call(16, 16, 16, 64, 16, 16, 16, 16, 16, 1, 2, 16, 1 << 20, N) == -1
    rc = call(16, 16, 16, 64, 12, 16, 16, 16, 16, 1, 1, 16, 1 << 20, N)
    assert rc == -1 and b"multiples of 8" in lib.mogt_last_error()
    rc = call(16, 16, 16, 64, 16, 16, 8, 16, 16, 1, 1, 16, 1 << 20, N)
    assert rc == -1 and b"stride" in lib.mogt_last_error()
    rc = call(8, 16, 16, 64, 16, 16, 16, 16, 16, 1, 1, 16, 1 << 20, N)
    assert rc == -1 and b"align" in lib.mogt_last_error()
    rc = call(16, 16, 16, 64, 16, 16, 16, 16, 16, 2, 1, 16, 16 * 16 * 4, N)
    assert rc == -2 and b"workspace" in lib.mogt_last_error()
    rc = call(16, N, 16, 64, 16, 16, 16, 16, 16, 1, 1, 16, 1 << 20, N)
    assert rc == -1 and b"null" in lib.mogt_last_error()
    # a slice whose rows span 2 GiB asks for more splits
    rc = call(16, 16, 16, 1 << 20, 1024, 1024, 1024, 1024, 1024, 1, 1, 16, 1 << 62, N)
    assert rc == -1 and b"splits" in lib.mogt_last_error()


def test_empty_problems_are_noops_without_device(lib):
    """Zero batch, length or rows: every compute entry point returns success
    before it needs a pointer or the device."""
    N = None
    calls = {
        "diag": lambda B, L: lib.mogt_diag_scan_fwd(N, N, N, N, B, L, 8, 0, 0, N, 0, N),
        "diag_rev": lambda B, L: lib.mogt_diag_scan_rev_fwd(N, N, N, B, L, 8, N, 0, N),
        "coupled": lambda B, L: lib.mogt_coupled_rank_scan_fwd(N, N, N, B, L, 4, 6, 1.0, 0, 0, 0, N, 0, N),
        "coupled_rev": lambda B, L: lib.mogt_coupled_rank_scan_rev_fwd(N, N, N, B, L, 4, 6, 1.0, 0, N, 0, N),
        "coupled_rev_cfg": lambda B, L: lib.mogt_coupled_rank_scan_rev_fwd_cfg(N, N, N, B, L, 4, 8, 1.0, 0, 4, 16,
                                                                                8, 8, N, 0, N),
        "coupled_grad": lambda B, L: lib.mogt_coupled_rank_scan_grad(N, N, N, N, N, N, B, L, 4, 8, 1.0, 0, N),
        "dense": lambda B, L: lib.mogt_affine_scan_fwd(N, N, N, N, B, L, 16, 8, 0, 0, N, 0, N),
        "dense_vk": lambda B, L: lib.mogt_affine_scan_vk_fwd(N, N, N, N, N, B, L, 16, 16, 0, 0, N, 0, N),
        "fused": lambda B, L: lib.mogt_fused_scan_fwd(N, N, B, L, 16, 0, N, 0, N),
        "local": lambda B, L: lib.mogt_affine_local_scan(N, N, N, N, N, N, B, L, 16, 8, 32, 0, N),
        "rank1": lambda B, L: lib.mogt_rank1_coupled_scan_fwd(N, N, N, N, N, B, L, 3, 64, 0, 0, 0, N, 0, N),
    }
    for name, call in calls.items():
        for B, L in ((0, 5), (2, 0)):
            assert call(B, L) == 0, (name, B, L, lib.mogt_last_error())
    rows = {
        "rmsnorm": lambda: lib.mogt_rmsnorm_fwd(N, N, N, 0, 64, 1e-6, 0, 0, N),
        "add_rmsnorm": lambda: lib.mogt_add_rmsnorm_fwd(N, N, 0.5, N, N, N, 0, 64, 1e-6, 0, 0, N),
        "silu_mul": lambda: lib.mogt_silu_mul_fwd(N, N, 0, 64, 0, N),
        "rmsnorm_bwd": lambda: lib.mogt_rmsnorm_bwd(N, N, N, N, N, N, 0, 64, 1e-6, 4, 0, 0, N, 1.0, 0, N),
        "silu_mul_bwd": lambda: lib.mogt_silu_mul_bwd(N, N, N, 0, 64, 0, N),
        "connection_map": lambda: lib.mogt_connection_map_fwd(N, N, 0, 16, 1.0, 1.0, 0, 0, N),
        "lm_ce_bwd": lambda: lib.mogt_lm_ce_bwd(N, 32, 0, N, N, 0, 32, -100, N, N, 32, 0, N),
        "embedding_bwd": lambda: lib.mogt_embedding_bwd(N, 64, N, 0, 0, 0, N, N, 0, 64, 10, N, N, N),
    }
    for name, call in rows.items():
        assert call() == 0, (name, lib.mogt_last_error())


def test_tile_lists(lib):
    for fam in (0, 1, 2, 3):
        tiles = _lib.diag_tiles(fam)
        assert tiles, fam
        for vec, lanes, steps, waves in tiles:
            # rows of >= 256 contiguous bytes at fp32 / bf16 input
            assert lanes in (16, 32, 64) and lanes * vec >= 64
            assert steps * waves * (64 // lanes) >= 128


def test_gpu_tile_lists_match_library(lib):
    from test_gpu_backward import TILES_COUPLED_REV
    from test_gpu_diag_scan import TILES_BF16, TILES_COUPLED, TILES_F32

    assert _lib.diag_tiles(0) == TILES_F32
    assert _lib.diag_tiles(1) == TILES_BF16
    assert _lib.diag_tiles(2) == TILES_COUPLED
    assert _lib.diag_tiles(3) == TILES_COUPLED_REV


def test_check_maps_codes_to_python_errors(lib):
    lib.mogt_diag_scan_fwd(None, None, None, None, 1, 8, 8, 7, 0, None, 0, None)
    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    with pytest.raises(_lib.MogtError):
        _lib.check(-3, "x")


def test_ops_reject_cpu_tensors():
    import torch

    import mogt_amd

    a = torch.rand(1, 4, 8)
    with pytest.raises(ValueError, match="CUDA"):
        mogt_amd.diag_scan(a, a)
    with pytest.raises(ValueError, match="CUDA"):
        mogt_amd.coupled_rank_scan(torch.zeros(1, 4, 2), torch.zeros(1, 4, 8))


def test_library_is_plain_c_abi():
    """No torch symbols leak into the shared object's dynamic imports."""
    import subprocess

    out = subprocess.run(["nm", "-D", "--undefined-only", str(_lib.library_path())],
                         capture_output=True, text=True).stdout
    assert "torch" not in out and "c10" not in out


def test_workspace_fault_query_validates_arguments(lib):
    import ctypes

    count = ctypes.c_uint32(7)
    assert lib.mogt_workspace_faults(None, 4096, ctypes.byref(count), None) == -1
    assert b"null" in lib.mogt_last_error()
    assert lib.mogt_workspace_faults(1, 16, ctypes.byref(count), None) == -2
    assert b"workspace" in lib.mogt_last_error()


def test_generic_scan_host_checks(lib):
    """The generic affine scan validates on the host: state dtype, rank limit,
    I/O dtypes, no prefix with the reverse scan, and a workspace for more
    than one chunk (the sequence is one chunk up to 16 steps)."""
    F32, BF16, F64 = _lib.MOGT_F32, _lib.MOGT_BF16, _lib.MOGT_F64
    ws = lib.mogt_affine_scan_generic_workspace_bytes
    assert ws(1, 16, 4, 3, 1, F64) == 256
    assert ws(1, 17, 4, 3, 1, F64) > ws(1, 17, 4, 3, 0, F64) > ws(1, 17, 4, 3, 0, F32) > 256
    assert ws(1, 17, 1025, 3, 0, F32) == 256
    fwd = lib.mogt_affine_scan_generic_fwd
    rc = fwd(1, 1, 1, None, 1, 8, 4, 3, F32, BF16, F32, 0, None, 0, None)
    assert rc == -1 and b"state dtype" in lib.mogt_last_error()
    rc = fwd(1, 1, 1, None, 1, 8, 1025, 3, F32, F32, F32, 0, None, 0, None)
    assert rc == -1 and b"limit" in lib.mogt_last_error()
    assert fwd(1, 1, 1, None, 1, 8, 4, 3, 7, F32, F32, 0, None, 0, None) == -1
    rc = fwd(1, 1, 1, 1, 1, 8, 4, 3, F32, F32, F32, 1, None, 0, None)
    assert rc == -1 and b"reverse" in lib.mogt_last_error()
    rc = fwd(1, 1, 1, None, 1, 17, 4, 3, F32, F64, F64, 0, None, 0, None)
    assert rc == -2 and b"workspace" in lib.mogt_last_error()
    assert fwd(None, None, None, None, 0, 17, 4, 3, F32, F64, F64, 0, None, 0, None) == 0
    rc = fwd(None, 1, 1, None, 1, 8, 4, 3, F32, F64, F64, 0, None, 0, None)
    assert rc == -1 and b"null" in lib.mogt_last_error()


def test_generic_local_scan_host_checks(lib):
    F32, F64 = _lib.MOGT_F32, _lib.MOGT_F64
    fn = lib.mogt_affine_local_scan_generic
    rc = fn(1, 1, 1, 1, 1, 8, 40, 3, 0, F32, F32, F32, None)
    assert rc == -1 and b"block_size" in lib.mogt_last_error()
    rc = fn(1, 1, None, 1, 1, 8, 40, 3, 4, F32, F32, F32, None)
    assert rc == -1 and b"null" in lib.mogt_last_error()
    assert fn(1, 1, 1, 1, 1, 8, 40, 3, 4, F32, 1, F32, None) == -1   # bf16 state
    assert fn(None, None, None, None, 0, 8, 40, 3, 4, F32, F64, F64, None) == 0
