"""mogt_diag_scan_fwd_noalloc (look-back state in the library's own device
array) gives the same results as mogt_diag_scan_fwd with a caller workspace,
call after call, including a smaller problem after a larger one.

Two launches of the single-pass scan agree to fp32 rounding, not bit for bit:
a chunk's look-back folds either a predecessor's aggregate or its inclusive
prefix, whichever it finds published first, and the products round
differently.  The bar is the fp32 parity bar (normwise relative error 1e-4)."""
import numpy as np
import pytest

from conftest import announce, rel_err, to_np

TOL = 1e-4

from mogt_amd import _lib


def _inputs(B, L, D, dtype, seed):
    import torch

    rng = np.random.default_rng(seed)
    a = 1.0 / (1.0 + np.exp(-rng.normal(3.0, 1.0, (B, L, D))))
    b = rng.normal(0.0, 0.5, (B, L, D))
    dev = torch.device("cuda:0")
    return (torch.from_numpy(a.astype(np.float32)).to(dev).to(dtype),
            torch.from_numpy(b.astype(np.float32)).to(dev).to(dtype))


def _run_both(lib, a, b, out_dtype, with_prefix):
    import torch

    from mogt_amd import ops

    B, L, D = a.shape
    ic, oc = ops.dtype_code(a.dtype, "t"), ops.dtype_code(out_dtype, "t")
    stream = torch.cuda.current_stream().cuda_stream
    h_ref = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    h_na = torch.full(a.shape, float("nan"), dtype=out_dtype, device=a.device)
    p_ref = torch.empty_like(h_ref) if with_prefix else None
    p_na = torch.full_like(h_na, float("nan")) if with_prefix else None
    ws = ops.workspace(lib.mogt_diag_scan_workspace_bytes(B, L, D, ic), a.device)
    rc = lib.mogt_diag_scan_fwd(a.data_ptr(), b.data_ptr(), h_ref.data_ptr(),
                                p_ref.data_ptr() if with_prefix else None, B, L, D, ic, oc,
                                ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "mogt_diag_scan_fwd")
    rc = lib.mogt_diag_scan_fwd_noalloc(a.data_ptr(), b.data_ptr(), h_na.data_ptr(),
                                        p_na.data_ptr() if with_prefix else None, B, L, D, ic, oc,
                                        stream)
    _lib.check(rc, "mogt_diag_scan_fwd_noalloc")
    torch.cuda.synchronize()
    return h_ref, h_na, p_ref, p_na


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(gpu):
    import torch

    lib = _lib.load()
    # first call: configs[1] headline shape, fp32 I/O
    announce("noalloc diag scan B1 L32768 D768 fp32")
    a, b = _inputs(1, 32768, 768, torch.float32, seed=11)
    h_ref, h_na, _, _ = _run_both(lib, a, b, torch.float32, False)
    assert rel_err(to_np(h_na), to_np(h_ref)) <= TOL
    # second call, smaller and of another kind: bf16 inputs, fp32 outputs, prefix
    announce("noalloc diag scan B2 L1000 D256 bf16 prefix")
    a, b = _inputs(2, 1000, 256, torch.bfloat16, seed=12)
    h_ref, h_na, p_ref, p_na = _run_both(lib, a, b, torch.float32, True)
    assert rel_err(to_np(h_na), to_np(h_ref)) <= TOL
    assert rel_err(to_np(p_na), to_np(p_ref)) <= TOL
    # third call back at a larger size: the array keeps working after shrinking
    announce("noalloc diag scan B1 L8192 D768 fp32 again")
    a, b = _inputs(1, 8192, 768, torch.float32, seed=13)
    h_ref, h_na, _, _ = _run_both(lib, a, b, torch.float32, False)
    assert rel_err(to_np(h_na), to_np(h_ref)) <= TOL
    assert bool(torch.isfinite(h_na).all())


def test_noalloc_rejects_problems_beyond_its_array():
    lib = _lib.load()
    # 4 x 2^20 x 4096 needs far more than the 8 MiB array; refused on the host
    rc = lib.mogt_diag_scan_fwd_noalloc(256, 256, 256, None, 4, 1 << 20, 4096, _lib.MOGT_F32,
                                        _lib.MOGT_F32, None)
    assert rc == -1
    assert b"no-allocation" in lib.mogt_last_error()
