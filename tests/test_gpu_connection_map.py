"""GPU parity of the connection-map kernels (model_mogt.py:79-102): batched
matrix exponential and Cayley transform of skew-symmetric generators, against
float64 library routines (torch.matrix_exp, torch.linalg.solve) on the same
inputs, plus the orthogonality the maps must produce.  Bar: the fp32 bar 1e-4
normwise (1e-5 for moderate norms; generators up to ||A||_F ~ 180 are
included, where 8 squarings amplify fp32 rounding); gradients (torch's
routines on the same inputs) against float64 autograd <= 1e-4."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np

pytestmark = pytest.mark.gpu


def _skew(n, r, std, seed):
    g = torch.Generator().manual_seed(seed)
    T = torch.randn(n, r, r, generator=g, dtype=torch.float64) * std
    return T - T.transpose(-1, -2)


def _ref(A64, impl):
    if impl == "matrix_exp":
        return torch.matrix_exp(A64)
    eye = torch.eye(A64.shape[-1], dtype=torch.float64)
    return torch.linalg.solve(eye - 0.5 * A64, eye + 0.5 * A64)


@pytest.mark.parametrize("impl", ["matrix_exp", "cayley"])
@pytest.mark.parametrize("r,std", [(16, 0.05), (16, 1.0), (16, 8.0), (5, 0.5), (32, 0.3), (24, 3.0), (1, 1.0)])
def test_connection_map_matches_library(gpu, impl, r, std):
    announce(f"connection map {impl} r={r} std={std}")
    import mogt_amd

    A64 = _skew(3001, r, std, seed=r * 100 + int(std * 10))
    U = mogt_amd.ops.connection_map(A64.float().to(gpu), impl)
    torch.cuda.synchronize()
    ref = _ref(A64.float().double(), impl)
    assert U.shape == A64.shape and U.dtype == torch.float32
    tol = 1e-5 if std <= 1.0 else 1e-4
    assert rel_err(to_np(U), ref.numpy()) <= tol
    # orthogonality of every map (fp32: U^T U - I is about twice U's error)
    Ud = U.double().cpu()
    eye = torch.eye(r, dtype=torch.float64)
    assert float((Ud.transpose(-1, -2) @ Ud - eye).abs().max()) <= 4 * tol


def test_connection_map_damping_scale_dtype(gpu):
    announce("connection map damping / scale / bf16")
    import mogt_amd

    A64 = _skew(500, 16, 2.0, seed=7)
    A = A64.float().to(gpu)
    for impl in ("matrix_exp", "cayley"):
        U = mogt_amd.ops.connection_map(A, impl, scale=1 / 16, damping=0.999, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        ref = 0.999 * _ref(A64.float().double() / 16, impl)
        assert U.dtype == torch.bfloat16
        assert rel_err(to_np(U), ref.numpy()) <= 1e-2


def test_connection_map_backward(gpu):
    announce("connection map backward")
    import mogt_amd

    A64 = _skew(64, 16, 0.5, seed=11)
    W = torch.randn(64, 16, 16, dtype=torch.float64, generator=torch.Generator().manual_seed(12))
    for impl in ("matrix_exp", "cayley"):
        A = A64.float().to(gpu).requires_grad_()
        U = mogt_amd.ops.connection_map(A, impl, damping=0.9)
        (U * W.float().to(gpu)).sum().backward()
        torch.cuda.synchronize()
        Ar = A64.clone().requires_grad_()
        ((0.9 * _ref(Ar, impl)) * W).sum().backward()
        assert rel_err(to_np(A.grad), Ar.grad.numpy()) <= 1e-4


def test_connection_map_errors(gpu):
    import mogt_amd

    with pytest.raises(ValueError):
        mogt_amd.ops.connection_map(torch.zeros(2, 33, 33, device=gpu), "cayley")
    with pytest.raises(ValueError):
        mogt_amd.ops.connection_map(torch.zeros(2, 4, 4, device=gpu), "qr")
    with pytest.raises(ValueError):
        mogt_amd.ops.connection_map(torch.zeros(2, 4, 5, device=gpu), "cayley")
