"""GPU parity of the rank-1 coupled write-forget scan
against the float64 oracle on the same bf16-rounded inputs; bar 2e-2 (bf16 I/O,
fp32 state)."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from mogt_amd import synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _run(gpu, B, L, H, seed, out_dtype=torch.bfloat16):
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(B, L, H, 64, seed=seed)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    y = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y, ref


@pytest.mark.parametrize("B,L,H", [(1, 1, 1), (1, 64, 2), (1, 200, 3), (2, 1000, 2)])
def test_small_and_ragged(gpu, B, L, H):
    announce(f"rank1 B={B} L={L} H={H}")
    y, ref = _run(gpu, B, L, H, seed=L + H)
    assert y.shape == (B, L, H, 64) and y.dtype == torch.bfloat16
    assert rel_err(to_np(y), ref) <= BF16_TOL
    # fp32 output: the bulk agrees much tighter than the bf16 bar
    y32, _ = _run(gpu, B, L, H, seed=L + H, out_dtype=torch.float32)
    assert rel_err(to_np(y32), ref) <= 5e-3


def test_cfg3_full_size(gpu):
    """B=2, L=8192, H=12, d=64, bf16 I/O."""
    announce("rank1 cfg3 full size")
    y, ref = _run(gpu, 2, 8192, 12, seed=0)
    assert rel_err(to_np(y), ref) <= BF16_TOL


def test_equals_dense_scan_with_scalar_transport(gpu):
    """Same recurrence through the dense pipeline with R = 1: U = f, V = (1-f) vec(v k^T)
    (C = 64*64), then y = S q."""
    announce("rank1 vs dense scan")
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(1, 300, 1, 64, seed=3)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16().float() for x in (f, k, v, q))
    U = ft[0, :, 0].reshape(1, 300, 1, 1).contiguous()
    V = ((1 - ft[0, :, 0, None, None]) * (vt[0, :, 0, :, None] * kt[0, :, 0, None, :]))
    S = mogt_amd.ops.affine_scan(U, V.reshape(1, 300, 1, 64 * 64).contiguous())
    y_dense = torch.einsum("tij,tj->ti", S.reshape(300, 64, 64), qt[0, :, 0])
    y = mogt_amd.ops.rank1_coupled_scan(ft.bfloat16(), kt.bfloat16(), vt.bfloat16(), qt.bfloat16(),
                                        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(to_np(y[0, :, 0]), to_np(y_dense).astype(np.float64)) <= 5e-3


@pytest.mark.parametrize("L,H", [(77, 1), (700, 2)])
def test_fp32_inputs(gpu, L, H):
    """fp32 f, k, v, q (rounded to bf16 inside the products): against the oracle
    on the unrounded inputs, fp32 output."""
    announce(f"rank1 fp32 inputs L={L} H={H}")
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(1, L, H, 64, seed=11 + L)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).float() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    y = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    assert rel_err(to_np(y), ref) <= 1e-2
