"""Empty inputs (B = 0 or L = 0, no rows) through every entry point: each
returns an empty result of the right shape and dtype without a launch (a
zero-size grid is a launch error on the device).  The reference's sequential
scan (affine_scan.py:48-58) has nothing to stack for L = 0; here the empty
sequence maps to an empty output."""
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,L", [(0, 5), (2, 0)])
def test_scans_empty(gpu, B, L):
    announce(f"empty scans B={B} L={L}")
    import mogt_amd
    from mogt_amd import ops, triton_scan

    a = torch.rand(B, L, 8, device=gpu)
    assert mogt_amd.diag_scan(a, a).shape == (B, L, 8)
    assert mogt_amd.diag_scan(a.bfloat16(), a.bfloat16(), out_dtype=torch.float32).dtype == torch.float32
    assert torch.ops.mogt.diag_scan_rev(a, a).shape == (B, L, 8)
    z = torch.zeros(B, L, 4, device=gpu)
    v = torch.zeros(B, L, 4 * 6, device=gpu)
    assert mogt_amd.coupled_rank_scan(z, v).shape == (B, L, 24)
    assert torch.ops.mogt.coupled_scan_rev(z, v, 4, 1.0).shape == (B, L, 24)
    U = torch.zeros(B, L, 16, 16, device=gpu)
    V = torch.zeros(B, L, 16, 8, device=gpu)
    assert triton_scan.triton_affine_scan_hybrid(U, V).shape == (B, L, 16, 8)
    up, hp = triton_scan.triton_affine_scan_hybrid(U, V, return_prefix=True)
    assert up.shape == (B, L, 16, 16) and hp.shape == (B, L, 16, 8)
    assert triton_scan.triton_fused_scan(U).shape == (B, L, 16, 16)
    vv = torch.zeros(B, L, 16, device=gpu)
    assert ops.dense_scan(U, v=vv, k=vv).shape == (B, L, 16, 16)
    f = torch.rand(B, L, 3, device=gpu)
    kq = torch.zeros(B, L, 3, 64, device=gpu, dtype=torch.bfloat16)
    assert ops.rank1_coupled_scan(f, kq, kq, kq).shape == (B, L, 3, 64)
    torch.cuda.synchronize()


def test_local_scan_and_rows_empty(gpu):
    announce("empty local scan, connection maps, row kernels")
    from mogt_amd import ops, triton_scan

    U = torch.zeros(1, 0, 16, 16, device=gpu)
    V = torch.zeros(1, 0, 16, 8, device=gpu)
    up, hp, us, hs = triton_scan.triton_affine_local_scan(U, V, block_size=32)
    assert up.shape == (1, 0, 16, 16) and hp.shape == (1, 0, 16, 8)
    assert us.shape == (1, 0, 16, 16) and hs.shape == (1, 0, 16, 8)
    A = torch.zeros(0, 16, 16, device=gpu)
    for impl in ("matrix_exp", "cayley"):
        assert ops.connection_map(A, impl).shape == (0, 16, 16)
    x = torch.zeros(0, 64, device=gpu)
    w = torch.ones(64, device=gpu)
    assert ops.rmsnorm(x, w, 1e-6).shape == (0, 64)
    xo, out = ops.add_rmsnorm(x, x, 0.5, w, 1e-6)
    assert xo.shape == (0, 64) and out.shape == (0, 64)
    assert ops.silu_mul(torch.zeros(0, 128, device=gpu)).shape == (0, 64)
    loss, lse = ops.lm_ce_forward(torch.zeros(0, 50, device=gpu), torch.zeros(0, dtype=torch.int64, device=gpu))
    assert loss.shape == (0,) and lse.shape == (0,)
    torch.cuda.synchronize()
