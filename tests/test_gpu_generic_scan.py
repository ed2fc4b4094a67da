"""GPU parity of the generic affine scan (float64 state, ranks above 32, fp16 /
fp64 I/O, host tensors, autograd) through the drop-in ``affine_scan`` /
``triton_scan`` names, against the float64 oracle and the reference's own
sanity checks (sanity_affine_scan.py:19-61, :102-135).

Bars: float64 state, float64 output: max abs error <= 1e-10 (the reference's
own bar between its three scans) and normwise relative error <= 1e-12 against
the oracle; fp32 state: relative error <= 1e-4; bf16 output 2e-2; fp16 output
2e-3."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err
from mogt_amd import synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

F64_TOL = 1e-12
FP32_TOL = 1e-4


def np64(t):
    return t.detach().double().cpu().numpy()


def _stable(B, L, R, C, seed, dtype=np.float64):
    """U = I + N(0, 0.3^2 / R) rescaled to spectral norm <= 1, V ~ N(0,1)."""
    g = synthetic.rng(seed)
    U = np.eye(R) + (0.3 / np.sqrt(R)) * g.standard_normal((B, L, R, R))
    U /= np.maximum(1.0, np.linalg.norm(U, ord=2, axis=(-2, -1)))[..., None, None]
    V = g.standard_normal((B, L, R, C))
    return U.astype(dtype), V.astype(dtype)


def _torch_seq(U, V, prefix):
    """H_t = U_t H_{t-1} + V_t as a torch loop on the host, so that
    torch.autograd derives its gradients (the reference's backward check,
    sanity_affine_scan.py:102-135)."""
    B, L, R, C = V.shape
    H = torch.zeros(B, R, C, dtype=U.dtype)
    P = torch.eye(R, dtype=U.dtype).expand(B, R, R)
    Hs, Ps = [], []
    for t in range(L):
        H = torch.bmm(U[:, t], H) + V[:, t]
        Hs.append(H)
        if prefix:
            P = torch.bmm(U[:, t], P)
            Ps.append(P)
    return (torch.stack(Ps, 1) if prefix else None), torch.stack(Hs, 1)


def test_reference_sanity_script_fp64_host_tensors(gpu):
    """run_affine_scan_sanity (sanity_affine_scan.py:19-61) as the reference
    writes it: host float64 tensors, state and output float64, the three scans
    with return_prefix=True agreeing within 1e-10; here also against the
    oracle."""
    announce("generic scan: reference sanity script, float64, host tensors")
    from mogt_amd import affine_scan as das

    U, V = synthetic.reference_test_case()
    kw = dict(state_dtype=torch.float64, output_dtype=torch.float64, return_prefix=True)
    U_seq, H_seq = das.affine_scan_sequential(U, V, **kw)
    U_par, H_par = das.affine_scan_doubling(U, V, **kw)
    U_blk, H_blk = das.affine_scan_block_reference(U, V, block_size=5, carry_scan="doubling", **kw)
    for t in (U_seq, H_seq, U_par, H_par, U_blk, H_blk):
        assert t.device.type == "cpu" and t.dtype == torch.float64
    for a, b in ((U_seq, U_par), (H_seq, H_par), (U_seq, U_blk), (H_seq, H_blk)):
        assert float((a - b).abs().max()) <= 1e-10
    P_ref, H_ref = so.affine_scan_sequential(U.numpy(), V.numpy(), return_prefix=True)
    assert np.max(np.abs(H_seq.numpy() - H_ref)) <= 1e-10
    assert np.max(np.abs(U_seq.numpy() - P_ref)) <= 1e-10
    assert rel_err(H_seq.numpy(), H_ref) <= F64_TOL and rel_err(U_seq.numpy(), P_ref) <= F64_TOL


def test_reference_backward_sanity_fp64(gpu):
    """run_affine_backward_sanity (sanity_affine_scan.py:102-135): autograd
    through affine_scan_sequential vs affine_scan_sequential_backward, float64,
    host tensors, bar 1e-10; both also against the oracle's backward."""
    announce("generic scan: reference backward sanity, float64")
    from mogt_amd import affine_scan as das

    U, V = synthetic.reference_test_case(seq_len=9, rank=4, channels=3)
    grad_out = torch.randn_like(V)
    U_ref = U.detach().clone().requires_grad_(True)
    V_ref = V.detach().clone().requires_grad_(True)
    H = das.affine_scan_sequential(U_ref, V_ref, state_dtype=torch.float64, output_dtype=torch.float64)
    gU_auto, gV_auto = torch.autograd.grad(H, (U_ref, V_ref), grad_outputs=grad_out)
    gU, gV = das.affine_scan_sequential_backward(U, V, grad_out, state_dtype=torch.float64)
    assert gU.device.type == "cpu" and gU.dtype == torch.float64
    assert float((gU_auto - gU).abs().max()) <= 1e-10
    assert float((gV_auto - gV).abs().max()) <= 1e-10
    gU_ref, gV_ref = so.affine_scan_sequential_backward(U.numpy(), V.numpy(), grad_out.numpy())
    assert np.max(np.abs(gU.numpy() - gU_ref)) <= 1e-10
    assert np.max(np.abs(gV.numpy() - gV_ref)) <= 1e-10


@pytest.mark.parametrize("B,L,R,C", [(2, 3000, 16, 48), (1, 5000, 4, 3), (3, 700, 24, 5), (1, 17, 1, 1),
                                     (1, 40, 1, 600), (2, 33, 2, 300)])
def test_fp64_state_multichunk(gpu, B, L, R, C):
    """float64 state across many chunks (carry pass and chunk summaries), with
    the prefix product, on the device."""
    announce(f"generic scan fp64 B={B} L={L} R={R} C={C}")
    import mogt_amd.ops as ops

    U, V = _stable(B, L, R, C, seed=L + R)
    P_ref, H_ref = so.affine_scan_sequential(U, V, return_prefix=True)
    Ug, Vg = torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu)
    P, H = ops.affine_scan(Ug, Vg, state_dtype=torch.float64, return_prefix=True)
    H_only = ops.affine_scan(Ug, Vg, state_dtype=torch.float64)
    torch.cuda.synchronize()
    assert H.dtype == torch.float64 and P.dtype == torch.float64
    assert rel_err(np64(H), H_ref) <= F64_TOL
    assert rel_err(np64(P), P_ref) <= F64_TOL
    assert torch.equal(H_only, H)


@pytest.mark.parametrize("R,L,C", [(33, 300, 4), (48, 257, 8), (64, 200, 3), (65, 150, 2), (100, 90, 5),
                                   (130, 40, 3)])
def test_ranks_above_32(gpu, R, L, C):
    """Ranks the matrix-core pipeline does not take: fp32 state (transitions
    staged in LDS up to R = 64, read from memory above), through the hybrid
    drop-in, with the prefix product; float64 state at the same shapes."""
    announce(f"generic scan R={R} L={L} C={C}")
    from mogt_amd import affine_scan as das
    from mogt_amd import triton_scan

    U, V = _stable(1, L, R, C, seed=R)
    P_ref, H_ref = so.affine_scan_sequential(U, V, return_prefix=True)
    U32, V32 = torch.from_numpy(U.astype(np.float32)).to(gpu), torch.from_numpy(V.astype(np.float32)).to(gpu)
    P, H = triton_scan.triton_affine_scan_hybrid(U32, V32, return_prefix=True)
    H2 = triton_scan.triton_affine_scan_hybrid(U32, V32)
    P64, H64 = das.affine_scan_sequential(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu),
                                          state_dtype=torch.float64, return_prefix=True)
    torch.cuda.synchronize()
    assert H.dtype == torch.float32
    assert rel_err(np64(H), H_ref) <= FP32_TOL and rel_err(np64(P), P_ref) <= FP32_TOL
    assert torch.equal(H, H2)
    assert rel_err(np64(H64), H_ref) <= F64_TOL and rel_err(np64(P64), P_ref) <= F64_TOL


@pytest.mark.parametrize("R", [40, 16])
def test_fused_scan_generic_ranks(gpu, R):
    """triton_fused_scan beyond R = 32 (the generic scan's prefix columns with
    no channels) and a float64 output at R = 16."""
    announce(f"generic fused scan R={R}")
    from mogt_amd import triton_scan

    U, _ = _stable(2, 333, R, 1, seed=5 + R)
    Y_ref = so.fused_scan(U)
    if R > 32:
        Y = triton_scan.triton_fused_scan(torch.from_numpy(U.astype(np.float32)).to(gpu))
        tol = FP32_TOL
    else:
        import mogt_amd.ops as ops
        Y = ops.fused_scan(torch.from_numpy(U.astype(np.float32)).to(gpu), output_dtype=torch.float64)
        tol = FP32_TOL
        assert Y.dtype == torch.float64
    torch.cuda.synchronize()
    assert rel_err(np64(Y), Y_ref) <= tol


@pytest.mark.parametrize("vdt,odt,sdt,tol", [
    (torch.bfloat16, torch.float64, torch.float64, F64_TOL),
    (torch.float16, torch.float16, torch.float64, 2e-3),
    (torch.float64, torch.bfloat16, torch.float64, 2e-2),
    (torch.float64, torch.float32, torch.float32, FP32_TOL),
    (torch.float16, torch.float32, torch.float32, FP32_TOL),
])
def test_io_dtypes(gpu, vdt, odt, sdt, tol):
    """Inputs and outputs in fp16 / bf16 / fp64: V is converted to the state
    dtype on load (V.to(state_dtype), affine_scan.py:36), outputs rounded from
    the state (H_t.to(output_dtype), :52)."""
    announce(f"generic scan V {vdt} out {odt} state {sdt}")
    import mogt_amd.ops as ops

    U, V = _stable(2, 400, 8, 6, seed=11)
    Vt = torch.from_numpy(V).to(vdt)
    P_ref, H_ref = so.affine_scan_sequential(U, Vt.double().numpy(), return_prefix=True)
    Ug = torch.from_numpy(U).to(gpu).to(sdt)
    P, H = ops.affine_scan(Ug, Vt.to(gpu), output_dtype=odt, state_dtype=sdt, return_prefix=True)
    torch.cuda.synchronize()
    assert H.dtype == odt and P.dtype == odt
    if sdt == torch.float32:
        P_ref, H_ref = so.affine_scan_sequential(U.astype(np.float32).astype(np.float64), Vt.double().numpy(),
                                                 return_prefix=True)
    assert rel_err(np64(H.double()), H_ref) <= tol
    assert rel_err(np64(P.double()), P_ref) <= tol


@pytest.mark.parametrize("R,L,C,sdt", [(40, 120, 5, torch.float64), (6, 300, 4, torch.float64),
                                       (12, 150, 7, torch.float32)])
def test_autograd_with_prefix(gpu, R, L, C, sdt):
    """Gradients through both outputs (U_prefix and H) of the differentiable
    drop-in against torch.autograd of a host float64 loop; without the prefix
    against the oracle's backward.  fp32 state (R <= 32) runs on the
    matrix-core pipeline and its autograd."""
    announce(f"generic scan autograd R={R} L={L} C={C} state {sdt}")
    from mogt_amd import affine_scan as das

    U, V = _stable(2, L, R, C, seed=R + C)
    g = synthetic.rng(99)
    dP = torch.from_numpy(g.standard_normal(U.shape))
    dH = torch.from_numpy(g.standard_normal(V.shape))
    Uc = torch.from_numpy(U).requires_grad_(True)
    Vc = torch.from_numpy(V).requires_grad_(True)
    P_c, H_c = _torch_seq(Uc, Vc, True)
    gU_ref, gV_ref = torch.autograd.grad((P_c * dP).sum() + (H_c * dH).sum(), (Uc, Vc))

    tdt = torch.float64 if sdt == torch.float64 else torch.float32
    tol = F64_TOL if sdt == torch.float64 else FP32_TOL
    Ug = torch.from_numpy(U).to(gpu, tdt).requires_grad_(True)
    Vg = torch.from_numpy(V).to(gpu, tdt).requires_grad_(True)
    P, H = das.affine_scan_sequential(Ug, Vg, state_dtype=sdt, return_prefix=True)
    gU, gV = torch.autograd.grad((P * dP.to(gpu, tdt)).sum() + (H * dH.to(gpu, tdt)).sum(), (Ug, Vg))
    torch.cuda.synchronize()
    assert gU.dtype == tdt and gV.dtype == tdt
    assert rel_err(np64(gU.double()), gU_ref.numpy()) <= tol
    assert rel_err(np64(gV.double()), gV_ref.numpy()) <= tol

    gU_o, gV_o = so.affine_scan_sequential_backward(U, V, dH.numpy())
    Ug2 = Ug.detach().requires_grad_(True)
    Vg2 = Vg.detach().requires_grad_(True)
    H2 = das.affine_scan_doubling(Ug2, Vg2, state_dtype=sdt)
    H2.backward(dH.to(gpu, tdt))
    torch.cuda.synchronize()
    assert rel_err(np64(Ug2.grad.double()), gU_o) <= tol
    assert rel_err(np64(Vg2.grad.double()), gV_o) <= tol


def test_hand_backward_fp64_long(gpu):
    """affine_scan_sequential_backward in float64 over many chunks (the
    generic reverse scan with transposed transitions), R = 20."""
    announce("generic reverse scan fp64 L=2500 R=20")
    from mogt_amd import affine_scan as das

    U, V = _stable(2, 2500, 20, 9, seed=3)
    G = synthetic.rng(4).standard_normal(V.shape)
    gU_ref, gV_ref = so.affine_scan_sequential_backward(U, V, G)
    gU, gV = das.affine_scan_sequential_backward(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu),
                                                 torch.from_numpy(G).to(gpu), state_dtype=torch.float64)
    only_v = das.affine_scan_sequential_backward(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu),
                                                 torch.from_numpy(G).to(gpu), state_dtype=torch.float64,
                                                 need_grad_u=False)
    torch.cuda.synchronize()
    assert only_v[0] is None and torch.equal(only_v[1], gV)
    assert rel_err(np64(gV), gV_ref) <= F64_TOL
    assert rel_err(np64(gU), gU_ref) <= F64_TOL


def test_generic_argument_errors(gpu):
    from mogt_amd import affine_scan as das
    import mogt_amd.ops as ops

    U = torch.zeros(1, 4, 3, 3, device=gpu)
    V = torch.zeros(1, 4, 3, 2, device=gpu)
    with pytest.raises(ValueError):
        das.affine_scan_sequential(U, V, state_dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.affine_scan(U, V, output_dtype=torch.int32)
    with pytest.raises(ValueError):
        das.affine_scan_sequential(torch.zeros(1, 2, 1025, 1025, device=gpu, dtype=torch.bfloat16),
                                   torch.zeros(1, 2, 1025, 1, device=gpu))
    # empty problems; no channels leaves the prefix product alone (U = 2 I: 2^(t+1) I)
    assert das.affine_scan_sequential(U[:, :0], V[:, :0], state_dtype=torch.float64).shape == (1, 0, 3, 2)
    U2 = (2 * torch.eye(3, device=gpu)).expand(1, 4, 3, 3)
    P, H = das.affine_scan_sequential(U2, V[..., :0], state_dtype=torch.float64, return_prefix=True)
    torch.cuda.synchronize()
    want = torch.stack([2.0 ** (t + 1) * torch.eye(3, dtype=torch.float64) for t in range(4)])[None]
    assert H.shape == (1, 4, 3, 0) and torch.equal(P.cpu(), want)


def test_zz_generic_no_lookback_wait_gave_up(gpu):
    import mogt_amd.ops as ops

    assert ops.workspace_faults() == 0


@pytest.mark.parametrize("R,block", [(40, 1), (40, 7), (64, 64), (100, 33)])
def test_local_scan_ranks_above_32(gpu, R, block):
    """triton_affine_local_scan beyond R = 32 (the generic kernel's block-local
    pass): per-step prefixes and per-block summaries against the oracle's
    local_scan, ragged tail block included."""
    announce(f"generic local scan R={R} block={block}")
    from mogt_amd import triton_scan

    U, V = _stable(2, 155, R, 3, seed=R + block)
    ref = so.local_scan(U, V, block_size=block)
    out = triton_scan.triton_affine_local_scan(torch.from_numpy(U.astype(np.float32)).to(gpu),
                                               torch.from_numpy(V.astype(np.float32)).to(gpu), block_size=block)
    torch.cuda.synchronize()
    for got, want in zip(out, ref):
        assert got.dtype == torch.float32 and tuple(got.shape) == want.shape
        assert rel_err(np64(got), want) <= FP32_TOL


def test_dense_scan_vk_rank_above_32(gpu):
    """dense_scan(A, v=v, k=k) at R = 48: B_t = v_t k_t^T formed as fp32
    products and scanned by the generic kernel, against the oracle."""
    announce("generic dense_scan vk R=48")
    import mogt_amd

    U, _ = _stable(2, 200, 48, 1, seed=48)
    g = synthetic.rng(5)
    v = g.standard_normal((2, 200, 48)).astype(np.float32)
    k = g.standard_normal((2, 200, 20)).astype(np.float32)
    V = (v[..., :, None] * k[..., None, :]).astype(np.float64)
    H_ref = so.affine_scan_sequential(U.astype(np.float32).astype(np.float64), V)
    S = mogt_amd.dense_scan(torch.from_numpy(U.astype(np.float32)).to(gpu), v=torch.from_numpy(v).to(gpu),
                            k=torch.from_numpy(k).to(gpu))
    torch.cuda.synchronize()
    assert S.dtype == torch.float32 and S.shape == (2, 200, 48, 20)
    assert rel_err(np64(S), H_ref) <= FP32_TOL


@pytest.mark.parametrize("sdt,tol", [(torch.float64, F64_TOL), (torch.float32, FP32_TOL)])
def test_hand_backward_rank_above_64(gpu, sdt, tol):
    """The reverse scan with U read transposed from memory (R > 64, not staged
    in LDS), several chunks: affine_scan_sequential_backward against the
    oracle."""
    announce(f"generic reverse scan R=70 L=300 state {sdt}")
    from mogt_amd import affine_scan as das

    U, V = _stable(1, 300, 70, 3, seed=70)
    G = synthetic.rng(8).standard_normal(V.shape)
    tdt = torch.float64 if sdt == torch.float64 else torch.float32
    if sdt == torch.float32:
        U, V, G = (x.astype(np.float32).astype(np.float64) for x in (U, V, G))
    gU_ref, gV_ref = so.affine_scan_sequential_backward(U, V, G)
    gU, gV = das.affine_scan_sequential_backward(torch.from_numpy(U).to(gpu, tdt), torch.from_numpy(V).to(gpu, tdt),
                                                 torch.from_numpy(G).to(gpu, tdt), state_dtype=sdt)
    torch.cuda.synchronize()
    assert gU.dtype == tdt and gV.dtype == tdt
    assert rel_err(np64(gV), gV_ref) <= tol
    assert rel_err(np64(gU), gU_ref) <= tol
