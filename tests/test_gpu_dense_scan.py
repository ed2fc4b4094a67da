"""GPU parity of the dense affine scan pipeline (drop-in triton_scan / affine_scan
API) against the CPU oracle on identical seeded inputs.  fp32 bar: normwise
max relative error <= 1e-4; bf16 V I/O: <= 2e-2."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from mogt_amd import synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _stable_affine(B, L, R, C, seed, scale=0.05):
    """U = I + scale*N(0,1) (the reference's sanity distribution) rescaled so the
    spectral norm stays <= 1 over long sequences; V ~ N(0,1)."""
    g = synthetic.rng(seed)
    U = np.eye(R, dtype=np.float32) + np.float32(scale) * g.standard_normal((B, L, R, R), dtype=np.float32)
    U /= np.maximum(1.0, np.linalg.norm(U, ord=2, axis=(-2, -1)))[..., None, None].astype(np.float32)
    V = g.standard_normal((B, L, R, C), dtype=np.float32)
    return U, V


def test_reference_sanity_case_fp32(gpu):
    """sanity_affine_scan.py:11-16 inputs (seed 42, B2 L17 R4 C3), prefix included."""
    announce("dense reference sanity case")
    from mogt_amd import triton_scan

    Ut, Vt = synthetic.reference_test_case()
    U, V = Ut.float().numpy(), Vt.float().numpy()
    P_ref, H_ref = so.affine_scan_sequential(U, V, return_prefix=True)
    P, H = triton_scan.triton_affine_scan_hybrid(
        torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu), block_size=5,
        carry_scan="doubling", output_dtype=torch.float32, return_prefix=True)
    torch.cuda.synchronize()
    assert rel_err(to_np(H), H_ref) <= FP32_TOL
    assert rel_err(to_np(P), P_ref) <= FP32_TOL


def test_reference_triton_sanity_case(gpu):
    """sanity_affine_scan.py:64-99: B1 L64 R16 C8, block 32, block_c 8; the
    reference asserts 5e-5 max abs against the sequential scan."""
    announce("dense triton sanity case")
    from mogt_amd import triton_scan

    Ut, Vt = synthetic.reference_test_case(batch_size=1, seq_len=64, rank=16, channels=8)
    U, V = Ut.float().numpy(), Vt.float().numpy()
    P_ref, H_ref = so.affine_scan_sequential(U, V, return_prefix=True)
    P, H = triton_scan.triton_affine_scan_hybrid(
        torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu), block_size=32, block_c=8,
        carry_scan="sequential", output_dtype=torch.float32, return_prefix=True)
    torch.cuda.synchronize()
    assert np.max(np.abs(to_np(H) - H_ref)) <= 5e-5
    assert np.max(np.abs(to_np(P) - P_ref)) <= 5e-5


@pytest.mark.parametrize("B,L,R,C", [
    (1, 1, 4, 3), (2, 31, 3, 5), (1, 1000, 16, 48), (3, 777, 7, 11), (1, 2049, 32, 32),
    (2, 600, 16, 70), (1, 500, 5, 130), (1, 4100, 1, 1), (1, 3000, 2, 9),
])
def test_random_shapes(gpu, B, L, R, C):
    announce(f"dense B={B} L={L} R={R} C={C}")
    import mogt_amd.affine_scan as gas

    U, V = _stable_affine(B, L, R, C, seed=B * 1000 + L + R)
    P_ref, H_ref = so.affine_scan_sequential(U, V, return_prefix=True)
    P, H = gas.affine_scan_sequential(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu),
                                      return_prefix=True)
    torch.cuda.synchronize()
    assert H.dtype == torch.float32 and P.shape == (B, L, R, R)
    assert rel_err(to_np(H), H_ref) <= FP32_TOL
    assert rel_err(to_np(P), P_ref) <= FP32_TOL


def test_bf16_values_and_output(gpu):
    announce("dense bf16 V / bf16 out")
    import mogt_amd

    U, V = _stable_affine(1, 3000, 16, 48, seed=9)
    Vt = torch.from_numpy(V).to(gpu).bfloat16()
    H_ref = so.affine_scan_sequential(U, to_np(Vt).astype(np.float64))
    H = mogt_amd.ops.affine_scan(torch.from_numpy(U).to(gpu), Vt)
    torch.cuda.synchronize()
    assert H.dtype == torch.bfloat16
    assert rel_err(to_np(H), H_ref) <= BF16_TOL
    H32 = mogt_amd.ops.affine_scan(torch.from_numpy(U).to(gpu), Vt, output_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(to_np(H32), H_ref) <= FP32_TOL


def test_identity_transport_is_cumsum_and_scalar_decay_is_diag(gpu):
    announce("dense U=I cumsum / U=f I")
    import mogt_amd

    g = synthetic.rng(4)
    L, R, C = 5000, 16, 48
    V = g.standard_normal((1, L, R, C), dtype=np.float32)
    U = np.broadcast_to(np.eye(R, dtype=np.float32), (1, L, R, R)).copy()
    H = mogt_amd.ops.affine_scan(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu))
    f = (1.0 / (1.0 + np.exp(-g.standard_normal((1, L), dtype=np.float32) - 3.0))).astype(np.float32)
    Uf = (f[..., None, None] * np.eye(R, dtype=np.float32)).astype(np.float32)
    Hf = mogt_amd.ops.affine_scan(torch.from_numpy(Uf).to(gpu), torch.from_numpy(V).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(H), np.cumsum(V.astype(np.float64), axis=1)) <= FP32_TOL
    a = np.broadcast_to(f[..., None], (1, L, R * C))
    ref = so.diag_scan(a, V.reshape(1, L, R * C)).reshape(1, L, R, C)
    assert rel_err(to_np(Hf), ref) <= FP32_TOL


@pytest.mark.parametrize("R,L", [(16, 2048), (4, 300), (32, 1500)])
def test_fused_scan(gpu, R, L):
    """triton_scan.py:480-494 demo: U = I + 0.01 N(0,1), prefix product."""
    announce(f"fused scan R={R} L={L}")
    from mogt_amd import triton_scan

    g = synthetic.rng(R + L)
    U = (np.eye(R, dtype=np.float32) + np.float32(0.01) * g.standard_normal((2, L, R, R), dtype=np.float32))
    Y = triton_scan.triton_fused_scan(torch.from_numpy(U).to(gpu))
    torch.cuda.synchronize()
    assert Y.dtype == torch.float32
    assert rel_err(to_np(Y), so.fused_scan(U)) <= FP32_TOL


@pytest.mark.parametrize("block", [1, 16, 32, 256, 1000])
def test_local_scan(gpu, block):
    announce(f"local scan block={block}")
    from mogt_amd import triton_scan

    U, V = _stable_affine(2, 777, 16, 24, seed=block)
    ref = so.local_scan(U, V, block_size=block)
    out = triton_scan.triton_affine_local_scan(torch.from_numpy(U).to(gpu),
                                               torch.from_numpy(V).to(gpu), block_size=block)
    torch.cuda.synchronize()
    for got, want in zip(out, ref):
        assert got.dtype == torch.float32 and tuple(got.shape) == want.shape
        assert rel_err(to_np(got), want) <= FP32_TOL


def test_validation_matches_reference(gpu):
    from mogt_amd import triton_scan

    U = torch.zeros(1, 4, 4, 4, device=gpu)
    V = torch.zeros(1, 4, 4, 3, device=gpu)
    with pytest.raises(ValueError):
        triton_scan.triton_affine_scan_hybrid(U, V, carry_scan="tree")
    with pytest.raises(ValueError):
        triton_scan.triton_affine_local_scan(U, V[:, :, :3])
    with pytest.raises(ValueError):
        triton_scan.triton_affine_local_scan(U.cpu(), V.cpu())
    with pytest.raises(ValueError):
        triton_scan.triton_affine_scan_hybrid(U[0], V)


@pytest.mark.parametrize("R,C", [(4, 3), (16, 8)])
def test_backward_matches_oracle(gpu, R, C):
    """sanity_affine_scan.py:102-135 (hand backward vs autograd): here the GPU
    autograd Function against the oracle's reverse scan."""
    announce(f"dense backward R={R} C={C}")
    from mogt_amd import triton_scan

    U, V = _stable_affine(2, 53, R, C, seed=R)
    G = synthetic.rng(7).standard_normal(V.shape, dtype=np.float32)
    gU_ref, gV_ref = so.affine_scan_sequential_backward(U.astype(np.float64), V.astype(np.float64), G)
    Ut = torch.from_numpy(U).to(gpu).requires_grad_(True)
    Vt = torch.from_numpy(V).to(gpu).requires_grad_(True)
    H = triton_scan.triton_affine_scan_hybrid(Ut, Vt, block_size=16)
    H.backward(torch.from_numpy(G).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(Vt.grad), gV_ref) <= FP32_TOL
    assert rel_err(to_np(Ut.grad), gU_ref) <= FP32_TOL


@pytest.mark.parametrize("B,L,R,C", [(1, 1, 4, 3), (2, 33, 16, 8), (1, 1000, 16, 48), (2, 3000, 5, 7),
                                     (1, 5000, 32, 32), (1, 1100, 32, 40), (1, 32768, 16, 48)])
def test_native_reverse_scan_and_grad_u(gpu, B, L, R, C):
    """The backward on the matrix-core pipeline through the C ABI: the
    reverse-time scan G_t = X_t + U_{t+1}^T G_{t+1} (mogt_affine_scan_rev_fwd,
    time walked backwards, U read transposed; one step, ragged lengths, up to
    three recursion levels, R = 32, C with and without 16-byte rows, the
    core-operator shape) and dU_t = G_t H_{t-1}^T (mogt_affine_scan_grad_u)
    against the oracle's backward recursion (affine_scan.py:110-124)."""
    announce(f"dense native reverse scan B={B} L={L} R={R} C={C}")
    from mogt_amd import _lib, ops

    lib = _lib.load()
    U, V = _stable_affine(B, L, R, C, seed=L + R)
    X = synthetic.rng(L + C).standard_normal(V.shape, dtype=np.float32)
    gU_ref, gV_ref = so.affine_scan_sequential_backward(U.astype(np.float64), V.astype(np.float64),
                                                        X.astype(np.float64))
    Ut, Vt, Xt = (torch.from_numpy(a).to(gpu) for a in (U, V, X))
    G = torch.empty_like(Xt)
    ws = ops.workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), gpu)
    sh = ops._stream_handle(gpu)
    _lib.check(lib.mogt_affine_scan_rev_fwd(Ut.data_ptr(), Xt.data_ptr(), G.data_ptr(), B, L, R, C,
                                            ws.data_ptr(), ws.numel(), sh), "rev")
    H = ops.affine_scan(Ut, Vt)
    dU = torch.empty(B, L, R, R, device=gpu)
    _lib.check(lib.mogt_affine_scan_grad_u(G.data_ptr(), H.data_ptr(), None, dU.data_ptr(), B, L, R, C, sh),
               "grad_u")
    torch.cuda.synchronize()
    assert rel_err(to_np(G), gV_ref) <= FP32_TOL
    assert rel_err(to_np(dU), gU_ref) <= FP32_TOL


def test_core_operator_shape_full_length(gpu):
    """The reference's core-operator benchmark shape (U [1, 32768, 16, 16],
    V [1, 32768, 16, 48], fp32; the bench's dense_affine_r16_c48_L32768 line)
    through triton_affine_scan_hybrid, against the oracle, with and without
    the prefix product."""
    announce("dense core shape R16 C48 L32768")
    from mogt_amd import triton_scan

    U, V = _stable_affine(1, 32768, 16, 48, seed=16)
    P_ref, H_ref = so.affine_scan_sequential(U.astype(np.float64), V.astype(np.float64), return_prefix=True)
    Ut, Vt = torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu)
    H = triton_scan.triton_affine_scan_hybrid(Ut, Vt)
    P, H2 = triton_scan.triton_affine_scan_hybrid(Ut, Vt, return_prefix=True)
    torch.cuda.synchronize()
    assert H.dtype == torch.float32
    assert rel_err(to_np(H), H_ref) <= FP32_TOL
    assert rel_err(to_np(H2), H_ref) <= FP32_TOL
    assert rel_err(to_np(P), P_ref) <= FP32_TOL


def test_affine_scan_dropin_names(gpu):
    """mogt_amd.affine_scan's drop-ins for affine_scan.py:14-278, called by
    their own names on the reference's sanity inputs (seed 42, B2 L17 R4 C3 and
    B1 L64 R16 C8): sequential, doubling and block_reference with and without
    return_prefix, the combine operator, and the hand backward."""
    announce("affine_scan drop-in names")
    from mogt_amd import affine_scan as das

    for shape in ((2, 17, 4, 3), (1, 64, 16, 8)):
        Ut, Vt = synthetic.reference_test_case(*shape)
        U, V = Ut.float(), Vt.float()
        P_ref, H_ref = so.affine_scan_sequential(U.double().numpy(), V.double().numpy(), return_prefix=True)
        Ug, Vg = U.to(gpu), V.to(gpu)
        outs = {
            "sequential": das.affine_scan_sequential(Ug, Vg, return_prefix=True),
            "doubling": das.affine_scan_doubling(Ug, Vg, return_prefix=True),
            "block5": das.affine_scan_block_reference(Ug, Vg, block_size=5, return_prefix=True),
            "block5d": das.affine_scan_block_reference(Ug, Vg, block_size=5, carry_scan="doubling",
                                                       return_prefix=True),
        }
        for name, (P, H) in outs.items():
            assert P.dtype == torch.float32 and H.dtype == torch.float32, name
            assert rel_err(to_np(H), H_ref) <= FP32_TOL, name
            assert rel_err(to_np(P), P_ref) <= FP32_TOL, name
        H_only = das.affine_scan_doubling(Ug, Vg, output_dtype=torch.bfloat16)
        assert H_only.dtype == torch.bfloat16 and rel_err(to_np(H_only), H_ref) <= BF16_TOL
        # affine_combine: (U2, V2) o (U1, V1) = (U2 U1, U2 V1 + V2)
        cu, cv = das.affine_combine(Ug[:, 1], Vg[:, 1], Ug[:, 0], Vg[:, 0])
        assert rel_err(to_np(cv), H_ref[:, 1]) <= FP32_TOL and rel_err(to_np(cu), P_ref[:, 1]) <= FP32_TOL
        G = synthetic.rng(3).standard_normal(V.shape).astype(np.float32)
        gU_ref, gV_ref = so.affine_scan_sequential_backward(U.double().numpy(), V.double().numpy(),
                                                            G.astype(np.float64))
        gU, gV = das.affine_scan_sequential_backward(Ug, Vg, torch.from_numpy(G).to(gpu))
        torch.cuda.synchronize()
        assert rel_err(to_np(gU), gU_ref) <= FP32_TOL and rel_err(to_np(gV), gV_ref) <= FP32_TOL
    with pytest.raises(ValueError):
        das.affine_scan_block_reference(Ug, Vg, carry_scan="bogus")
    with pytest.raises(ValueError):
        das.affine_scan_block_reference(Ug, Vg, block_size=0)


def test_cfg4_dense_cayley_full_size(gpu):
    """H=8, d_h=32, B=1, L=16384, fp32, A_t = gate * Cayley(W_t),
    B_t = v k^T; output S_t for every step."""
    announce("cfg4 dense cayley full size")
    import mogt_amd

    U, V = synthetic.dense_cayley_inputs(1, 16384, 8, 32, seed=0)
    ref = so.affine_scan_sequential(U, V)
    S = mogt_amd.ops.affine_scan(torch.from_numpy(U).to(gpu), torch.from_numpy(V).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(S), ref) <= FP32_TOL


@pytest.mark.parametrize("B,L,R,C", [(2, 1000, 16, 48), (1, 777, 7, 11), (3, 300, 32, 32), (1, 64, 5, 130)])
@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_dense_scan_vk_equals_materialised(gpu, B, L, R, C, dt):
    """B_t = v_t k_t^T formed in registers: bit-identical to the scan of the
    materialised fp32 V = v k^T (same fp32 products, same MFMA sequence)."""
    announce(f"dense vk B={B} L={L} R={R} C={C} {dt}")
    import mogt_amd

    g = np.random.default_rng(B * 1000 + L + R + C)
    U = (np.eye(R, dtype=np.float32) * 0.95 + 0.03 * g.standard_normal((B, L, R, R), dtype=np.float32))
    v = g.standard_normal((B, L, R), dtype=np.float32)
    k = g.standard_normal((B, L, C), dtype=np.float32)
    Ut = torch.from_numpy(U).to(gpu)
    vt, kt = torch.from_numpy(v).to(gpu), torch.from_numpy(k).to(gpu)
    if dt == "bf16":
        vt, kt = vt.bfloat16(), kt.bfloat16()
    V = vt.float()[..., :, None] * kt.float()[..., None, :]
    for out in (torch.float32, torch.bfloat16):
        S = mogt_amd.dense_scan(Ut, v=vt, k=kt, output_dtype=out)
        S_ref = mogt_amd.ops.affine_scan(Ut, V.contiguous(), output_dtype=out)
        torch.cuda.synchronize()
        assert S.shape == (B, L, R, C) and S.dtype == out
        assert torch.equal(S, S_ref)
    ref = so.affine_scan_sequential(U, to_np(V))
    S32 = mogt_amd.dense_scan(Ut, v=vt, k=kt, output_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(to_np(S32), ref) <= FP32_TOL


def test_cfg4_dense_cayley_vk_full_size(gpu):
    """configs[3] with B_t = v_t k_t^T never materialised: bit-identical to the
    materialised-V scan (itself checked against the oracle above)."""
    announce("cfg4 dense cayley vk full size")
    import mogt_amd

    U, V, v, k = synthetic.dense_cayley_inputs(1, 16384, 8, 32, seed=0, return_vk=True)
    Ut = torch.from_numpy(U).to(gpu)
    S_vk = mogt_amd.dense_scan(Ut, v=torch.from_numpy(v).to(gpu), k=torch.from_numpy(k).to(gpu))
    S = mogt_amd.dense_scan(Ut, torch.from_numpy(V).to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(S_vk, S)


def test_dense_scan_argument_errors(gpu):
    import mogt_amd

    U = torch.zeros(1, 4, 3, 3, device=gpu)
    v = torch.zeros(1, 4, 3, device=gpu)
    k = torch.zeros(1, 4, 5, device=gpu)
    with pytest.raises(ValueError):
        mogt_amd.dense_scan(U)
    with pytest.raises(ValueError):
        mogt_amd.dense_scan(U, torch.zeros(1, 4, 3, 5, device=gpu), v=v, k=k)
    with pytest.raises(ValueError):
        mogt_amd.dense_scan(U, v=v)
    with pytest.raises(ValueError):
        mogt_amd.dense_scan(U, v=torch.zeros(1, 4, 2, device=gpu), k=k)


def test_zz_dense_no_lookback_wait_gave_up(gpu):
    from mogt_amd import ops

    assert ops.workspace_faults() == 0
