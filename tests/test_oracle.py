"""Pins of the CPU oracle (oracle/scan_oracle.py) against closed forms, library
routines, the reference's own relational checks and brute force.  Each pin is
chosen so that a plausible mistake (dropped term, off-by-one, transposed
operand, wrong fold order) fails; test_planted_mistakes_are_caught checks that
by planting such mistakes in a copy of the oracle."""
import numpy as np
import pytest
import scipy.signal
import torch

from conftest import rel_err
from mogt_amd import synthetic
from oracle import scan_oracle as so
from oracle import torch_ref


def _rand_affine(seed, B=2, L=23, R=4, C=3, scale=0.3):
    g = synthetic.rng(seed)
    U = np.eye(R) + scale * g.standard_normal((B, L, R, R))
    V = g.standard_normal((B, L, R, C))
    return U, V


def _closed_form_H(U, V):
    """H_t = sum_{s<=t} (U_t ... U_{s+1}) V_s, built independently of any scan."""
    B, L, R, C = V.shape
    H = np.zeros_like(V)
    for b in range(B):
        for t in range(L):
            acc = np.zeros((R, C))
            for s in range(t + 1):
                M = np.eye(R)
                for u in range(s + 1, t + 1):
                    M = U[b, u] @ M
                acc += M @ V[b, s]
            H[b, t] = acc
    return H


# --------------------------------------------------------------------------- dense scans
def test_sequential_matches_closed_form():
    U, V = _rand_affine(1, L=9)
    H = so.affine_scan_sequential(U, V)
    assert rel_err(H, _closed_form_H(U, V)) < 1e-12


def test_identity_transport_is_cumsum():
    B, L, R, C = 2, 31, 3, 5
    V = synthetic.rng(2).standard_normal((B, L, R, C))
    U = np.broadcast_to(np.eye(R), (B, L, R, R)).copy()
    assert rel_err(so.affine_scan_sequential(U, V), np.cumsum(V, axis=1)) < 1e-13


def test_constant_transport_prefix_is_matrix_power():
    R = 4
    g = synthetic.rng(3)
    M = np.eye(R) + 0.2 * g.standard_normal((R, R))
    L = 12
    U = np.broadcast_to(M, (1, L, R, R)).copy()
    V = g.standard_normal((1, L, R, 2))
    P, _ = so.affine_scan_sequential(U, V, return_prefix=True)
    for t in range(L):
        assert rel_err(P[0, t], np.linalg.matrix_power(M, t + 1)) < 1e-12


def test_reference_sanity_case_relations():
    """sanity_affine_scan.py:19-61: sequential == doubling == block(5, doubling), fp64, 1e-10."""
    Ut, Vt = synthetic.reference_test_case()
    U, V = Ut.numpy(), Vt.numpy()
    Ps, Hs = so.affine_scan_sequential(U, V, return_prefix=True)
    Pd, Hd = so.affine_scan_doubling(U, V, return_prefix=True)
    Pb, Hb = so.affine_scan_block_reference(U, V, block_size=5, carry_scan="doubling",
                                            return_prefix=True)
    for x, y in ((Ps, Pd), (Hs, Hd), (Ps, Pb), (Hs, Hb)):
        assert np.max(np.abs(x - y)) < 1e-10


@pytest.mark.parametrize("block", [1, 2, 5, 8, 23, 64])
@pytest.mark.parametrize("carry", ["sequential", "doubling"])
def test_block_reference_chunk_invariance(block, carry):
    U, V = _rand_affine(4, L=23)
    H = so.affine_scan_sequential(U, V)
    Hb = so.affine_scan_block_reference(U, V, block_size=block, carry_scan=carry)
    assert np.max(np.abs(H - Hb)) < 1e-10


def test_local_scan_matches_blockwise_sequential():
    U, V = _rand_affine(5, L=21)
    Up, Hp, Us, Hs = so.local_scan(U, V, block_size=8)
    for k, (s, e) in enumerate([(0, 8), (8, 16), (16, 21)]):
        P, H = so.affine_scan_sequential(U[:, s:e], V[:, s:e], return_prefix=True)
        assert np.max(np.abs(Up[:, s:e] - P)) < 1e-13
        assert np.max(np.abs(Hp[:, s:e] - H)) < 1e-13
        assert np.max(np.abs(Us[:, k] - P[:, -1])) < 1e-13
        assert np.max(np.abs(Hs[:, k] - H[:, -1])) < 1e-13


def test_fused_scan_is_prefix_product():
    U, V = _rand_affine(6, L=13)
    P, _ = so.affine_scan_sequential(U, V, return_prefix=True)
    assert np.max(np.abs(so.fused_scan(U) - P)) < 1e-13


def test_backward_matches_finite_differences_and_autograd():
    """sanity_affine_scan.py:102-135 checks the hand backward against autograd (fp64)."""
    Ut, Vt = synthetic.reference_test_case(seq_len=9)
    G = torch.randn_like(Vt)
    Ur = Ut.clone().requires_grad_(True)
    Vr = Vt.clone().requires_grad_(True)
    H = torch_ref.affine_scan_sequential_torch(Ur, Vr, state_dtype=torch.float64)
    gU_ref, gV_ref = torch.autograd.grad(H, (Ur, Vr), grad_outputs=G)
    gU, gV = so.affine_scan_sequential_backward(Ut.numpy(), Vt.numpy(), G.numpy())
    assert np.max(np.abs(gU - gU_ref.numpy())) < 1e-10
    assert np.max(np.abs(gV - gV_ref.numpy())) < 1e-10
    # independent finite-difference check of one U and one V entry
    U, V, Gn = Ut.numpy(), Vt.numpy(), G.numpy()
    eps = 1e-6
    for (arr, grad, idx) in ((U, gU, (1, 4, 2, 3)), (V, gV, (0, 6, 1, 2))):
        plus, minus = arr.copy(), arr.copy()
        plus[idx] += eps
        minus[idx] -= eps
        if arr is U:
            fp = np.sum(Gn * so.affine_scan_sequential(plus, V))
            fm = np.sum(Gn * so.affine_scan_sequential(minus, V))
        else:
            fp = np.sum(Gn * so.affine_scan_sequential(U, plus))
            fm = np.sum(Gn * so.affine_scan_sequential(U, minus))
        assert abs((fp - fm) / (2 * eps) - grad[idx]) < 1e-6


def test_validation_errors_match_reference():
    U, V = _rand_affine(7)
    with pytest.raises(ValueError):
        so.affine_scan_sequential(U[0], V)
    with pytest.raises(ValueError):
        so.affine_scan_sequential(U, V[:, :, :2])
    with pytest.raises(ValueError):
        so.affine_scan_block_reference(U, V, block_size=0)
    with pytest.raises(ValueError):
        so.affine_scan_block_reference(U, V, carry_scan="tree")


# --------------------------------------------------------------------------- diagonal scans
def test_diag_special_cases():
    g = synthetic.rng(8)
    b = g.standard_normal((2, 40, 6))
    assert rel_err(so.diag_scan(np.ones_like(b), b), np.cumsum(b, axis=1)) < 1e-13
    assert rel_err(so.diag_scan(np.zeros_like(b), b), b) < 1e-15
    assert np.all(so.diag_scan(g.random(b.shape), np.zeros_like(b)) == 0.0)


def test_diag_constant_decay_is_iir_filter():
    g = synthetic.rng(9)
    b = g.standard_normal((1, 300, 3))
    for alpha in (0.3, 0.9, 0.999):
        h = so.diag_scan(np.full_like(b, alpha), b)
        ref = scipy.signal.lfilter([1.0], [1.0, -alpha], b, axis=1)
        assert rel_err(h, ref) < 1e-12


def test_diag_brute_force_and_prefix():
    g = synthetic.rng(10)
    a = g.random((2, 11, 3))
    b = g.standard_normal((2, 11, 3))
    P, h = so.diag_scan(a, b, return_prefix=True)
    for t in range(11):
        ref = sum(np.prod(a[:, s + 1:t + 1], axis=1) * b[:, s] for s in range(t + 1))
        assert rel_err(h[:, t], ref) < 1e-13
        assert rel_err(P[:, t], np.prod(a[:, :t + 1], axis=1)) < 1e-13


def test_diag_equals_folded_affine_scan():
    a, b = synthetic.cfg1_inputs(seed=3)
    a, b = a[:, :64, :16], b[:, :64, :16]
    h = so.diag_scan(a, b)
    U, V = torch_ref.diag_as_affine(torch.from_numpy(a), torch.from_numpy(b))
    H = so.affine_scan_sequential(U.numpy(), V.numpy(), output_dtype=np.float64)
    H = torch_ref.unfold_affine(torch.from_numpy(H), 2, 16).numpy()
    assert rel_err(h, H) < 1e-13


def test_diag_linear_in_b():
    g = synthetic.rng(11)
    a = g.random((1, 50, 4))
    b1, b2 = g.standard_normal((2, 1, 50, 4))
    lhs = so.diag_scan(a, 2.0 * b1 - 3.0 * b2)
    rhs = 2.0 * so.diag_scan(a, b1) - 3.0 * so.diag_scan(a, b2)
    assert rel_err(lhs, rhs) < 1e-12


def test_torch_port_matches_numpy_oracle():
    a, b = synthetic.cfg1_inputs(seed=4)
    a, b = a[:, :128], b[:, :128]
    U, V = torch_ref.diag_as_affine(torch.from_numpy(a), torch.from_numpy(b))
    Hs = torch_ref.affine_scan_sequential_torch(U, V, state_dtype=torch.float64,
                                                output_dtype=torch.float64)
    Hd = torch_ref.affine_scan_doubling_torch(U, V, state_dtype=torch.float64,
                                              output_dtype=torch.float64)
    ref = so.diag_scan(a, b)
    assert rel_err(torch_ref.unfold_affine(Hs, 2, 128).numpy(), ref) < 1e-12
    assert rel_err(torch_ref.unfold_affine(Hd, 2, 128).numpy(), ref) < 1e-12


# --------------------------------------------------------------------------- coupled mixer scan
@pytest.mark.parametrize("bf16", [False, True])
def test_coupled_scan_equals_reference_U_V_construction(bf16):
    """model_mogt.py:91-102,166-182: U = I*damping*(1-g) (diag over ranks),
    V = V_raw * g; scan H = U H + V on [B, L, r, c]."""
    r, c, damping = 4, 6, 0.97
    z, v = synthetic.coupled_inputs(2, 30, r, c, seed=12)
    if bf16:
        v = so.round_bf16(v)
    h = so.coupled_rank_scan(z, v, r, damping=damping, v_is_bf16=bf16)
    g = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    U = np.eye(r)[None, None] * (damping * (1.0 - g))[..., None]
    gv = g[..., None].astype(np.float32)
    if bf16:
        Vm = so.round_bf16(v.reshape(2, 30, r, c) * so.round_bf16(gv))
    else:
        Vm = v.reshape(2, 30, r, c) * g[..., None]
    H = so.affine_scan_sequential(U, Vm.astype(np.float64))
    assert rel_err(h, H.reshape(2, 30, r * c)) < 1e-6


def test_round_bf16_known_values():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.140625, 1e-40, np.inf],
                 dtype=np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2 ** -6, -2.5, 3.140625, 0.0, np.inf], dtype=np.float32)
    got = so.round_bf16(x)
    assert np.isclose(got[5], 0.0, atol=1e-38)
    np.testing.assert_array_equal(np.delete(got, 5), np.delete(want, 5))
    assert torch.equal(torch.from_numpy(got[:5]),
                       torch.from_numpy(x[:5]).to(torch.bfloat16).float())


# --------------------------------------------------------------------------- rank-1 coupled
def test_rank1_coupled_matches_decayed_attention_bruteforce():
    f, k, v, q = synthetic.rank1_inputs(1, 13, 2, 5, seed=13)
    y = so.rank1_coupled_scan(f, k, v, q)
    f64 = f.astype(np.float64)
    k, v, q = (x.astype(np.float64) for x in (k, v, q))
    ref = np.zeros_like(y)
    for t in range(13):
        for s in range(t + 1):
            w = np.prod(f64[:, s + 1:t + 1], axis=1) * (1.0 - f64[:, s])   # [B, H]
            kq = np.sum(k[:, s] * q[:, t], axis=-1)                          # [B, H]
            ref[:, t] += (w * kq)[..., None] * v[:, s]
    assert rel_err(y, ref) < 1e-12


def test_rank1_coupled_equals_dense_affine_scan():
    f, k, v, q = synthetic.rank1_inputs(1, 9, 1, 4, seed=14)
    f, k, v, q = (x.astype(np.float64) for x in (f, k, v, q))
    d = 4
    U = f[0, :, 0, None, None] * np.eye(d)[None]
    V = (1.0 - f[0, :, 0, None, None]) * (v[0, :, 0, :, None] * k[0, :, 0, None, :])
    S = so.affine_scan_sequential(U[None].astype(np.float64), V[None].astype(np.float64))
    y = np.einsum("tij,tj->ti", S[0], q[0, :, 0])
    assert rel_err(so.rank1_coupled_scan(f, k, v, q)[0, :, 0], y) < 1e-12


# --------------------------------------------------------------------------- cayley
def test_cayley_is_orthogonal_and_solves():
    g = synthetic.rng(15)
    W = synthetic.skew_generators(5, 8, g=g).astype(np.float64)
    Q = so.cayley(W)
    for i in range(5):
        assert np.max(np.abs(Q[i].T @ Q[i] - np.eye(8))) < 1e-12
        assert np.max(np.abs((np.eye(8) - W[i]) @ Q[i] - (np.eye(8) + W[i]))) < 1e-12


# --------------------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught():
    """Plant plausible bugs in the oracle (on the CPU) and check a pin fails."""
    U, V = _rand_affine(16, L=9)
    ref = _closed_form_H(U, V)

    def seq_transposed(U, V):   # transposed transport operand
        return so.affine_scan_sequential(np.swapaxes(U, -1, -2), V)

    assert rel_err(seq_transposed(U, V), ref) > 1e-3

    def seq_off_by_one(U, V, **kw):   # state written before the update
        B, L, R, C = V.shape
        H = np.zeros((B, R, C))
        out = np.empty_like(V)
        for t in range(L):
            out[:, t] = H
            H = U[:, t] @ H + V[:, t]
        return out

    assert rel_err(seq_off_by_one(U, V), ref) > 1e-3

    def diag_dropped_term(a, b, **kw):   # forgets the decay of the carried state
        return np.cumsum(np.asarray(b, dtype=np.float64), axis=1)

    g = synthetic.rng(17)
    b = g.standard_normal((1, 60, 2))
    alpha = 0.9
    iir = scipy.signal.lfilter([1.0], [1.0, -alpha], b, axis=1)
    assert rel_err(diag_dropped_term(np.full_like(b, alpha), b), iir) > 1e-2

    def fold_wrong_order(U, V, block_size=5):   # carry applied as H_carry U_loc
        Up, Hp, Us, Hs = so.local_scan(U, V, block_size=block_size)
        out = Hp.copy()
        carry = np.zeros_like(Hs[:, 0])
        for k in range(Us.shape[1]):
            s, e = k * block_size, min((k + 1) * block_size, V.shape[1])
            out[:, s:e] = Hp[:, s:e] + np.swapaxes(Up[:, s:e], -1, -2) @ carry[:, None]
            carry = out[:, e - 1]
        return out

    assert rel_err(fold_wrong_order(U, V), ref) > 1e-3


# --------------------------------------------------------------------------- chunked tied-head CE
def _ce_case(seed, rows=37, vocab=53, ignore_every=0):
    g = synthetic.rng(seed)
    x = g.standard_normal((rows, vocab)) * 3.0
    lab = g.integers(0, vocab, size=rows)
    if ignore_every:
        lab[::ignore_every] = -100
    return x, lab


def test_ce_rows_match_torch_cross_entropy():
    from oracle import lm_loss_oracle as lo
    import torch.nn.functional as F

    for ignore_every in (0, 4):
        x, lab = _ce_case(31, ignore_every=ignore_every)
        loss, lse = lo.ce_rows(x, lab)
        xt = torch.from_numpy(x)
        ref = F.cross_entropy(xt, torch.from_numpy(lab), reduction="none").numpy()
        assert rel_err(loss, ref) <= 1e-12
        assert rel_err(lse, torch.logsumexp(xt, dim=1).numpy()) <= 1e-12
        # a per-row constant shift leaves the loss unchanged and moves lse with it
        loss2, lse2 = lo.ce_rows(x + 1000.0, lab)
        assert rel_err(loss2, loss) <= 1e-9 and rel_err(lse2 - 1000.0, lse) <= 1e-9


def test_ce_rows_grad_matches_autograd():
    from oracle import lm_loss_oracle as lo
    import torch.nn.functional as F

    x, lab = _ce_case(32, ignore_every=5)
    xt = torch.from_numpy(x).requires_grad_()
    (F.cross_entropy(xt, torch.from_numpy(lab), reduction="sum") * 0.37).backward()
    assert rel_err(lo.ce_rows_grad(x, lab, 0.37), xt.grad.numpy()) <= 1e-12


@pytest.mark.parametrize("chunk", [1, 7, 1000])
def test_chunked_linear_ce_matches_unchunked_autograd(chunk):
    from oracle import lm_loss_oracle as lo
    import torch.nn.functional as F

    g = synthetic.rng(33)
    B, L, D, V = 2, 9, 12, 29
    h = g.standard_normal((B, L, D))
    w = g.standard_normal((V, D)) * 0.5
    lab = g.integers(0, V, size=(B, L))
    lab[0, 3] = -100
    loss, gh, gw = lo.chunked_linear_ce(h, w, lab, chunk, grad_output=1.7)
    ht = torch.from_numpy(h).requires_grad_()
    wt = torch.from_numpy(w).requires_grad_()
    ref = F.cross_entropy((ht @ wt.t()).reshape(-1, V), torch.from_numpy(lab).reshape(-1),
                          reduction="sum") / (B * L)
    (ref * 1.7).backward()
    assert abs(loss - float(ref.detach())) <= 1e-12 * abs(float(ref.detach()))
    assert rel_err(gh, ht.grad.numpy()) <= 1e-12
    assert rel_err(gw, wt.grad.numpy()) <= 1e-12


def test_ce_planted_mistakes_are_caught():
    """Plausible slips in the CE restatement fail the library pins."""
    import torch.nn.functional as F

    x, lab = _ce_case(34)
    ref = F.cross_entropy(torch.from_numpy(x), torch.from_numpy(lab), reduction="none").numpy()
    no_max = np.log(np.exp(x).sum(1)) - x[np.arange(len(lab)), lab]   # fine in float64 ...
    assert rel_err(no_max, ref) <= 1e-9                                 # ... so the shift test matters:
    big = x + 1000.0
    with np.errstate(over="ignore", invalid="ignore"):
        no_max_big = np.log(np.exp(big).sum(1)) - big[np.arange(len(lab)), lab]
    assert not np.all(np.isfinite(no_max_big))
    wrong_pick = np.log(np.exp(x).sum(1)) - x[np.arange(len(lab)), (lab + 1) % x.shape[1]]
    assert rel_err(wrong_pick, ref) > 1e-2
