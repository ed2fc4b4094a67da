"""GPU backward of the diagonal and coupled scans (the reverse-time HIP scan
behind ``torch.library.register_autograd``) against the float64 oracle.

The diagonal case is checked against ``affine_scan_sequential_backward``
(affine_scan.py:65-124 restated) in the folded R = C = 1 mapping, including a
full-size L = 32768 run; the coupled mixer scan against ``torch.autograd`` of a
float64 CPU restatement of the same recurrence (model_mogt.py:166-182 with the
identity connection), the reference's own way of checking its backward
(sanity_affine_scan.py:102-135).  Bars: fp32 <= 1e-4, bf16 inputs <= 2e-2.
"""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from mogt_amd import synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _fold(x):
    """[B, L, D] -> [B*D, L, 1, 1] (the reference's per-feature mapping)."""
    B, L, D = x.shape
    return np.ascontiguousarray(np.transpose(x, (0, 2, 1)).reshape(B * D, L, 1, 1))


def _unfold(x, B, D):
    BD, L = x.shape[:2]
    return np.transpose(x.reshape(B, D, L), (0, 2, 1))


def _diag_oracle_grads(a, b, w):
    B, L, D = a.shape
    gU, gV = so.affine_scan_sequential_backward(_fold(a.astype(np.float64)), _fold(b.astype(np.float64)),
                                                _fold(w.astype(np.float64)))
    return _unfold(gU, B, D), _unfold(gV, B, D)


@pytest.mark.parametrize("B,L,D", [(2, 300, 64), (1, 1, 8), (1, 2049, 768), (3, 77, 10)])
def test_diag_scan_backward_fp32(gpu, B, L, D):
    announce(f"diag backward fp32 B={B} L={L} D={D}")
    import mogt_amd

    a, b = synthetic.diag_inputs(B, L, D, seed=L + D)
    w = np.random.default_rng(L).standard_normal((B, L, D)).astype(np.float32)
    at = torch.from_numpy(a).to(gpu).requires_grad_()
    bt = torch.from_numpy(b).to(gpu).requires_grad_()
    h = mogt_amd.diag_scan(at, bt)
    (h * torch.from_numpy(w).to(gpu)).sum().backward()
    torch.cuda.synchronize()
    da_ref, db_ref = _diag_oracle_grads(a, b, w)
    assert rel_err(to_np(bt.grad), db_ref) <= FP32_TOL
    assert rel_err(to_np(at.grad), da_ref) <= FP32_TOL


def test_diag_scan_backward_bf16(gpu):
    announce("diag backward bf16 B=1 L=1000 D=256")
    import mogt_amd

    a, b = synthetic.diag_inputs(1, 1000, 256, seed=5)
    w = np.random.default_rng(6).standard_normal((1, 1000, 256)).astype(np.float32)
    at = torch.from_numpy(a).to(gpu).bfloat16().requires_grad_()
    bt = torch.from_numpy(b).to(gpu).bfloat16().requires_grad_()
    h = mogt_amd.diag_scan(at, bt, out_dtype=torch.float32)
    (h * torch.from_numpy(w).to(gpu)).sum().backward()
    torch.cuda.synchronize()
    assert at.grad.dtype == torch.bfloat16 and bt.grad.dtype == torch.bfloat16
    da_ref, db_ref = _diag_oracle_grads(to_np(at.detach()), to_np(bt.detach()), w)
    assert rel_err(to_np(bt.grad), db_ref) <= BF16_TOL
    assert rel_err(to_np(at.grad), da_ref) <= BF16_TOL


@pytest.mark.parametrize("L", [16384, 32768])
def test_diag_scan_backward_full_size(gpu, L):
    """configs[1] shapes (B=1, D=768, L=16384 and 32768, which take different
    default tiles), fp32."""
    announce(f"diag backward full size L={L}")
    import mogt_amd

    a, b = synthetic.cfg2_inputs(L, seed=9)
    w = np.random.default_rng(10).standard_normal(a.shape).astype(np.float32)
    at = torch.from_numpy(a).to(gpu).requires_grad_()
    bt = torch.from_numpy(b).to(gpu).requires_grad_()
    h = mogt_amd.diag_scan(at, bt)
    (h * torch.from_numpy(w).to(gpu)).sum().backward()
    torch.cuda.synchronize()
    da_ref, db_ref = _diag_oracle_grads(a, b, w)
    assert rel_err(to_np(bt.grad), db_ref) <= FP32_TOL
    assert rel_err(to_np(at.grad), da_ref) <= FP32_TOL


def _coupled_ref(z, v, r, damping):
    """float64 CPU restatement with autograd: g = sigmoid(z), a = damping (1 - g)
    per rank, h_t = a_t h_{t-1} + v_t g_t (model_mogt.py:166-182, identity U)."""
    B, L, D = v.shape
    c = D // r
    g = torch.sigmoid(z)
    a = damping * (1.0 - g)
    vv = v.view(B, L, r, c) * g.unsqueeze(-1)
    h = torch.zeros(B, r, c, dtype=v.dtype)
    out = []
    for t in range(L):
        h = a[:, t, :, None] * h + vv[:, t]
        out.append(h)
    return torch.stack(out, 1).reshape(B, L, D)


@pytest.mark.parametrize("L,r,c,vdt", [(200, 4, 6, "fp32"), (513, 16, 48, "fp32"), (300, 16, 48, "bf16"),
                                        (150, 3, 5, "fp32")])
def test_coupled_scan_backward(gpu, L, r, c, vdt):
    announce(f"coupled backward L={L} r={r} c={c} v={vdt}")
    import mogt_amd

    z, v = synthetic.coupled_inputs(1, L, r, c, seed=L + r)
    w = np.random.default_rng(L).standard_normal((1, L, r * c)).astype(np.float32)
    zt = torch.from_numpy(z).to(gpu).requires_grad_()
    vt = torch.from_numpy(v).to(gpu)
    if vdt == "bf16":
        vt = vt.bfloat16()
    vt.requires_grad_()
    h = mogt_amd.coupled_rank_scan(zt, vt, damping=0.999)
    (h * torch.from_numpy(w).to(gpu)).sum().backward()
    torch.cuda.synchronize()

    z64 = torch.from_numpy(z).double().requires_grad_()
    v64 = torch.from_numpy(to_np(vt.detach())).double().requires_grad_()
    (_coupled_ref(z64, v64, r, 0.999) * torch.from_numpy(w).double()).sum().backward()
    tol = FP32_TOL if vdt == "fp32" else BF16_TOL
    assert vt.grad.dtype == vt.dtype
    assert rel_err(to_np(vt.grad), v64.grad.numpy()) <= tol
    assert rel_err(to_np(zt.grad), z64.grad.numpy()) <= tol


def _coupled_rev64(z, dh, r, damping):
    """float64 reverse recurrence G_t = dh_t + a_{t+1} G_{t+1}, G_L = 0, with
    a = damping (1 - sigmoid(z)) per rank (triton_scan.py:359-426 for the
    diagonal U of the coupled identity connection)."""
    B, L, D = dh.shape
    c = D // r
    a = np.repeat(damping * (1.0 - 1.0 / (1.0 + np.exp(-z.astype(np.float64)))), c, axis=2)
    G = np.zeros((B, L, D))
    acc = np.zeros((B, D))
    for t in range(L - 1, -1, -1):
        acc = dh[:, t].astype(np.float64) + (a[:, t + 1] * acc if t + 1 < L else 0.0)
        G[:, t] = acc
    return G


@pytest.mark.parametrize("B,L,r,c,zdt", [(2, 300, 4, 6, "fp32"), (1, 1, 16, 48, "fp32"), (1, 2049, 16, 48, "bf16"),
                                         (2, 77, 3, 5, "fp32"), (1, 16384, 16, 48, "fp32"),
                                         (1, 32768, 16, 48, "fp32")])
def test_coupled_reverse_scan(gpu, B, L, r, c, zdt):
    """The coupled reverse scan (decay formed from the gate logits inside the
    scan) against the float64 recurrence; odd channel counts take the
    one-feature-per-lane tiles."""
    announce(f"coupled reverse scan B={B} L={L} r={r} c={c} z={zdt}")
    from mogt_amd import ops  # noqa: F401  (registers the ops)

    rng = np.random.default_rng(L + c)
    z = (rng.standard_normal((B, L, r)) * 2).astype(np.float32)
    dh = rng.standard_normal((B, L, r * c)).astype(np.float32)
    zt = torch.from_numpy(z).to(gpu)
    if zdt == "bf16":
        zt = zt.bfloat16()
    G = torch.ops.mogt.coupled_scan_rev(zt, torch.from_numpy(dh).to(gpu), r, 0.995)
    torch.cuda.synchronize()
    ref = _coupled_rev64(to_np(zt).astype(np.float64), dh, r, 0.995)
    assert G.dtype == torch.float32 and G.shape == (B, L, r * c)
    assert rel_err(to_np(G), ref) <= FP32_TOL


TILES_COUPLED_REV = [(2, 32, 32, 8), (2, 32, 32, 4), (2, 32, 16, 8), (2, 32, 8, 16), (4, 16, 16, 8), (4, 16, 8, 16),
                     (4, 16, 8, 8), (1, 64, 32, 16), (1, 64, 16, 16), (1, 64, 8, 16)]


@pytest.mark.parametrize("tile", TILES_COUPLED_REV)
def test_every_coupled_reverse_tile(gpu, tile):
    """Every compiled tile of the coupled reverse scan through its tile-override
    entry point: ragged L, two sequences, 48 channels per gate (divisible by
    every vector width), bf16 logits for the vector-4 tiles."""
    announce(f"coupled reverse tile {tile}")
    from mogt_amd import _lib, ops

    B, L, r, c = 2, 2777, 4, 48
    rng = np.random.default_rng(sum(tile))
    z = (rng.standard_normal((B, L, r)) * 2).astype(np.float32)
    dh = rng.standard_normal((B, L, r * c)).astype(np.float32)
    zt = torch.from_numpy(z).to(gpu)
    if tile[0] == 4:
        zt = zt.bfloat16()
    dht = torch.from_numpy(dh).to(gpu)
    G = torch.empty_like(dht)
    lib = _lib.load()
    ws = ops.workspace(lib.mogt_diag_scan_workspace_bytes_cfg(B, L, r * c, *tile), gpu, "coupled_rev",
                       ("cfg-test", B, L, r, c, tile))
    rc = lib.mogt_coupled_rank_scan_rev_fwd_cfg(zt.data_ptr(), dht.data_ptr(), G.data_ptr(), B, L, r, c, 0.995,
                                                ops.dtype_code(zt.dtype, "z"), *tile, ws.data_ptr(), ws.numel(),
                                                ops._stream_handle(gpu))
    _lib.check(rc, "mogt_coupled_rank_scan_rev_fwd_cfg")
    torch.cuda.synchronize()
    ref = _coupled_rev64(to_np(zt).astype(np.float64), dh, r, 0.995)
    assert rel_err(to_np(G), ref) <= FP32_TOL
    assert ops.workspace_faults() == 0


@pytest.mark.parametrize("B,L,r,c,dt,prev,with_const", [(2, 200, 4, 8, "fp32", True, True),
                                                        (1, 300, 16, 48, "fp32", True, True),
                                                        (2, 150, 4, 12, "fp32", False, False),
                                                        (1, 256, 16, 48, "bf16", True, True)])
def test_projection_fed_scan_gradients(gpu, B, L, r, c, dt, prev, with_const):
    """The differentiable projection-fed coupled scan (the training mixer):
    gradients of the projection -- v columns, current-token gate columns and
    the previous-token gate columns (shifted by one step) -- and of the
    per-sequence logit term, against float64 autograd of z = P[t][D+i] +
    P[t-1][D+r+i] + const, g = sigmoid(z), h_t = d (1-g) h_{t-1} + v g."""
    announce(f"projection-fed scan gradients B={B} L={L} r={r} c={c} {dt} prev={prev}")
    from mogt_amd import ops

    D = r * c
    ld = D + r * (2 if prev else 1)
    g = torch.Generator().manual_seed(L + c)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    proj = torch.randn(B, L, ld, generator=g)
    proj[..., D:] = proj[..., D:] - 0.5
    proj = proj.to(tdt)
    gc = (torch.randn(B, r, generator=g) - 1.0) if with_const else None
    w = torch.randn(B, L, D, generator=g)
    pt = proj.to(gpu).requires_grad_()
    gct = gc.to(gpu).requires_grad_() if gc is not None else None
    h = ops.coupled_proj_scan(pt, D, rank=r, gate_prev=prev, gate_const=gct, damping=0.99)
    (h * w.to(gpu)).sum().backward()
    torch.cuda.synchronize()
    p64 = proj.double().requires_grad_()
    g64 = gc.double().requires_grad_() if gc is not None else None
    z = p64[..., D:D + r]
    if prev:
        z = torch.cat([z[:, :1], z[:, 1:] + p64[:, :-1, D + r:D + 2 * r]], dim=1)
    if g64 is not None:
        z = z + g64[:, None, :]
    gate = torch.sigmoid(z)
    # the gate as multiplied into bf16 v (the cast passes gradients through)
    gio = gate.to(tdt).double() if dt == "bf16" else gate
    a = (0.99 * (1.0 - gate)).repeat_interleave(c, dim=-1)
    bv = p64[..., :D] * gio.repeat_interleave(c, dim=-1)
    hh = torch.zeros(B, D, dtype=torch.float64)
    outs = []
    for t in range(L):
        hh = a[:, t] * hh + bv[:, t]
        outs.append(hh)
    ref = (torch.stack(outs, 1) * w.double()).sum()
    ref.backward()
    tol = FP32_TOL if dt == "fp32" else BF16_TOL
    assert rel_err(to_np(h), torch.stack(outs, 1).detach().numpy()) <= tol
    gp = to_np(pt.grad)
    assert rel_err(gp[..., :D], p64.grad[..., :D].numpy()) <= tol
    assert rel_err(gp[..., D:], p64.grad[..., D:].numpy()) <= tol
    if prev:
        assert np.all(gp[:, -1, D + r:] == 0)
    if gc is not None:
        assert rel_err(to_np(gct.grad), g64.grad.numpy()) <= tol
