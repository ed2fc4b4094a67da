"""HIP-graph capture of the scan ops.

Each op is captured once into a ``torch.cuda.CUDAGraph`` (after warm-up on the
capture stream), then replayed several times on fresh inputs copied into the
captured buffers, with eager launches of the same op and host
synchronisations between replays.  Every replay must match the eager result
on the same inputs and the oracle.  This exercises the claims that the native
library allocates nothing and records no memset, and that the diagonal scan's
look-back workspace is reusable across launches without clearing (its epoch
advances inside the replayed kernel).
"""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from mogt_amd import synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_diag_scan_graph_replays(gpu):
    import mogt_amd

    B, L, D = 1, 4096, 768
    a0, b0 = synthetic.diag_inputs(B, L, D, seed=70)
    a = torch.from_numpy(a0).to(gpu)
    b = torch.from_numpy(b0).to(gpu)
    announce(f"graph diag B={B} L={L} D={D}: capture")
    g, out = _capture(lambda: mogt_amd.ops.diag_scan(a, b))
    for i in range(REPLAYS):
        an, bn = synthetic.diag_inputs(B, L, D, seed=71 + i)
        a.copy_(torch.from_numpy(an))
        b.copy_(torch.from_numpy(bn))
        announce(f"graph diag replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = mogt_amd.ops.diag_scan(a, b)
        torch.cuda.synchronize()
        assert rel_err(to_np(replayed), to_np(eager)) <= 1e-6
        assert rel_err(to_np(replayed), so.diag_scan(an, bn)) <= 1e-4
    assert mogt_amd.ops.workspace_faults() == 0


def test_coupled_scan_graph_replays(gpu):
    import mogt_amd

    B, L, r, c = 1, 3000, 16, 48
    z0, v0 = synthetic.coupled_inputs(B, L, r, c, seed=80)
    z = torch.from_numpy(z0).to(gpu)
    v = torch.from_numpy(v0).to(gpu).bfloat16()
    announce(f"graph coupled L={L} r={r} c={c}: capture")
    g, out = _capture(lambda: mogt_amd.coupled_rank_scan(z, v, damping=0.999))
    for i in range(REPLAYS):
        zn, vn = synthetic.coupled_inputs(B, L, r, c, seed=81 + i)
        z.copy_(torch.from_numpy(zn))
        v.copy_(torch.from_numpy(vn).bfloat16())
        announce(f"graph coupled replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = mogt_amd.coupled_rank_scan(z, v, damping=0.999)
        torch.cuda.synchronize()
        assert rel_err(to_np(replayed), to_np(eager)) <= 1e-6
        # bf16 V: the product V*g is rounded to bf16, so a last-bit difference of
        # the fp32 sigmoid can flip one rounding -> bf16 bar, exact bulk
        ref = so.coupled_rank_scan(zn, to_np(v), r, damping=0.999, v_is_bf16=True)
        err = np.abs(to_np(replayed).astype(np.float64) - ref) / np.max(np.abs(ref))
        assert float(err.max()) <= 2e-2
        assert float(np.median(err)) <= 1e-6
    assert mogt_amd.ops.workspace_faults() == 0


def test_dense_scan_graph_replays(gpu):
    import mogt_amd

    B, L, R, C = 1, 2000, 16, 48
    gen = np.random.default_rng(90)
    mk = lambda: (np.eye(R, dtype=np.float32) * 0.97 + 0.02 * gen.standard_normal((B, L, R, R), dtype=np.float32),
                  gen.standard_normal((B, L, R, C), dtype=np.float32))
    U0, V0 = mk()
    U = torch.from_numpy(U0).to(gpu)
    V = torch.from_numpy(V0).to(gpu)
    announce(f"graph dense L={L} R={R} C={C}: capture")
    g, out = _capture(lambda: mogt_amd.ops.affine_scan(U, V))
    for i in range(REPLAYS):
        Un, Vn = mk()
        U.copy_(torch.from_numpy(Un))
        V.copy_(torch.from_numpy(Vn))
        announce(f"graph dense replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = mogt_amd.ops.affine_scan(U, V)
        torch.cuda.synchronize()
        assert rel_err(to_np(replayed), to_np(eager)) <= 1e-6
        assert rel_err(to_np(replayed), so.affine_scan_sequential(Un, Vn)) <= 1e-4


def test_rank1_scan_graph_replays(gpu):
    import mogt_amd

    B, L, H = 1, 700, 2
    f0, k0, v0, q0 = synthetic.rank1_inputs(B, L, H, 64, seed=100)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f0, k0, v0, q0))
    announce(f"graph rank1 L={L} H={H}: capture")
    g, out = _capture(lambda: mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt))
    for i in range(REPLAYS):
        for dst, src in zip((ft, kt, vt, qt), synthetic.rank1_inputs(B, L, H, 64, seed=101 + i)):
            dst.copy_(torch.from_numpy(src).bfloat16())
        announce(f"graph rank1 replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt)
        torch.cuda.synchronize()
        assert rel_err(to_np(replayed), to_np(eager)) <= 1e-6
        ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
        assert rel_err(to_np(replayed), ref) <= 2e-2


def test_generic_scan_graph_replays(gpu):
    """The generic scan (float64 state, R = 40, prefix product, three passes)
    under capture: its workspace needs no clearing, so replays match eager
    launches exactly."""
    import mogt_amd

    B, L, R, C = 2, 600, 40, 5
    gen = np.random.default_rng(95)
    mk = lambda: (np.eye(R) * 0.95 + (0.2 / np.sqrt(R)) * gen.standard_normal((B, L, R, R)),
                  gen.standard_normal((B, L, R, C)))
    U0, V0 = mk()
    U = torch.from_numpy(U0).to(gpu)
    V = torch.from_numpy(V0).to(gpu)
    announce(f"graph generic fp64 L={L} R={R} C={C}: capture")
    g, out = _capture(lambda: mogt_amd.ops.affine_scan(U, V, state_dtype=torch.float64, return_prefix=True))
    for i in range(REPLAYS):
        Un, Vn = mk()
        U.copy_(torch.from_numpy(Un))
        V.copy_(torch.from_numpy(Vn))
        announce(f"graph generic replay {i}")
        g.replay()
        torch.cuda.synchronize()
        P_rep, H_rep = out[0].clone(), out[1].clone()
        P_eag, H_eag = mogt_amd.ops.affine_scan(U, V, state_dtype=torch.float64, return_prefix=True)
        torch.cuda.synchronize()
        assert torch.equal(P_rep, P_eag) and torch.equal(H_rep, H_eag)
        P_ref, H_ref = so.affine_scan_sequential(Un, Vn, return_prefix=True)
        assert rel_err(H_rep.cpu().numpy(), H_ref) <= 1e-12
        assert rel_err(P_rep.cpu().numpy(), P_ref) <= 1e-12


def test_diag_scan_graph_of_chained_calls(gpu):
    """Three dependent scans captured in one graph (each later scan reads the
    previous output), so consecutive launches inside one replay share the
    look-back workspace; every replay matches the same chain run eagerly."""
    import mogt_amd

    B, L, D = 1, 8192, 768
    a0, b0 = synthetic.diag_inputs(B, L, D, seed=80)
    a = torch.from_numpy(a0).to(gpu)
    b = torch.from_numpy(b0).to(gpu)
    a2 = torch.flip(a, dims=[1]).contiguous()

    def chain():
        h1 = mogt_amd.ops.diag_scan(a, b)
        h2 = mogt_amd.ops.diag_scan(a2, h1)
        return mogt_amd.ops.diag_scan(a, h2)

    announce(f"graph diag chain B={B} L={L} D={D}: capture")
    g, out = _capture(chain)
    for i in range(REPLAYS):
        an, bn = synthetic.diag_inputs(B, L, D, seed=81 + i)
        a.copy_(torch.from_numpy(an))
        b.copy_(torch.from_numpy(bn))
        a2.copy_(torch.flip(a, dims=[1]))
        announce(f"graph diag chain replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = chain()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        ref = so.diag_scan(an, so.diag_scan(np.ascontiguousarray(an[:, ::-1]), so.diag_scan(an, bn)))
        assert rel_err(to_np(replayed), ref) <= 1e-4
    assert mogt_amd.ops.workspace_faults() == 0


def test_linear_wgrad_graph_replays(gpu):
    """The split-K weight-gradient GEMM (its partial-sum workspace and both
    launches) under capture: replays match eager launches bit for bit."""
    from mogt_amd import ops

    T, O, I = 8192, 768, 800
    gen = torch.Generator(device="cpu").manual_seed(90)
    mk = lambda: (torch.randn(T, O, generator=gen).bfloat16(), torch.randn(T, I, generator=gen).bfloat16())
    dy0, x0 = mk()
    dy, x = dy0.to(gpu), x0.to(gpu)
    announce(f"graph linear_wgrad T={T} O={O} I={I}: capture")
    g, out = _capture(lambda: ops.linear_wgrad(dy, x))
    for i in range(REPLAYS):
        dyn, xn = mk()
        dy.copy_(dyn)
        x.copy_(xn)
        announce(f"graph linear_wgrad replay {i}")
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = ops.linear_wgrad(dy, x)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        ref = dy.double().t() @ x.double()
        assert rel_err(to_np(replayed), to_np(ref)) <= 2e-2
