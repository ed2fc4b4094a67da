"""GPU parity of the single-pass diagonal scan and the coupled mixer scan
against the CPU oracle on identical seeded inputs.

Bars (normwise max relative error, float64): fp32 I/O <= 1e-4; bf16 I/O with
fp32 state <= 2e-2.  Full-size (L = 32768) runs are checked against the oracle
too (it takes < 1 s per case at D = 768) plus size-independent properties.
"""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from mogt_amd import _lib, synthetic
from oracle import scan_oracle as so

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2

# every compiled tile (vec, lanes per row, steps per lane, waves); the CPU test
# test_capi.py::test_gpu_tile_lists_match_library keeps these in step
TILES_F32 = [(2, 32, 32, 8), (2, 32, 16, 16), (2, 32, 16, 8), (2, 32, 32, 4), (2, 32, 8, 16),
             (1, 64, 32, 16), (1, 64, 16, 16), (1, 64, 8, 16)]
TILES_BF16 = [(4, 16, 16, 8), (4, 16, 16, 16), (4, 16, 8, 8), (4, 32, 16, 8), (2, 32, 16, 8),
              (2, 32, 16, 16), (2, 32, 8, 16), (1, 64, 32, 16), (1, 64, 16, 16), (1, 64, 8, 16)]
TILES_COUPLED = [(4, 16, 8, 16), (4, 16, 8, 8), (4, 16, 16, 8), (4, 16, 16, 16), (4, 32, 8, 16), (2, 32, 16, 8),
                 (2, 32, 16, 16), (2, 32, 8, 16), (1, 64, 32, 16), (1, 64, 16, 16), (1, 64, 8, 16)]


def _run_cfg(a, b, out_dtype, cfg, prefix=False):
    from mogt_amd import ops

    h = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    p = torch.empty(a.shape, dtype=out_dtype, device=a.device) if prefix else None
    ops._diag_scan_launch(a.contiguous(), b.contiguous(), h, p, cfg)
    return (p, h) if prefix else h


def test_cfg1_fp32(gpu):
    announce("diag cfg1 B=2 L=512 D=128 fp32")
    import mogt_amd

    a, b = synthetic.cfg1_inputs(seed=0)
    ref = so.diag_scan(a, b)
    h = mogt_amd.diag_scan(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    torch.cuda.synchronize()
    assert h.dtype == torch.float32
    assert rel_err(to_np(h), ref) <= FP32_TOL


@pytest.mark.parametrize("dt,tile", [("fp32", t) for t in TILES_F32] + [("bf16", t) for t in TILES_BF16])
def test_every_tile_ragged(gpu, tile, dt):
    """Ragged L (not a multiple of any chunk), several chunks per chain, D a
    multiple of the vector but not of the feature-group width; with prefix."""
    announce(f"diag tile {tile} {dt} B=3 L=4237 D=320")
    a, b = synthetic.diag_inputs(3, 4237, 320, a_mean=2.0, b_std=1.0, seed=5)
    at, bt = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    if dt == "bf16":
        at, bt = at.bfloat16(), bt.bfloat16()
        a, b = to_np(at), to_np(bt)
    P_ref, ref = so.diag_scan(a, b, return_prefix=True)
    p, h = _run_cfg(at, bt, torch.float32, tile, prefix=True)
    torch.cuda.synchronize()
    assert rel_err(to_np(h), ref) <= FP32_TOL
    assert rel_err(to_np(p), P_ref) <= FP32_TOL


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 4097])
def test_edge_lengths(gpu, L):
    announce(f"diag edge L={L}")
    import mogt_amd

    a, b = synthetic.diag_inputs(2, L, 40, a_mean=1.0, b_std=1.0, seed=L)
    h = mogt_amd.diag_scan(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(h), so.diag_scan(a, b)) <= FP32_TOL


def test_odd_feature_count_uses_scalar_tile(gpu):
    announce("diag D=131 (odd)")
    import mogt_amd

    a, b = synthetic.diag_inputs(1, 777, 131, seed=2)
    h = mogt_amd.diag_scan(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(h), so.diag_scan(a, b)) <= FP32_TOL


def test_empty_input(gpu):
    import mogt_amd

    a = torch.empty(1, 0, 8, device=gpu)
    assert mogt_amd.diag_scan(a, a).shape == (1, 0, 8)


def test_special_cases_cumsum_and_identity(gpu):
    """a = 1 -> cumsum(b) (long chains of unit decay through every chunk);
    a = 0 -> h = b."""
    announce("diag a=1 / a=0 L=20000 D=64")
    import mogt_amd

    g = synthetic.rng(3)
    b = g.standard_normal((1, 20000, 64)).astype(np.float32)
    bt = torch.from_numpy(b).to(gpu)
    h1 = mogt_amd.diag_scan(torch.ones_like(bt), bt)
    h0 = mogt_amd.diag_scan(torch.zeros_like(bt), bt)
    torch.cuda.synchronize()
    assert rel_err(to_np(h1), np.cumsum(b.astype(np.float64), axis=1)) <= FP32_TOL
    assert np.array_equal(to_np(h0), b)


@pytest.mark.parametrize("L", [8192, 16384, 32768])
def test_cfg2_fp32_full_size(gpu, L):
    announce(f"diag cfg2 fp32 L={L}")
    import mogt_amd

    a, b = synthetic.cfg2_inputs(L, seed=1)
    ref = so.diag_scan(a, b)
    h = mogt_amd.diag_scan(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    torch.cuda.synchronize()
    assert rel_err(to_np(h), ref) <= FP32_TOL


@pytest.mark.parametrize("L", [8192, 16384, 32768])
def test_cfg2_bf16_io_full_size(gpu, L):
    announce(f"diag cfg2 bf16 L={L}")
    import mogt_amd

    a, b = synthetic.cfg2_inputs(L, seed=2)
    at = torch.from_numpy(a).to(gpu).bfloat16()
    bt = torch.from_numpy(b).to(gpu).bfloat16()
    ref = so.diag_scan(to_np(at), to_np(bt))   # oracle sees the same bf16-rounded inputs
    h = mogt_amd.diag_scan(at, bt)
    torch.cuda.synchronize()
    assert h.dtype == torch.bfloat16
    assert rel_err(to_np(h), ref) <= BF16_TOL
    hf = mogt_amd.diag_scan(at, bt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(to_np(hf), ref) <= FP32_TOL   # fp32 state: only input rounding differs


def test_repeated_launches_reuse_workspace(gpu):
    """The workspace is only zeroed once; 50 back-to-back launches of different
    shapes must all stay exact (epoch/ticket reset at the end of every launch)."""
    announce("diag workspace reuse x50")
    import mogt_amd

    cases = []
    for i, (L, D) in enumerate([(3000, 768), (515, 64), (8192, 256), (77, 1024)]):
        a, b = synthetic.diag_inputs(1, L, D, seed=10 + i)
        cases.append((torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu),
                      so.diag_scan(a, b)))
    outs = []
    for it in range(50):
        at, bt, ref = cases[it % len(cases)]
        outs.append((mogt_amd.diag_scan(at, bt), ref))
    torch.cuda.synchronize()
    for h, ref in outs:
        assert rel_err(to_np(h), ref) <= FP32_TOL


def test_linearity_at_full_size(gpu):
    """Size-independent property at L = 32768: scan(a, 2b1 - 3b2) = 2scan(a,b1) - 3scan(a,b2)."""
    announce("diag linearity L=32768")
    import mogt_amd

    a, b1 = synthetic.cfg2_inputs(32768, seed=7)
    _, b2 = synthetic.cfg2_inputs(32768, seed=8)
    at = torch.from_numpy(a).to(gpu)
    t1, t2 = torch.from_numpy(b1).to(gpu), torch.from_numpy(b2).to(gpu)
    lhs = mogt_amd.diag_scan(at, 2 * t1 - 3 * t2)
    rhs = 2 * mogt_amd.diag_scan(at, t1) - 3 * mogt_amd.diag_scan(at, t2)
    torch.cuda.synchronize()
    assert rel_err(to_np(lhs), to_np(rhs).astype(np.float64)) <= FP32_TOL


# --------------------------------------------------------------------------- coupled mixer scan
@pytest.mark.parametrize("L,r,c", [(300, 4, 6), (4096, 16, 48), (32768, 16, 48)])
@pytest.mark.parametrize("vdt", ["fp32", "bf16"])
def test_coupled_rank_scan(gpu, L, r, c, vdt):
    announce(f"coupled L={L} r={r} c={c} v={vdt}")
    import mogt_amd

    z, v = synthetic.coupled_inputs(1, L, r, c, seed=L + r)
    zt = torch.from_numpy(z).to(gpu)
    vt = torch.from_numpy(v).to(gpu)
    if vdt == "bf16":
        vt = vt.bfloat16()
    ref = so.coupled_rank_scan(z, to_np(vt), r, damping=0.999, v_is_bf16=(vdt == "bf16"))
    h = mogt_amd.coupled_rank_scan(zt, vt, damping=0.999)
    torch.cuda.synchronize()
    assert h.shape == (1, L, r * c) and h.dtype == torch.float32
    # bf16 V: the product V*g is rounded to bf16 (model_mogt.py:180), so a
    # last-bit difference of the fp32 sigmoid can flip one rounding -> bf16 bar.
    tol = FP32_TOL if vdt == "fp32" else BF16_TOL
    err = np.abs(to_np(h).astype(np.float64) - ref) / np.max(np.abs(ref))
    assert float(err.max()) <= tol
    assert float(np.median(err)) <= 1e-6   # the bulk is exact to fp32 accumulation


@pytest.mark.parametrize("B,L,r,c,vdt,odt", [(2, 1000, 16, 48, "bf16", "bf16"), (1, 32768, 16, 48, "bf16", "bf16"),
                                              (1, 300, 4, 8, "fp32", "fp32"), (2, 517, 4, 24, "bf16", "fp32"),
                                              (1, 77, 3, 20, "fp32", "bf16")])
def test_coupled_rank_scan_row_statistics(gpu, B, L, r, c, vdt, odt):
    """The statistics variant: the same h (in out_dtype), and per row and group
    of 64 features the sum of squares of the fp32 state (groups past D hold
    fewer features); against the oracle's float64 h."""
    announce(f"coupled scan statistics B={B} L={L} r={r} c={c} v={vdt} out={odt}")
    from mogt_amd import ops

    z, v = synthetic.coupled_inputs(B, L, r, c, seed=L + r)
    zt = torch.from_numpy(z).to(gpu)
    vt = torch.from_numpy(v).to(gpu)
    if vdt == "bf16":
        vt = vt.bfloat16()
    odt_t = torch.bfloat16 if odt == "bf16" else torch.float32
    h, stats = ops.coupled_rank_scan_stats(zt, vt, damping=0.997, out_dtype=odt_t)
    h32 = ops.coupled_rank_scan(zt, vt, damping=0.997, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = so.coupled_rank_scan(z, to_np(vt), r, damping=0.997, v_is_bf16=vdt == "bf16")
    D = r * c
    G = -(-D // 64)
    assert h.dtype == odt_t and stats.shape == (B, L, G)
    # the scan against the oracle (bf16 v: a last-bit difference of the fp32
    # sigmoid can flip the bf16 rounding of v * g -> bf16 bar, exact bulk)
    err = np.abs(to_np(h32).astype(np.float64) - ref) / np.max(np.abs(ref))
    assert float(err.max()) <= (BF16_TOL if vdt == "bf16" else FP32_TOL)
    assert float(np.median(err)) <= 1e-6
    # the statistics variant against the same arithmetic without statistics
    h64 = to_np(h32).astype(np.float64)
    assert rel_err(to_np(h), h64) <= (2.0 ** -8 if odt == "bf16" else 1e-6)
    pad = np.zeros((B, L, G * 64))
    pad[..., :D] = h64
    ref_stats = (pad.reshape(B, L, G, 64) ** 2).sum(-1)
    assert rel_err(to_np(stats), ref_stats) <= 1e-5


@pytest.mark.parametrize("B,L,r,c,dt,prev,const", [(2, 1000, 16, 48, "bf16", True, "batch"),
                                                   (1, 32768, 16, 48, "bf16", True, "batch"),
                                                   (1, 300, 4, 24, "fp32", False, None),
                                                   (2, 77, 3, 20, "fp32", False, "rank"),
                                                   (1, 129, 4, 8, "bf16", True, None)])
def test_coupled_rank_scan_projection_fed(gpu, B, L, r, c, dt, prev, const):
    """The scan fed by one projection row [v | gate pre-logits (current) |
    (previous)]: against the statistics scan on logits assembled by torch from
    the same projection, and against the oracle.  Row strides not a multiple of
    the vector fall back to narrower tiles."""
    announce(f"coupled scan projection-fed B={B} L={L} r={r} c={c} {dt} prev={prev} const={const}")
    from mogt_amd import ops

    D = r * c
    ld = D + r * (2 if prev else 1)
    g = torch.Generator().manual_seed(L + r)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    proj = torch.randn(B, L, ld, generator=g)
    proj[..., D:] = proj[..., D:] * 1.5 - 1.0
    proj = proj.to(tdt).to(gpu)
    gc = None
    if const == "batch":
        gc = (torch.randn(B, r, generator=g) - 1.0).to(gpu)
    elif const == "rank":
        gc = (torch.randn(r, generator=g) - 1.0).to(gpu)
    h, stats = ops.coupled_rank_scan_proj(proj, D, rank=r, gate_prev=prev, gate_const=gc, damping=0.995)
    z = proj[..., D:D + r].float()
    if prev:
        z = torch.cat([z[:, :1], z[:, 1:] + proj[:, :-1, D + r:D + 2 * r].float()], dim=1)
    if gc is not None:
        z = z + gc.expand(B, r)[:, None, :]
    v = proj[..., :D]
    h2, stats2 = ops.coupled_rank_scan_stats(z.contiguous(), v.contiguous(), damping=0.995, out_dtype=tdt)
    torch.cuda.synchronize()
    assert h.shape == (B, L, D) and h.dtype == tdt
    assert rel_err(to_np(h), to_np(h2)) <= (2.0 ** -8 if dt == "bf16" else 1e-6)
    assert rel_err(to_np(stats), to_np(stats2)) <= 1e-5
    ref = so.coupled_rank_scan(to_np(z), to_np(v), r, damping=0.995, v_is_bf16=dt == "bf16")
    err = np.abs(to_np(h).astype(np.float64) - ref) / np.max(np.abs(ref))
    assert float(err.max()) <= (BF16_TOL if dt == "bf16" else FP32_TOL)
    # the training form returns the logits it assembled: the same fp32 sums
    # in the same order ((current + previous) + constant)
    # and h is the plain coupled scan of exactly those logits (v read in place
    # from the projection rows instead of a contiguous copy; the row stride can
    # select a narrower tile, whose chunking rounds differently)
    if gc is None or gc.ndim == 2:
        h3, z3 = torch.ops.mogt.coupled_proj_scan(proj, gc, D, r, prev, 0.995)
        h4 = ops.coupled_rank_scan(z.contiguous(), v.contiguous(), damping=0.995)
        torch.cuda.synchronize()
        assert torch.equal(z3, z)
        assert rel_err(to_np(h3), to_np(h4)) <= 1e-6


@pytest.mark.parametrize("vdt", ["fp32", "bf16"])
@pytest.mark.parametrize("tile", TILES_COUPLED)
def test_every_coupled_tile(gpu, tile, vdt):
    """Every compiled coupled tile through the tile-override entry point: ragged
    L, two sequences, 48 channels per gate (divisible by every vector width);
    bf16 z, bf16 output for half of the cases."""
    announce(f"coupled tile {tile} v={vdt}")
    from mogt_amd import ops

    B, L, r, c = 2, 2777, 4, 48
    z, v = synthetic.coupled_inputs(B, L, r, c, seed=sum(tile))
    zt, vt = torch.from_numpy(z).to(gpu), torch.from_numpy(v).to(gpu)
    if vdt == "bf16":
        vt = vt.bfloat16()
    zb = tile[0] % 2 == 0 and vdt == "bf16"   # bf16 gate logits on some cases
    if zb:
        zt = zt.bfloat16()
    ob = tile[2] % 16 == 0                     # bf16 output on some cases
    h = torch.empty(B, L, r * c, device=gpu, dtype=torch.bfloat16 if ob else torch.float32)
    lib = _lib.load()
    nbytes = lib.mogt_diag_scan_workspace_bytes_cfg(B, L, r * c, *tile)
    ws = ops.workspace(nbytes, zt.device, "coupled", ("cfg-test", B, L, r, c, tile))
    rc = lib.mogt_coupled_rank_scan_fwd_cfg(zt.data_ptr(), vt.data_ptr(), h.data_ptr(), B, L, r, c, 0.999,
                                            ops.dtype_code(zt.dtype, "z"), ops.dtype_code(vt.dtype, "v"),
                                            ops.dtype_code(h.dtype, "h"), *tile, ws.data_ptr(), ws.numel(),
                                            ops._stream_handle(zt.device))
    _lib.check(rc, "mogt_coupled_rank_scan_fwd_cfg")
    torch.cuda.synchronize()
    ref = so.coupled_rank_scan(to_np(zt), to_np(vt), r, damping=0.999, v_is_bf16=(vdt == "bf16"))
    tol = FP32_TOL if (vdt == "fp32" and not ob) else BF16_TOL
    assert rel_err(to_np(h), ref) <= tol
    assert ops.workspace_faults() == 0


def test_mixed_modes_share_workspace(gpu):
    """Forward (fp32, bf16), coupled and both reverse-time scans of different shapes
    interleaved on one stream (as a training step runs them), each family on
    its look-back workspace and the forward scans switching layouts on theirs:
    every result stays exact."""
    announce("diag / coupled / reverse / coupled reverse interleaved x25")
    import mogt_amd
    from mogt_amd import ops

    a, b = synthetic.diag_inputs(1, 5000, 768, seed=31)
    at, bt = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    ab, bb = at.bfloat16(), bt.bfloat16()
    ref_f = so.diag_scan(a, b)
    ref_b = so.diag_scan(to_np(ab), to_np(bb))
    z, v = synthetic.coupled_inputs(1, 3001, 16, 48, seed=32)
    zt, vt = torch.from_numpy(z).to(gpu), torch.from_numpy(v).to(gpu)
    ref_c = so.coupled_rank_scan(z, v, 16)
    a2, g2 = synthetic.diag_inputs(2, 777, 320, seed=33)
    a2t, g2t = torch.from_numpy(a2).to(gpu), torch.from_numpy(g2).to(gpu)
    # reverse-time recurrence = forward scan of the time-reversed sequence with
    # the decay shifted by one step (a_{t+1}, and 0 past the end)
    a_sh = np.concatenate([a2[:, 1:], np.zeros_like(a2[:, :1])], axis=1)
    ref_r = so.diag_scan(a_sh[:, ::-1], g2[:, ::-1])[:, ::-1]
    # coupled reverse scan: the same with a = 0.999 (1 - sigmoid(z)) per rank
    dh = np.random.default_rng(34).standard_normal(v.shape).astype(np.float32)
    dht = torch.from_numpy(dh).to(gpu)
    a_c = np.repeat(0.999 * (1.0 - 1.0 / (1.0 + np.exp(-z.astype(np.float64)))), 48, axis=2)
    a_c = np.concatenate([a_c[:, 1:], np.zeros_like(a_c[:, :1])], axis=1).astype(np.float32)
    ref_cr = so.diag_scan(a_c[:, ::-1], dh[:, ::-1])[:, ::-1]
    outs = []
    for it in range(25):
        k = it % 5
        if k == 0:
            outs.append((mogt_amd.diag_scan(at, bt), ref_f, FP32_TOL))
        elif k == 1:
            outs.append((mogt_amd.diag_scan(ab, bb, out_dtype=torch.float32), ref_b, FP32_TOL))
        elif k == 2:
            outs.append((mogt_amd.coupled_rank_scan(zt, vt), ref_c, FP32_TOL))
        elif k == 3:
            outs.append((torch.ops.mogt.diag_scan_rev(a2t, g2t), ref_r, FP32_TOL))
        else:
            outs.append((torch.ops.mogt.coupled_scan_rev(zt, dht, 16, 0.999), ref_cr, FP32_TOL))
    torch.cuda.synchronize()
    for h, ref, tol in outs:
        assert rel_err(to_np(h), ref) <= tol
    assert ops.workspace_faults() == 0


def test_zz_no_lookback_wait_gave_up(gpu):
    """Every bounded wait of every launch above completed normally."""
    from mogt_amd import ops

    assert ops.workspace_faults() == 0
