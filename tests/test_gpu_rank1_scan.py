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


PATHS = ["single", "three"]


def _run(gpu, B, L, H, seed, out_dtype=torch.bfloat16, path="auto"):
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(B, L, H, 64, seed=seed)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    y = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, out_dtype=out_dtype, path=path)
    torch.cuda.synchronize()
    return y, ref


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("B,L,H", [(1, 1, 1), (1, 64, 2), (1, 200, 3), (1, 256, 1), (1, 257, 2),
                                   (2, 1000, 2), (1, 3000, 3)])
def test_small_and_ragged(gpu, B, L, H, path):
    announce(f"rank1 B={B} L={L} H={H} path={path}")
    y, ref = _run(gpu, B, L, H, seed=L + H, path=path)
    assert y.shape == (B, L, H, 64) and y.dtype == torch.bfloat16
    assert rel_err(to_np(y), ref) <= BF16_TOL
    # fp32 output: the bulk agrees much tighter than the bf16 bar
    y32, _ = _run(gpu, B, L, H, seed=L + H, out_dtype=torch.float32, path=path)
    assert rel_err(to_np(y32), ref) <= 5e-3
    from mogt_amd import ops
    assert ops.workspace_faults() == 0


@pytest.mark.parametrize("path", PATHS)
def test_cfg3_full_size(gpu, path):
    """B=2, L=8192, H=12, d=64, bf16 I/O."""
    announce(f"rank1 cfg3 full size path={path}")
    y, ref = _run(gpu, 2, 8192, 12, seed=0, path=path)
    assert rel_err(to_np(y), ref) <= BF16_TOL


def test_paths_agree_and_repeat(gpu):
    """The one-launch and three-launch forms agree (they round different
    bf16 operands: per-sub-chunk vs per-super-chunk decay weights, so the bar
    is the fp32-output bar against the oracle), and repeated one-launch calls
    (workspace reused without clearing, a new epoch each time) agree to fp32
    rounding."""
    announce("rank1 paths agree, repeated calls")
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(2, 4096, 5, 64, seed=21)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
    run = lambda path: mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, out_dtype=torch.float32, path=path)
    y1 = run("single")
    y3 = run("three")
    y1b = run("single")
    y1c = run("single")
    torch.cuda.synchronize()
    assert rel_err(to_np(y1), to_np(y3)) <= 5e-3
    assert rel_err(to_np(y1b), to_np(y1)) <= 1e-5
    assert rel_err(to_np(y1c), to_np(y1)) <= 1e-5
    assert mogt_amd.ops.workspace_faults() == 0


def test_length_switch(gpu):
    """L = 16384 (64 super-chunks) runs in one launch, L = 16640 in three; both
    against the oracle on one head."""
    announce("rank1 length switch")
    import mogt_amd

    for L in (16384, 16640):
        y, ref = _run(gpu, 1, L, 1, seed=L)
        assert rel_err(to_np(y), ref) <= BF16_TOL
    with pytest.raises(ValueError):
        f, k, v, q = synthetic.rank1_inputs(1, 16640, 1, 64, seed=1)
        ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
        mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, path="single")
    assert mogt_amd.ops.workspace_faults() == 0


def test_auto_path_follows_residency(gpu):
    """path 0 ("auto") takes the one-launch kernel only when all of its
    B * H * ceil(L / 256) work-groups are resident together, three per compute
    unit.  The one-launch kernel advances the workspace epoch (header word 2);
    the three launches leave the header alone.  The op's own mirror of the
    rule (which picks the workspace family) must agree with the C entry
    point."""
    announce("rank1 auto path by residency")
    from mogt_amd import _lib, ops

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    L, H = 16384, 12                                            # 64 super-chunks per sequence
    b_big = (ops.R1_GROUPS_PER_CU * cus) // (H * 64) + 1       # one generation does not hold them
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for B, heads, expect_single in ((1, 1, True), (b_big, H, False)):
        g = torch.Generator(device=gpu).manual_seed(B)
        f = torch.sigmoid(2 + torch.randn(B, L, heads, generator=g, device=gpu)).bfloat16()
        k, v, q = (torch.randn(B, L, heads, 64, generator=g, device=gpu).bfloat16() for _ in range(3))
        y = torch.empty_like(q)
        nbytes = lib.mogt_rank1_coupled_scan_workspace_bytes(B, L, heads, 64)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
        rc = lib.mogt_rank1_coupled_scan_fwd_cfg(f.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr(),
                                                 y.data_ptr(), B, L, heads, 64, 1, 1, 1, ws.data_ptr(),
                                                 ws.numel(), 0, stream)
        _lib.check(rc, "mogt_rank1_coupled_scan_fwd_cfg")
        torch.cuda.synchronize()
        epoch = int(ws[8:12].view(torch.int32).item())
        assert (epoch == 1) == expect_single, (B, heads, epoch)
        assert ops._rank1_single(0, B, L, heads, torch.bfloat16, gpu) == expect_single
        assert bool(torch.isfinite(y.float()).all())


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
    """fp32 k, v, q take the three-launch path (the one-launch kernel refuses
    them); checked through the default path and the refusal of the forced one."""
    # fp32 f, k, v, q (rounded to bf16 inside the products): against the oracle
    # on the unrounded inputs, fp32 output
    announce(f"rank1 fp32 inputs L={L} H={H}")
    import mogt_amd

    f, k, v, q = synthetic.rank1_inputs(1, L, H, 64, seed=11 + L)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).float() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    y = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    assert rel_err(to_np(y), ref) <= 1e-2
    with pytest.raises(ValueError):
        mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, path="single")


@pytest.mark.parametrize("L,H", [(700, 2), (3000, 1)])
def test_fp32_gate_bf16_operands_one_launch(gpu, L, H):
    """fp32 f with bf16 k, v, q (the default path's one-launch kernel at these
    lengths; several super-chunks, so the carry exchange runs): against the
    oracle, and no wait gave up."""
    announce(f"rank1 fp32 f, bf16 k v q, one launch, L={L} H={H}")
    import mogt_amd
    from mogt_amd import ops

    f, k, v, q = synthetic.rank1_inputs(1, L, H, 64, seed=40 + L)
    ft = torch.from_numpy(f).to(gpu).float()
    kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    before = ops.workspace_faults()
    for path in ("auto", "single"):
        y = mogt_amd.ops.rank1_coupled_scan(ft, kt, vt, qt, out_dtype=torch.float32, path=path)
        torch.cuda.synchronize()
        assert rel_err(to_np(y), ref) <= 5e-3, path
    assert ops.workspace_faults() == before == 0


def _launch_path(gpu, ws, f, k, v, q, path):
    """One call of mogt_rank1_coupled_scan_fwd_cfg through the C ABI on the
    workspace ``ws``; returns y and the workspace's give-up count."""
    import ctypes

    from mogt_amd import _lib, ops

    lib = _lib.load()
    B, L, H, d = k.shape
    y = torch.empty(k.shape, dtype=torch.float32, device=gpu)
    sh = ops._stream_handle(gpu)
    rc = lib.mogt_rank1_coupled_scan_fwd_cfg(f.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr(), y.data_ptr(),
                                             B, L, H, d, _lib.MOGT_BF16, _lib.MOGT_BF16, _lib.MOGT_F32,
                                             ws.data_ptr(), ws.numel(), path, sh)
    _lib.check(rc, "mogt_rank1_coupled_scan_fwd_cfg")
    count = ctypes.c_uint32(0)
    _lib.check(lib.mogt_workspace_faults(ws.data_ptr(), ws.numel(), ctypes.byref(count), sh), "faults")
    return y, int(count.value)


def test_giveup_poisons_and_counts(gpu):
    """The give-up handling of the one-launch kernel, forced from the host
    (path 3: super-chunk 0 withholds its aggregate and waits end after 64
    polls; every kernel exits normally).  Every work-group waits on that
    aggregate once, so the count grows by B*H*nsc; the first super-chunk's
    outputs (which need no carry) stay right and every later one is NaN; a
    normal launch afterwards on the same workspace is right and counts
    nothing."""
    announce("rank1 forced give-up (path 3) B=1 L=700 H=2")
    B, L, H = 1, 700, 2
    nsc = -(-L // 256)
    f, k, v, q = synthetic.rank1_inputs(B, L, H, 64, seed=77)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    from mogt_amd import _lib

    # a private zero-filled workspace: the give-ups stay out of the cached ones
    ws = torch.zeros(_lib.load().mogt_rank1_coupled_scan_workspace_bytes(B, L, H, 64), dtype=torch.uint8,
                     device=gpu)
    _, c0 = _launch_path(gpu, ws, ft, kt, vt, qt, 1)
    y, c1 = _launch_path(gpu, ws, ft, kt, vt, qt, 3)
    torch.cuda.synchronize()
    assert c1 - c0 == B * H * nsc
    yn = to_np(y)
    assert np.isnan(yn[:, 256:]).all()
    assert np.isfinite(yn[:, :256]).all()
    assert rel_err(yn[:, :256], ref[:, :256]) <= 5e-3
    y2, c2 = _launch_path(gpu, ws, ft, kt, vt, qt, 1)
    torch.cuda.synchronize()
    assert c2 == c1
    assert rel_err(to_np(y2), ref) <= 5e-3


def test_checked_mode_falls_back_to_three_launches(gpu, monkeypatch):
    """In checked mode a one-launch call whose waits gave up (forced as above)
    is recomputed on the three-launch path, with a warning, and its result is
    right."""
    announce("rank1 checked-mode fallback")
    from mogt_amd import ops

    monkeypatch.setattr(ops, "CHECK_WORKSPACE", True)
    # a registry of workspaces for this test only: the forced give-ups stay
    # out of the process's cached workspaces
    for name in ("_ws_cache", "_ws_layout", "_ws_faults_seen"):
        monkeypatch.setattr(ops, name, {})
    monkeypatch.setattr(ops, "_ws_retired", [])
    monkeypatch.setattr(ops, "_ws_retired_lookback", [])
    f, k, v, q = synthetic.rank1_inputs(1, 900, 2, 64, seed=78)
    ft, kt, vt, qt = (torch.from_numpy(x).to(gpu).bfloat16() for x in (f, k, v, q))
    ref = so.rank1_coupled_scan(*(to_np(x) for x in (ft, kt, vt, qt)))
    with pytest.warns(RuntimeWarning, match="three-launch"):
        y = torch.ops.mogt.rank1_coupled_scan(ft, kt, vt, qt, torch.float32, ops._RANK1_GIVEUP_TEST)
    torch.cuda.synchronize()
    assert np.isfinite(to_np(y)).all()
    assert rel_err(to_np(y), ref) <= 5e-3
    # a normal call in checked mode afterwards: no new give-up, no warning
    import warnings

    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = ops.rank1_coupled_scan(ft, kt, vt, qt, out_dtype=torch.float32, path="single")
    assert rel_err(to_np(y), ref) <= 5e-3
