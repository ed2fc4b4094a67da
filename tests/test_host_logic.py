"""Host-side logic that needs no GPU: the GEMM-weight cache of the MOGT
blocks (built from parameters, reused only while no gradient is recorded and
no parameter changed), the workspace families and checked-mode accounting,
bench.py's profile provenance, the rocprof summariser, the rank-1 kernels'
buffer ranges, and the m0 use of the bf16 GEMMs' generated code."""
from pathlib import Path

import pytest
import torch
import torch.nn as nn

from mogt_amd.model_mogt import _gemm_weight


def test_gemm_weight_cache_reuse_and_invalidation():
    torch.manual_seed(0)
    owner = nn.Module()
    a, b = nn.Linear(4, 3, bias=False), nn.Linear(4, 2, bias=False)
    build = lambda: torch.cat([a.weight, b.weight], dim=0)
    with torch.no_grad():
        w1 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
        assert _gemm_weight(owner, "ab", (a.weight, b.weight), build) is w1   # reused
        a.weight.mul_(2.0)                                                    # version bump
        w2 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
        assert w2 is not w1 and torch.equal(w2, build())
        b.weight.data = torch.randn(2, 4)                                     # new storage
        w3 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
        assert w3 is not w2 and torch.equal(w3, build())
    with torch.inference_mode():
        w4 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
        assert w4 is not w3                                                   # inference-mode entry of its own
        assert _gemm_weight(owner, "ab", (a.weight, b.weight), build) is w4
    # with gradients: rebuilt every call and differentiable to the parameters
    g1 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
    g2 = _gemm_weight(owner, "ab", (a.weight, b.weight), build)
    assert g1 is not g2 and g1.grad_fn is not None
    g1.sum().backward()
    assert torch.equal(a.weight.grad, torch.ones(3, 4)) and torch.equal(b.weight.grad, torch.ones(2, 4))


def test_gemm_weight_cache_invalidation_paths():
    """Writes through p.data bypass the version counter; invalidate_weight_cache,
    train()/eval() and load_state_dict drop the cached operands."""
    from mogt_amd.model_mogt import SwiGLU, MOGTBlock

    blk = MOGTBlock(d_model=32, r=4, ffn_hidden=64)
    ffn: SwiGLU = blk.ffn
    build = lambda: torch.cat([ffn.w1.weight, ffn.w2.weight], dim=0)   # noqa: E731
    with torch.no_grad():
        w = _gemm_weight(ffn, "w12", (ffn.w1.weight, ffn.w2.weight), build)
        ffn.w1.weight.data.mul_(2.0)                     # not seen by the version counter
        assert _gemm_weight(ffn, "w12", (ffn.w1.weight, ffn.w2.weight), build) is w
        blk.invalidate_weight_cache()
        w2 = _gemm_weight(ffn, "w12", (ffn.w1.weight, ffn.w2.weight), build)
        assert w2 is not w and torch.equal(w2[:64], ffn.w1.weight)
        blk.eval()
        w3 = _gemm_weight(ffn, "w12", (ffn.w1.weight, ffn.w2.weight), build)
        assert w3 is not w2
        blk.load_state_dict(blk.state_dict())
        assert _gemm_weight(ffn, "w12", (ffn.w1.weight, ffn.w2.weight), build) is not w3


def test_gemm_table_is_well_formed():
    """The tuned GEMM table: TunableOp's validator header for gfx950 and one
    solution per backbone GEMM shape (bf16, the d_model 768 projections)."""
    from mogt_amd import gemm_tuning

    lines = gemm_tuning.TABLE.read_text().splitlines()
    head = {ln.split(",")[1]: ln.split(",")[2] for ln in lines if ln.startswith("Validator,")}
    assert head["GCN_ARCH_NAME"].startswith("gfx950") and "PT_VERSION" in head
    rows = [ln.split(",") for ln in lines if ln.startswith("GemmTunableOp_")]
    assert len(rows) >= 40 and all(len(r) == 4 and float(r[3]) > 0 for r in rows)
    shapes = {r[1] for r in rows}
    assert any(s.startswith("tn_6144_32768_768") for s in shapes)   # the fused [w1; w2] projection


def test_cast_groups_values_and_gradients():
    """ops.cast_groups: each group concatenated along rows in the target dtype
    (the values of cast-then-cat), and every parameter's gradient its rows of
    the group's gradient cast back to the parameter's dtype -- what separate
    casts and a torch.cat would give."""
    from mogt_amd import ops

    torch.manual_seed(0)
    a = torch.randn(3, 4, requires_grad=True)
    b = torch.randn(2, 4, requires_grad=True)
    c = torch.randn(5, 2, requires_grad=True)
    d = torch.randn(1, 2, requires_grad=True)   # no gradient reaches it
    ab, cc, dd = ops.cast_groups([[a, b], [c], [d]], torch.bfloat16)
    assert ab.dtype == torch.bfloat16 and ab.shape == (5, 4) and cc.shape == (5, 2)
    assert torch.equal(ab, torch.cat([a, b]).bfloat16()) and torch.equal(cc, c.bfloat16())
    w0, w1 = torch.randn(5, 4), torch.randn(5, 2)
    ((ab.float() * w0).sum() + (cc.float() * w1).sum()).backward()
    ref = [t.detach().clone().requires_grad_() for t in (a, b, c)]
    ((torch.cat(ref[:2]).bfloat16().float() * w0).sum() + (ref[2].bfloat16().float() * w1).sum()).backward()
    for got, want in zip((a, b, c), ref):
        assert got.grad.dtype == torch.float32 and torch.equal(got.grad, want.grad)
    assert d.grad is None


def test_affine_scan_dropins_need_a_gpu():
    """Host tensors are scanned on the GPU; without one the drop-ins raise
    instead of computing on the CPU."""
    import pytest
    import torch

    from mogt_amd import affine_scan as das

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    U = torch.eye(3, dtype=torch.float64).expand(1, 5, 3, 3)
    V = torch.ones(1, 5, 3, 2, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="GPU"):
        das.affine_scan_sequential(U, V, state_dtype=torch.float64)
    with pytest.raises(RuntimeError, match="GPU"):
        das.affine_scan_sequential_backward(U, V, V, state_dtype=torch.float64)
    # argument errors come first, as in the reference
    with pytest.raises(ValueError):
        das.affine_scan_sequential(U, V, state_dtype=torch.int64)
    with pytest.raises(ValueError):
        das.affine_scan_block_reference(U, V, block_size=0)


def test_bench_traffic_needs_a_profile_of_this_build(tmp_path, monkeypatch):
    """bench.py takes the headline's HBM traffic only from a profile whose
    kernel-source hashes equal the loaded library's manifest."""
    import bench

    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "p.md").write_text(
        "# profile\n\n| `k` | 1 |\n\nkernel_sources=diag_kernel.h:aaaa,common.h:bbbb,flags:cccc\n"
        "avg_us=56.8\nhbm_bytes_per_launch=307157755\n")
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    manifest = {"diag_kernel.h": "aaaa", "common.h": "bbbb", "flags": "cccc", "rank1_scan.hip": "dddd"}
    t, info = bench.read_traffic("p.md", manifest)
    assert t == 307157755.0 and info["status"] == "matches this build"
    t, info = bench.read_traffic("p.md", dict(manifest, **{"common.h": "eeee"}))
    assert t is None and "common.h" in info["status"]
    t, info = bench.read_traffic("p.md", dict(manifest, flags="ffff"))
    assert t is None and "flags" in info["status"]
    t, info = bench.read_traffic("missing.md", manifest)
    assert t is None and info["status"] == "missing"
    (prof / "q.md").write_text("avg_us=1\nhbm_bytes_per_launch=5\n")   # names no sources
    t, info = bench.read_traffic("q.md", manifest)
    assert t is None and "refused" in info["status"]


def test_rocprof_summary_groups_and_calibrates(tmp_path):
    """The profile summariser groups dispatches by kernel and launch shape and
    scales the counters by the process's first five copy dispatches."""
    import csv

    from mogt_amd import rocprof_summary as rs

    assert rs.short_name("void mogt::diag_scan_kernel<0, float, 2>(float const*, int)") == \
        "diag_scan_kernel<0, float, 2>"
    assert rs.display_name("Cijk_Ailk_Bjlk_BBS_BH_UserArgs_MT192x192x64_MI16x16x1_SN") == "library GEMM MT192x192x64"
    assert rs.display_name("diag_scan_kernel<0, float, 2>") == "diag_scan_kernel<0, float, 2>"
    # kernels in an anonymous namespace: its parenthesis is not the parameter list
    assert rs.short_name("mogt::(anonymous namespace)::wgrad_gemm_kernel(mogt::(anonymous namespace)::"
                         "WgradParams)") == "wgrad_gemm_kernel"
    assert rs.short_name("void mogt::(anonymous namespace)::wgrad_reduce_kernel<false>(float const*, void*, "
                         "long, int, int, int)") == "wgrad_reduce_kernel<false>"
    rows = []
    for i in range(5):      # calibration: 256 MiB copied, counter reads half of it
        rows.append(dict(Counter_Name="FETCH_SIZE", Counter_Value="131072", Dispatch_Id=str(i + 1),
                         Kernel_Name="__amd_rocclr_copyBuffer", Workgroup_Size="512", Grid_Size="131072"))
    rows.append(dict(Counter_Name="FETCH_SIZE", Counter_Value="999999", Dispatch_Id="9",
                     Kernel_Name="__amd_rocclr_copyBuffer", Workgroup_Size="512", Grid_Size="262144"))
    for i, v in enumerate((100.0, 200.0)):
        rows.append(dict(Counter_Name="FETCH_SIZE", Counter_Value=str(v), Dispatch_Id=str(10 + i),
                         Kernel_Name="void mogt::k<1>(int)", Workgroup_Size="256", Grid_Size="2048"))
    per, copy = rs.counter_table(rows, "FETCH_SIZE")
    assert copy == 131072.0                      # the later, larger copy is not the calibration
    assert per[("k<1>", 8, 256)] == 150.0


def test_rocprof_summary_per_step_table():
    """The per-step kernel table: every dispatch divided by the step count,
    grouped into this library's kernels, library GEMMs and the rest, kernels
    ranked by total time."""
    from mogt_amd import rocprof_summary as rs

    def row(name, us, t0):
        return dict(Kernel_Name=name, Start_Timestamp=str(t0), End_Timestamp=str(t0 + int(us * 1000)))

    rows = [row("void mogt::swiglu_gemm_persistent_kernel(mogt::SwigluParams)", 300.0, 0),
            row("void mogt::swiglu_gemm_persistent_kernel(mogt::SwigluParams)", 310.0, 10 ** 6),
            row("Cijk_Ailk_Bljk_BBS_BH_MT256x256x64_MI16x16x1_SN", 80.0, 2 * 10 ** 6),
            row("Cijk_Ailk_Bljk_BBS_BH_MT256x256x64_MI16x16x1_SN", 90.0, 3 * 10 ** 6),
            row("void at::native::vectorized_gather_kernel<16, long>(char*)", 20.0, 4 * 10 ** 6)]
    lines = rs.per_step_lines(rows, steps=2, top=0)
    assert lines[0] == "400 us of kernels per step"
    text = "\n".join(lines)
    assert "| HIP kernels of this library | 305 | 76% |" in text
    assert "| hipBLASLt GEMMs | 85 | 21% |" in text
    assert "| PyTorch kernels and copies | 10 | 2% |" in text
    kern = [ln for ln in lines if ln.startswith("| `")]
    assert kern[0] == "| `swiglu_gemm_persistent_kernel` | 1.0 | 305.0 | 305 |"
    assert kern[1] == "| `library GEMM MT256x256x64` | 1.0 | 85.0 | 85 |"
    assert len(rs.per_step_lines(rows, steps=2, top=1)) == len(lines) - 2


def test_rank1_buffer_ranges_stay_in_bounds():
    """Every buffer range the rank-1 kernels build (K_A's prefetches, the
    output and one-launch tiles, padding tiles past L) lies inside its tensor,
    covers the rows before L and no row after, for ragged lengths and both
    element sizes -- evaluated by the same helper the kernels call."""
    from mogt_amd import _lib

    lib = _lib.load()
    for L in (1, 2, 63, 64, 65, 255, 256, 257, 700, 1000, 3000, 8192, 16383, 16385):
        for B, H in ((1, 1), (2, 3), (1, 12)):
            for elem in (2, 4):
                rc = lib.mogt_rank1_check_ranges(B, L, H, elem)
                assert rc == 0, (B, L, H, elem, lib.mogt_last_error())
    assert lib.mogt_rank1_check_ranges(1, 100, 1, 3) == -1
    assert lib.mogt_rank1_check_ranges(0, 100, 1, 2) == -1


def _fake_device_workspace(monkeypatch):
    """ops.workspace on host tensors: one fake stream, no capture."""
    from mogt_amd import ops

    monkeypatch.setattr(ops, "_stream_handle", lambda device: 7)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(ops, "_ws_cache", {})
    monkeypatch.setattr(ops, "_ws_layout", {})
    monkeypatch.setattr(ops, "_ws_retired", [])
    monkeypatch.setattr(ops, "_ws_retired_lookback", [])
    return ops, torch.device("cpu", 0)


def test_swiglu_persistent_schedule_covers_every_tile_once():
    """The persistent SwiGLU GEMM's tile assignment (a contiguous run per XCD,
    dealt to that XCD's work-groups in turn, each tile mapped to its row and
    output block): every tile taken by exactly one work-group, for CU counts of
    other GPUs as well as MI355X's 256 and for fewer tiles than work-groups."""
    from mogt_amd import _lib

    lib = _lib.load()
    for grid in (1, 3, 7, 8, 9, 37, 80, 104, 228, 255, 256, 304):
        for rows in (1, 255, 256, 257, 300, 2049, 32768, 32768 + 100):
            for hidden in (128, 384, 3072):
                rc = lib.mogt_swiglu_check_schedule(rows, hidden, grid)
                assert rc == 0, (grid, rows, hidden, lib.mogt_last_error())
    assert lib.mogt_swiglu_check_schedule(0, 128, 256) != 0
    assert lib.mogt_swiglu_check_schedule(100, 100, 256) != 0


def test_lookback_workspaces_are_kept_apart_and_cleared_on_layout_change(monkeypatch):
    import pytest

    ops, dev = _fake_device_workspace(monkeypatch)
    a = ops.workspace(4096, dev, "diag", (1, 2, 3))
    a[:8] = 5          # header: epoch and give-up count
    a[256:4096] = 9    # tagged words of the launch
    assert ops.workspace(4096, dev, "diag", (1, 2, 3)) is a          # same layout: kept as is
    assert int(a[300]) == 9
    p = ops.workspace(4096, dev)                                       # plain data: its own buffer
    assert p is not a
    r = ops.workspace(4096, dev, "rank1", (1,))
    assert r is not a and r is not p
    b = ops.workspace(2048, dev, "diag", (4, 5, 6))                    # another layout: cleared past the header
    assert b is a
    assert int(a[0]) == 5 and int(a[256:2048].max()) == 0 and int(a[3000]) == 9
    with pytest.raises(ValueError):
        ops.workspace(64, dev, "coupled")                              # look-back families name their layout
    # growth: a new zeroed buffer, the old one kept for captured graphs
    c = ops.workspace(1 << 20, dev, "diag", (4, 5, 6))
    assert c is not a and c.numel() >= 1 << 20 and int(c.max()) == 0 and a in ops._ws_retired


def test_captured_workspace_is_pinned_to_its_layout(monkeypatch):
    """A look-back buffer used under graph capture keeps serving its layout
    (no clearing fill recorded when the capture repeats the warm-up's layout);
    a launch of another layout afterwards gets a new buffer, and the pinned
    one stays alive and untouched."""
    ops, dev = _fake_device_workspace(monkeypatch)
    capturing = [False]
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing[0])
    a = ops.workspace(4096, dev, "coupled", ("A",))     # eager warm-up
    a[256:] = 7
    capturing[0] = True
    assert ops.workspace(4096, dev, "coupled", ("A",)) is a
    assert int(a[300]) == 7                               # not cleared for the capture
    capturing[0] = False
    assert ops.workspace(4096, dev, "coupled", ("A",)) is a   # eager, same layout: shared
    b = ops.workspace(4096, dev, "coupled", ("B",))       # another layout: a new buffer
    assert b is not a and a in ops._ws_retired and int(a[300]) == 7 and int(b.max()) == 0
    assert ops.workspace(4096, dev, "coupled", ("C",)) is b   # b is not pinned: cleared in place
    # a first capture with another layout than the eager one clears in place and pins
    b[256:] = 3
    capturing[0] = True
    assert ops.workspace(4096, dev, "coupled", ("D",)) is b and int(b[256:4096].max()) == 0
    capturing[0] = False
    assert ops.workspace(4096, dev, "coupled", ("E",)) is not b


def test_workspace_made_under_inference_mode_is_cleared_outside_it(monkeypatch):
    """A buffer first made inside torch.inference_mode() (an inference-mode
    forward) is still cleared in place when a later launch of another layout
    runs outside that mode (a no-grad or training call)."""
    ops, dev = _fake_device_workspace(monkeypatch)
    with torch.inference_mode():
        a = ops.workspace(4096, dev, "coupled", ("A",))
        a[256:] = 7
    assert not a.is_inference()
    with torch.no_grad():
        assert ops.workspace(4096, dev, "coupled", ("B",)) is a
    assert int(a[256:4096].max()) == 0
    with torch.inference_mode():
        a[256:] = 7
        assert ops.workspace(4096, dev, "coupled", ("C",)) is a and int(a[256:4096].max()) == 0


def test_fault_count_reads_only_lookback_headers(monkeypatch):
    """Only look-back buffers carry the give-up counter in their header; a
    plain buffer's first bytes are data (e.g. the weight-gradient GEMM's fp32
    partials) and are never read as a count, live or retired."""
    ops, dev = _fake_device_workspace(monkeypatch)
    read = []
    monkeypatch.setattr(ops, "_faults_of", lambda buf: read.append(buf) or 0)
    plain = ops.workspace(4096, dev)
    plain[:] = 255
    diag = ops.workspace(4096, dev, "diag", (1,))
    assert ops.workspace_faults() == 0 and len(read) == 1 and read[0] is diag
    ops.workspace(1 << 20, dev)                      # plain grows: old one retired
    ops.workspace(1 << 20, dev, "diag", (1,))        # diag grows: old one retired
    read.clear()
    ops.workspace_faults()
    assert len(read) == 2 and any(b is diag for b in read) and not any(b is plain for b in read)


def test_checked_mode_reports_each_give_up_once(monkeypatch):
    import pytest

    from mogt_amd import ops

    counts = iter([0, 2, 2, 3])
    monkeypatch.setattr(ops, "_faults_of", lambda buf: next(counts))
    monkeypatch.setattr(ops, "CHECK_WORKSPACE", True)
    monkeypatch.setattr(ops, "_ws_faults_seen", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    ws = torch.zeros(512, dtype=torch.uint8)
    ops._checked(ws, "scan")                      # 0: fine
    with pytest.raises(ops.WorkspaceFault, match="2 look-back"):
        ops._checked(ws, "scan")                  # 2 new give-ups
    ops._checked(ws, "scan")                      # still 2: nothing new
    with pytest.raises(ops.WorkspaceFault, match="1 look-back"):
        ops._checked(ws, "scan")                  # one more


@pytest.mark.parametrize("source", ["swiglu_gemm.hip", "wgrad_gemm.hip", "rank1_scan.hip"])
def test_gemm_m0_only_feeds_lds_dma(tmp_path, source):
    """The bf16 GEMMs (fused SwiGLU, split-K weight gradient) and the rank-1
    scan's carry exchange set m0 in inline assembly for their direct-to-LDS
    loads (clang warns that m0 is reserved).
    On the code this build generates for gfx950: every write of m0 is one of
    those asm blocks, immediately followed by the load that reads it, and no
    other instruction of the kernel reads m0 (no LDS-direct, interpolation,
    GWS, movrel or message instructions), so no compiler-held m0 value is
    overwritten."""
    import re
    import shutil
    import subprocess

    import pytest

    from mogt_amd import _build

    if not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()):
        pytest.skip("hipcc not available")
    out = tmp_path / "gemm.s"
    flags = [f for f in _build.HIPCC_FLAGS if f != "-fPIC"] + _build.FILE_FLAGS.get(source, [])
    cmd = [_build.hipcc(), *flags, f"-I{_build.INCLUDE}", "--cuda-device-only", "-S",
           str(_build.CSRC / source), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    lines = [ln.split(";")[0].strip() for ln in out.read_text().splitlines()]
    code = [ln for ln in lines if ln and not ln.startswith((".", "//")) and not ln.endswith(":")]
    writes = [i for i, ln in enumerate(code) if re.match(r"s_mov_b32\s+m0\b", ln)]
    dma = [i for i, ln in enumerate(code) if re.match(r"buffer_load_dword\w*\s.*\blds$", ln)]
    assert writes and len(writes) == len(dma)
    for i in writes:
        assert code[i + 1] == "s_nop 0" and code[i + 2] in [code[j] for j in dma], code[i:i + 3]
    # the asm blocks' m0 source is any scalar register the compiler picked (vcc_lo is one)
    others = [ln for ln in code if "m0" in ln and not re.match(r"s_mov_b32\s+m0, (s\d+|vcc_lo|vcc_hi)$", ln)]
    assert not others, others[:5]
    implicit = [ln for ln in code if re.match(r"(s_sendmsg|s_movrel|v_movrel|ds_gws|ds_append|ds_consume|"
                                              r"ds_ordered|v_interp|ds_param|ds_direct|lds_param|lds_direct)", ln)]
    assert not implicit, implicit[:5]
