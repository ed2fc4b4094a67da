#!/usr/bin/env python3
"""Benchmark of the MI355X MOGT scan operator (one GPU).

Headline: the diagonal affine scan core at B=1,
D=768, L=32768, fp32 I/O.  One "step" = one launch of the single-pass scan
over one batch with inputs already resident in HBM.  Three input/output sets
are rotated (906 MB working set) so the 256 MB Infinity Cache cannot serve the
re-reads.  Timing: HIP events on the launch stream around K launches, after W
warm-up launches; the roofline uses algorithmic bytes (read a, read b, write h
= 3 * 4 * D bytes per token) over the average launch duration.

The CPU baseline is the reference's sequential PyTorch scan restated in
oracle/torch_ref.py (a Python loop over L of torch.bmm, fp32 state), run on the
host cores over the same folded workload.

Prints ONE JSON line on stdout.  Extra measurements (other lengths, bf16 I/O,
the coupled mixer scan) go under "extras".
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "scan core ms + HBM GB/s at D768 L=32768; MOGT 4-layer fwd ms"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
REF_TRITON_CORE_MS_L4 = 5.48   # reference hybrid core @ L=32768 (R=16, C=48, NVIDIA L4)
# rocprofv3 profile of the headline kernel (trace + FETCH_SIZE / WRITE_SIZE)
HEADLINE_PROFILE = "diag_scan_d768_l32768_fp32.md"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    p.add_argument("--only", default="all",
                   help="after the headline: every extra (all), none (diag), or a comma list of "
                        "coupled (the mixer scan), rank1 (configs[2]), dense (core shape and configs[3]), "
                        "swiglu, wgrad (the training path's weight-gradient GEMMs), backbone (configs[4] "
                        "forward and training step)")
    p.add_argument("--tile", default=None,
                   help="vec,lanes,steps,waves override for the headline diag scan")
    p.add_argument("--sweep", action="store_true", help="time every compiled diag tile")
    p.add_argument("--calib-copy", action="store_true",
                   help="also run a plain 256 MiB device copy (PMC calibration)")
    args = p.parse_args()
    groups = {"diag", "coupled", "rank1", "dense", "swiglu", "wgrad", "backbone", "all"}
    args.only = set(args.only.split(","))
    if not args.only <= groups:
        p.error(f"--only takes a comma list of {sorted(groups)}")
    return args


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------- helpers
class EventTimer:
    """HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch = torch
        self.stream = stream

    def time(self, fn, steps: int, warmup: int) -> float:
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for i in range(steps):
            fn(i)
        end.record(self.stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps   # ms per launch


def diag_launcher(torch, lib, ops, B, L, D, dtype, out_dtype, sets, tile=None, seed=1):
    """Rotating input/output sets and a closure that launches one scan via the C ABI."""
    from mogt_amd import synthetic

    a, b = synthetic.diag_inputs(B, L, D, a_mean=3.0, b_std=0.5, seed=seed)
    dev = torch.device("cuda:0")
    a0 = torch.from_numpy(a).to(dev).to(dtype)
    b0 = torch.from_numpy(b).to(dev).to(dtype)
    bufs = []
    for _ in range(sets):
        bufs.append((a0.clone(), b0.clone(), torch.empty(B, L, D, dtype=out_dtype, device=dev)))
    del a0, b0
    ic = ops.dtype_code(dtype, "bench")
    oc = ops.dtype_code(out_dtype, "bench")
    if tile is None:
        nbytes = lib.mogt_diag_scan_workspace_bytes(B, L, D, ic)
    else:
        nbytes = lib.mogt_diag_scan_workspace_bytes_cfg(B, L, D, *tile)
    ws = ops.workspace(nbytes, dev, "diag", ("bench", B, L, D, ic, tile))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    args = [(x.data_ptr(), y.data_ptr(), z.data_ptr()) for x, y, z in bufs]
    wsp, wsn = ws.data_ptr(), ws.numel()

    if tile is None:
        fn = lib.mogt_diag_scan_fwd

        def launch(i):
            pa, pb, ph = args[i % sets]
            rc = fn(pa, pb, ph, None, B, L, D, ic, oc, wsp, wsn, sh)
            if rc:
                raise RuntimeError(lib.mogt_last_error().decode())
    else:
        fn = lib.mogt_diag_scan_fwd_cfg
        v, fl, s, w = tile

        def launch(i):
            pa, pb, ph = args[i % sets]
            rc = fn(pa, pb, ph, None, B, L, D, ic, oc, v, fl, s, w, wsp, wsn, sh)
            if rc:
                raise RuntimeError(lib.mogt_last_error().decode())

    return launch, stream, bufs


def measure_diag(torch, lib, ops, L, dtype, out_dtype, steps, warmup, tile=None, D=768, B=1):
    esz = 2 if dtype == torch.bfloat16 else 4
    osz = 2 if out_dtype == torch.bfloat16 else 4
    total = B * L * D * (2 * esz + osz)
    sets = max(2, min(6, int((1 << 30) // total) + 1))
    launch, stream, bufs = diag_launcher(torch, lib, ops, B, L, D, dtype, out_dtype, sets, tile)
    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    del bufs
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9}


def measure_diag_op(torch, L, steps, warmup, graph, D=768, B=1, sets=3, per_graph=1):
    """Op-level time of ``mogt_amd.diag_scan`` (fp32): per call through the
    Python boundary (custom-op dispatch, output allocation, C-ABI launch), or
    the same call captured in a HIP graph and replayed: ``per_graph`` calls
    (cycling through the input sets) per graph, one graph per input set, time
    per call."""
    import mogt_amd

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(17)
    bufs = [(torch.sigmoid(torch.randn(B, L, D, generator=gen, device=dev) + 3.0),
             torch.randn(B, L, D, generator=gen, device=dev) * 0.5) for _ in range(sets)]
    cur = torch.cuda.current_stream(dev)
    if not graph:
        fn = lambda i: mogt_amd.diag_scan(*bufs[i % sets])
    else:
        s = torch.cuda.Stream()
        graphs = []
        for a, b in bufs:
            s.wait_stream(cur)
            with torch.cuda.stream(s):   # warm-up on the capture stream: its workspace exists before capture
                for _ in range(2):
                    mogt_amd.diag_scan(a, b)
            cur.wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph(keep_graph=True)
            k0 = len(graphs)
            with torch.cuda.graph(g, stream=s):
                out = [mogt_amd.diag_scan(*bufs[(k0 + n) % sets]) for n in range(per_graph)]
            g.instantiate()
            graphs.append((g, out))
        torch.cuda.synchronize()
        fn = lambda i: graphs[i % sets][0].replay()
    ms = EventTimer(torch, cur).time(fn, steps, warmup) / (per_graph if graph else 1)
    return {"ms": ms, "graph_nodes": [graph_nodes(g) for g, _ in graphs] if graph else None}


def graph_nodes(g):
    """Number of nodes of a captured graph (hipGraphGetNodes on its raw
    hipGraph_t), so a replay's cost can be told apart from extra captured work."""
    import ctypes

    try:
        hip = ctypes.CDLL("libamdhip64.so")
    except OSError:
        return None
    n = ctypes.c_size_t(0)
    rc = hip.hipGraphGetNodes(ctypes.c_void_p(g.raw_cuda_graph()), None, ctypes.byref(n))
    return int(n.value) if rc == 0 else None


def measure_diag_rev(torch, lib, ops, L, steps, warmup, D=768, B=1, sets=3):
    """Reverse-time diagonal scan (the backward's G_t = dH_t + a_{t+1} G_{t+1}),
    fp32 a, dH in, G out, via mogt_diag_scan_rev_fwd."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(13)
    bufs = [(torch.sigmoid(torch.randn(B, L, D, generator=gen, device=dev) + 3.0),
             torch.randn(B, L, D, generator=gen, device=dev), torch.empty(B, L, D, device=dev))
            for _ in range(sets)]
    ws = ops.workspace(lib.mogt_diag_scan_workspace_bytes(B, L, D, 0), dev, "diag_rev", ("bench", B, L, D))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def launch(i):
        a, g, out = bufs[i % sets]
        rc = lib.mogt_diag_scan_rev_fwd(a.data_ptr(), g.data_ptr(), out.data_ptr(), B, L, D,
                                        ws.data_ptr(), ws.numel(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    total = B * L * D * 12
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9}


def measure_connection_map(torch, lib, ops, impl, n, r, steps, warmup):
    """Batched transport maps of skew generators (model_mogt.py:79-102):
    the HIP kernel via the C ABI, and torch's routine on the same inputs."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(21)
    T = torch.randn(n, r, r, generator=gen, device=dev) * 0.1
    A = (T - T.transpose(-1, -2)).contiguous()
    U = torch.empty_like(A)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    from mogt_amd import _lib as mlib

    code = mlib.MOGT_CONN_EXP if impl == "matrix_exp" else mlib.MOGT_CONN_CAYLEY

    def launch(i):
        rc = lib.mogt_connection_map_fwd(A.data_ptr(), U.data_ptr(), n, r, 1.0, 1.0, code, 0, sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    eye = torch.eye(r, device=dev)

    def launch_torch(i):
        if impl == "matrix_exp":
            torch.matrix_exp(A)
        else:
            torch.linalg.solve(eye - 0.5 * A, eye + 0.5 * A)

    ms_torch = EventTimer(torch, stream).time(launch_torch, max(3, steps // 10), 2)
    return {"ms": ms, "ms_torch": ms_torch}


def _reference_chunked_ce_torch(torch, hidden, weight, labels, chunk):
    """The reference's chunked tied-head CE (chunked_lm_loss.py:7-72) restated
    with torch ops -- forward and backward -- for a same-GPU timing comparison:
    per chunk an fp32 GEMM and F.cross_entropy, then softmax, one-hot update,
    scale and the two gradient GEMMs."""
    import torch.nn.functional as F

    T, D = hidden.shape[0] * hidden.shape[1], hidden.shape[2]
    hf = hidden.reshape(T, D)
    lf = labels.reshape(T)
    wf = weight.float()
    loss = hidden.new_zeros((), dtype=torch.float32)
    with torch.no_grad():
        for s in range(0, T, chunk):
            e = min(s + chunk, T)
            loss = loss + F.cross_entropy(hf[s:e].float().matmul(wf.t()), lf[s:e], reduction="sum")
        gh = torch.empty_like(hf)
        gw = torch.zeros_like(weight, dtype=torch.float32)
        scale = 1.0 / T
        for s in range(0, T, chunk):
            e = min(s + chunk, T)
            hc = hf[s:e]
            probs = torch.softmax(hc.float().matmul(wf.t()), dim=-1)
            probs[torch.arange(e - s, device=hidden.device), lf[s:e]] -= 1.0
            probs = probs * scale
            gh[s:e] = probs.matmul(wf).to(hidden.dtype)
            gw = gw + probs.t().matmul(hc.float())
    return loss / T, gh, gw


def measure_swiglu(torch, steps, warmup, rows=32768, d_in=768, hidden=3072):
    """The FFN's gate (model_mogt.py:29-30) at configs[4]'s shape: the fused
    SwiGLU GEMM (csrc/swiglu_gemm.hip) against the unfused path (one library
    GEMM against [w1; w2], then the silu_mul row kernel), bf16."""
    import torch.nn.functional as F
    from mogt_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(41)
    x = torch.randn(rows, d_in, generator=gen, device=dev).bfloat16()
    wg = (torch.randn(hidden, d_in, generator=gen, device=dev) / d_in ** 0.5).bfloat16()
    wu = (torch.randn(hidden, d_in, generator=gen, device=dev) / d_in ** 0.5).bfloat16()
    w12 = torch.cat([wg, wu], 0)
    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    from mogt_amd import _lib

    lib = _lib.load()
    y1 = torch.empty(rows, hidden, device=dev, dtype=torch.bfloat16)

    def one_tile(i):   # the same GEMM with one tile per work-group (schedule 1)
        _lib.check(lib.mogt_swiglu_gate_fwd_cfg(x.data_ptr(), wg.data_ptr(), wu.data_ptr(), y1.data_ptr(), rows, d_in,
                                                hidden, d_in, hidden, _lib.MOGT_BF16, 1, stream.cuda_stream),
                   "mogt_swiglu_gate_fwd_cfg")

    runs = {"fused": lambda i: ops.swiglu_gate(x, wg, wu), "unfused": lambda i: ops.silu_mul(F.linear(x, w12)),
            "gemm": lambda i: F.linear(x, w12), "one_tile": one_tile}
    # the three are timed in turn, three rounds, best of each: the first
    # kernels of a process otherwise run before the clocks have settled
    best = {k: float("inf") for k in runs}
    for _ in range(3):
        for k, f in runs.items():
            best[k] = min(best[k], timer.time(f, steps, warmup))
    ms_fused, ms_unfused, ms_gemm = best["fused"], best["unfused"], best["gemm"]
    flop = 2.0 * rows * d_in * 2 * hidden
    return {"ms": ms_fused, "ms_unfused": ms_unfused, "ms_gemm_only": ms_gemm, "ms_one_tile": best["one_tile"],
            "tflops": flop / ms_fused / 1e9}


WGRAD_SHAPES = ((768, 768, "theta_read"), (800, 768, "phi_val + value gate"), (768, 3072, "w3"),
                (6144, 768, "w1; w2"))


def measure_wgrad(torch, steps, warmup, tokens=32768):
    """Weight gradients of the training path's linear layers (model_mogt.py:
    25-27, 57, 61) at configs[4]'s T = B * L: the split-K HIP GEMM
    (csrc/wgrad_gemm.hip, both of its launches) against the library GEMM that
    autograd calls for F.linear's weight (dY^T X), bf16 in, bf16 out.  With
    the tuned GEMM table when the caller activated it."""
    from mogt_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(43)
    stream = torch.cuda.current_stream(dev)
    timer = EventTimer(torch, stream)
    out = {}
    for d_out, d_in, what in WGRAD_SHAPES:
        dy = torch.randn(tokens, d_out, generator=gen, device=dev).bfloat16()
        x = torch.randn(tokens, d_in, generator=gen, device=dev).bfloat16()
        runs = {"hip": lambda i: ops.linear_wgrad(dy, x), "library": lambda i: dy.t().mm(x)}
        best = {k: float("inf") for k in runs}
        for _ in range(3):
            for k, f in runs.items():
                best[k] = min(best[k], timer.time(f, steps, warmup))
        flop = 2.0 * tokens * d_out * d_in
        splits = int(ops._lib.load().mogt_linear_wgrad_splits(tokens, d_out, d_in, 0, 0))
        out[f"{d_out}x{d_in}"] = {
            "layer": what, "us": round(best["hip"] * 1e3, 2), "library_us": round(best["library"] * 1e3, 2),
            "TFLOP/s": round(flop / best["hip"] / 1e9, 1), "splits": splits,
            "frac_bf16_mfma_peak": round(flop / best["hip"] / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)}
        del dy, x
    return out


def measure_lm_ce(torch, lib, steps, warmup, rows=4096, vocab=32000, L=32768, D=768, chunk=4096):
    """Chunked tied-head CE (chunked_lm_loss.py): the HIP cross-entropy rows on
    one [rows, vocab] fp32 logits block (forward reads it once; backward reads
    it and writes the gradient), and chunked_linear_cross_entropy forward +
    backward at B=1, L, D, vocab against the reference's torch ops."""
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn(rows, vocab, generator=gen, device=dev) * 4.0
    g = torch.empty_like(x)
    lab = torch.randint(0, vocab, (rows,), generator=gen, device=dev)
    loss = torch.empty(rows, device=dev)
    lse = torch.empty(rows, device=dev)
    scale = torch.ones(1, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def fwd(i):
        rc = lib.mogt_lm_ce_fwd(x.data_ptr(), vocab, 0, lab.data_ptr(), rows, vocab, -100, loss.data_ptr(),
                                lse.data_ptr(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    def bwd(i):
        rc = lib.mogt_lm_ce_bwd(x.data_ptr(), vocab, 0, lab.data_ptr(), lse.data_ptr(), rows, vocab, -100,
                                scale.data_ptr(), g.data_ptr(), vocab, 0, sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    timer = EventTimer(torch, stream)
    ms_f = timer.time(fwd, steps, warmup)
    ms_b = timer.time(bwd, steps, warmup)
    blk = rows * vocab * 4

    h = (torch.randn(1, L, D, generator=gen, device=dev) * 0.5).bfloat16().requires_grad_()
    w = (torch.randn(vocab, D, generator=gen, device=dev) * 0.02).requires_grad_()
    labels = torch.randint(0, vocab, (1, L), generator=gen, device=dev)

    def ours(i):
        h.grad = None
        w.grad = None
        chunked_linear_cross_entropy(h, w, labels, chunk_size=chunk).backward()

    def ref(i):
        _reference_chunked_ce_torch(torch, h.detach(), w.detach(), labels, chunk)

    ms_e2e = timer.time(ours, 3, 1)
    ms_ref = timer.time(ref, 3, 1)
    return {"fwd_ms": ms_f, "bwd_ms": ms_b, "fwd_gbs": blk / ms_f / 1e6, "bwd_gbs": 2 * blk / ms_b / 1e6,
            "e2e_ms": ms_e2e, "ref_ms": ms_ref}


def measure_coupled(torch, lib, ops, L, steps, warmup, r=16, c=48, tile=None):
    """Model-shaped coupled per-rank gate scan (config 2'): z fp32 [1,L,16],
    v bf16 [1,L,768] -> h fp32 [1,L,768]; ``tile`` forces a compiled tile."""
    from mogt_amd import synthetic

    dev = torch.device("cuda:0")
    z, v = synthetic.coupled_inputs(1, L, r, c, seed=3)
    zt = torch.from_numpy(z).to(dev)
    vt = torch.from_numpy(v).to(dev).bfloat16()
    sets = 4
    bufs = [(zt.clone(), vt.clone(), torch.empty(1, L, r * c, device=dev)) for _ in range(sets)]
    if tile is None:
        nbytes = lib.mogt_coupled_rank_scan_workspace_bytes(1, L, r, c, 1)
    else:
        nbytes = lib.mogt_diag_scan_workspace_bytes_cfg(1, L, r * c, *tile)
    ws = ops.workspace(nbytes, dev, "coupled", ("bench", L, r, c, tile))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def launch(i):
        zz, vv, hh = bufs[i % sets]
        if tile is None:
            rc = lib.mogt_coupled_rank_scan_fwd(zz.data_ptr(), vv.data_ptr(), hh.data_ptr(), 1, L, r, c, 1.0, 0, 1,
                                                0, ws.data_ptr(), ws.numel(), sh)
        else:
            rc = lib.mogt_coupled_rank_scan_fwd_cfg(zz.data_ptr(), vv.data_ptr(), hh.data_ptr(), 1, L, r, c, 1.0,
                                                    0, 1, 0, *tile, ws.data_ptr(), ws.numel(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    total = L * (r * 4 + r * c * 2 + r * c * 4)
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9}


def _cayley_transport_gpu(torch, n_seq, L, d, seed):
    """U_t = sigmoid(N(2,1)) * (I - W)^{-1} (I + W), W = T - T^T, T strictly upper
    N(0, 0.05): the configs[3] distribution, generated on the GPU (the Cayley
    solve on this library's connection-map kernel, which the GPU tests check
    against torch.linalg.solve; a few launches instead of torch's batched solve,
    so the inputs are made quickly also under a counter-collecting profiler)."""
    from mogt_amd import ops

    gen = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda:0")
    T = torch.triu(torch.randn(n_seq, L, d, d, generator=gen, device=dev) * 0.05, 1)
    W = T - T.transpose(-1, -2)
    del T
    gate = torch.sigmoid(torch.randn(n_seq, L, 1, 1, generator=gen, device=dev) + 2.0)
    U = ops.connection_map(W, "cayley", scale=2.0) * gate
    del W
    v = torch.randn(n_seq, L, d, 1, generator=gen, device=dev)
    k = torch.nn.functional.normalize(torch.randn(n_seq, L, 1, d, generator=gen, device=dev), dim=-1)
    return U, (v * k).contiguous(), v[..., 0].contiguous(), k[..., 0, :].contiguous()


def _unit_spectral(torch, U):
    """U / max(1, 1.1 * ||U||_2), the norm from power iteration on U^T U (a
    few dozen batched products rather than a batched SVD)."""
    G = torch.matmul(U.transpose(-1, -2).contiguous(), U)
    x = torch.ones(*U.shape[:-1], 1, device=U.device, dtype=U.dtype)
    x[..., 1::2, :] = -1.0
    for _ in range(30):
        x = torch.matmul(G, x)
        x = x / x.norm(dim=-2, keepdim=True)
    s = torch.matmul(G, x).norm(dim=-2, keepdim=True).sqrt()
    return U / (1.1 * s).clamp(min=1.0)


def measure_dense(torch, lib, ops, B, L, R, C, steps, warmup, cayley=False, sets=2, vk=False):
    """Dense U [B,L,R,R] fp32, V [B,L,R,C] fp32 -> H fp32 via the C ABI
    (chunk summaries, carries, output).  vk: B_t = v_t k_t^T from v [B,L,R] and
    k [B,L,C] formed in registers (mogt_affine_scan_vk_fwd)."""
    dev = torch.device("cuda:0")
    if vk:
        U0, _, v0, k0 = _cayley_transport_gpu(torch, B, L, R, seed=11)
        bufs = [(U0.clone(), v0.clone(), k0.clone(), torch.empty(B, L, R, C, device=dev)) for _ in range(sets)]
        del U0, v0, k0
        ws = ops.workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), dev)
        stream = torch.cuda.current_stream(dev)
        sh = stream.cuda_stream

        def launch_vk(i):
            u, vv, kk, h = bufs[i % sets]
            rc = lib.mogt_affine_scan_vk_fwd(u.data_ptr(), vv.data_ptr(), kk.data_ptr(), h.data_ptr(), None,
                                             B, L, R, C, 0, 0, ws.data_ptr(), ws.numel(), sh)
            if rc:
                raise RuntimeError(lib.mogt_last_error().decode())

        ms = EventTimer(torch, stream).time(launch_vk, steps, warmup)
        total = B * L * (R * R + R + C + R * C) * 4
        flops = B * L * (2 * R * R * C + 2 * R * C)   # U_t H_{t-1} + v_t k_t^T
        return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9,
                "tflops": flops / (ms * 1e-3) / 1e12}
    if cayley:
        U0, V0, _, _ = _cayley_transport_gpu(torch, B, L, R, seed=11)
    else:
        gen = torch.Generator(device="cuda").manual_seed(5)
        U0 = torch.eye(R, device=dev) + 0.05 * torch.randn(B, L, R, R, generator=gen, device=dev)
        U0 = _unit_spectral(torch, U0)
        V0 = torch.randn(B, L, R, C, generator=gen, device=dev)
    bufs = [(U0.clone(), V0.clone(), torch.empty(B, L, R, C, device=dev)) for _ in range(sets)]
    del U0, V0
    ws = ops.workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    fn = lib.mogt_affine_scan_fwd

    def launch(i):
        u, v, h = bufs[i % sets]
        rc = fn(u.data_ptr(), v.data_ptr(), h.data_ptr(), None, B, L, R, C, 0, 0,
                ws.data_ptr(), ws.numel(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    total = B * L * (R * R + 2 * R * C) * 4
    flops = B * L * (2 * R * R * C + R * C)      # U_t H_{t-1} + V_t
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9,
            "tflops": flops / (ms * 1e-3) / 1e12}


def measure_dense_backward(torch, lib, ops, B, L, R, C, steps, warmup, sets=2):
    """Backward of the dense scan (triton_scan.py:359-426, affine_scan.py:65-124)
    at one shape: the reverse-time scan G_t = X_t + U_{t+1}^T G_{t+1} alone
    (mogt_affine_scan_rev_fwd via the C ABI), and the whole gradient
    (forward recompute, reverse scan, dU_t = G_t H_{t-1}^T) through
    ops.affine_scan_grad; beside them the construction the reverse scan used
    to be built from (the reference's U_back = [I, flip(U^T[1:])], flipped
    inputs and outputs, the forward scan, dU by a batched matmul of copies)."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda").manual_seed(23)
    bufs = []
    for _ in range(sets):
        U = _unit_spectral(torch, torch.eye(R, device=dev) + 0.05 * torch.randn(B, L, R, R, generator=gen,
                                                                                   device=dev))
        bufs.append((U, torch.randn(B, L, R, C, generator=gen, device=dev),
                     torch.randn(B, L, R, C, generator=gen, device=dev), torch.empty(B, L, R, C, device=dev)))
    ws = ops.workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def rev(i):
        U, _, X, G = bufs[i % sets]
        rc = lib.mogt_affine_scan_rev_fwd(U.data_ptr(), X.data_ptr(), G.data_ptr(), B, L, R, C, ws.data_ptr(),
                                          ws.numel(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    def full(i):
        U, V, X, _ = bufs[i % sets]
        ops.affine_scan_grad(U, V, X)

    eye = torch.eye(R, device=dev).view(1, 1, R, R).expand(B, 1, R, R)
    zeros = torch.zeros(B, 1, R, C, device=dev)

    def glue(i):
        U, V, X, _ = bufs[i % sets]
        U_back = torch.cat([eye, U.transpose(-2, -1)[:, 1:].flip(1)], dim=1)
        G = ops.affine_scan(U_back, X.flip(1).contiguous()).flip(1)
        H = ops.affine_scan(U, V)
        M_prev = torch.cat([zeros, H[:, :-1]], dim=1)
        torch.matmul(G, M_prev.transpose(-2, -1).contiguous())

    t = EventTimer(torch, stream)
    ms_rev = t.time(rev, steps, warmup)
    ms_full = t.time(full, steps, warmup)
    ms_glue = t.time(glue, steps, warmup)
    rev_bytes = B * L * (R * R + 2 * R * C) * 4
    return {"rev_ms": ms_rev, "rev_gbs": rev_bytes / (ms_rev * 1e-3) / 1e9, "grad_ms": ms_full,
            "glue_ms": ms_glue}


def measure_generic(torch, lib, ops, B, L, R, C, steps, warmup, f64=True, sets=2):
    """The generic affine scan (mogt_affine_scan_generic_fwd): U, V, H in the
    state dtype (float64 or fp32), U = I + small noise scaled to norm <= 1."""
    dev = torch.device("cuda:0")
    dt = torch.float64 if f64 else torch.float32
    code = 2 if f64 else 0   # MOGT_F64 / MOGT_F32
    gen = torch.Generator(device="cuda").manual_seed(9)
    U0 = torch.eye(R, device=dev, dtype=dt) + (0.3 / R ** 0.5) * torch.randn(B, L, R, R, generator=gen,
                                                                             device=dev, dtype=dt)
    U0 = _unit_spectral(torch, U0)
    V0 = torch.randn(B, L, R, C, generator=gen, device=dev, dtype=dt)
    bufs = [(U0.clone(), V0.clone(), torch.empty(B, L, R, C, device=dev, dtype=dt)) for _ in range(sets)]
    del U0, V0
    ws = ops.workspace(lib.mogt_affine_scan_generic_workspace_bytes(B, L, R, C, 0, code), dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def launch(i):
        u, v, h = bufs[i % sets]
        rc = lib.mogt_affine_scan_generic_fwd(u.data_ptr(), v.data_ptr(), h.data_ptr(), None, B, L, R, C,
                                              code, code, code, 0, ws.data_ptr(), ws.numel(), sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    total = B * L * (R * R + 2 * R * C) * (8 if f64 else 4)
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9}


def measure_rank1(torch, lib, ops, steps, warmup, B=2, L=8192, H=12, d=64, sets=3, path=0):
    """rank-1 coupled write-forget scan with readout, bf16 I/O.
    path: 0 = the library's choice (one launch at this length), 2 = the
    three-launch form."""
    from mogt_amd import synthetic

    dev = torch.device("cuda:0")
    f, k, v, q = (torch.from_numpy(x).to(dev).bfloat16() for x in synthetic.rank1_inputs(B, L, H, d, seed=0))
    bufs = [(f.clone(), k.clone(), v.clone(), q.clone(), torch.empty_like(q)) for _ in range(sets)]
    nbytes = lib.mogt_rank1_coupled_scan_workspace_bytes(B, L, H, d)
    ws = ops.workspace(nbytes, dev, "rank1", ("bench", B, L, H)) if path in (0, 1) else ops.workspace(nbytes, dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    fn = lib.mogt_rank1_coupled_scan_fwd_cfg

    def launch(i):
        ff, kk, vv, qq, yy = bufs[i % sets]
        rc = fn(ff.data_ptr(), kk.data_ptr(), vv.data_ptr(), qq.data_ptr(), yy.data_ptr(), B, L, H, d,
                1, 1, 1, ws.data_ptr(), ws.numel(), path, sh)
        if rc:
            raise RuntimeError(lib.mogt_last_error().decode())

    ms = EventTimer(torch, stream).time(launch, steps, warmup)
    total = B * L * H * (4 * d * 2 + 2)   # f, k, v, q in + y out (bf16)
    return {"ms": ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9}


def measure_backbone(torch, layers, ffn_hidden, vocab, L, iters, warmup):
    """MOGT backbone forward (embedding -> blocks -> norm_f) under bf16 autocast
    and inference_mode, identity-coupled slot-addressed blocks, random N(0,0.02)
    weights including theta_read / ffn.w3 / value-gate weight (the reference's
    zero-inits would make every block the identity)."""
    from mogt_amd.model_mogt import MOGTModel, configure_coupled_gate

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = MOGTModel(vocab_size=vocab, d_model=768, num_layers=layers, r=16,
                      ffn_hidden=ffn_hidden).to(dev)
    configure_coupled_gate(model, zero_gate_weight=False)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" not in name and not name.endswith("bias"):
                prm.normal_(0.0, 0.02)
    model.eval()
    ids = torch.randint(0, vocab, (1, L), device=dev)

    def run():
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(ids)

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        out = run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / iters
    assert torch.isfinite(out).all()
    params = sum(p.numel() for p in model.parameters())
    del model
    return {"ms": round(ms, 3), "tokens_per_s": round(L * 1000.0 / ms),
            "peak_mem_mb": round(torch.cuda.max_memory_allocated(dev) / 2**20, 1),
            "params": params}


def backbone_lengths(torch, layers, ffn_hidden, vocab, lengths=(8192, 16384, 32768), iters=10, warmup=3):
    """The reference harness's length sweep (benchmark_backbone_throughput.py:92-131):
    per length a status ("ok" or "oom" when the forward runs out of device
    memory), ms, tokens/s and peak memory."""
    rows = {}
    for L in lengths:
        torch.cuda.empty_cache()
        try:
            r = measure_backbone(torch, layers, ffn_hidden, vocab, L, iters, warmup)
            rows[str(L)] = dict(status="ok", **{k: r[k] for k in ("ms", "tokens_per_s", "peak_mem_mb")})
        except torch.cuda.OutOfMemoryError as exc:
            torch.cuda.empty_cache()
            rows[str(L)] = {"status": "oom", "ms": None, "tokens_per_s": None, "error": str(exc)[:200]}
    return rows


def measure_backbone_train(torch, layers, ffn_hidden, vocab, L, iters, warmup, fused=True):
    """One training step of the backbone (forward + backward of a mean-square
    loss on its output, bf16 autocast, no optimizer): through the fused block
    path (every kernel with its backward) or forced onto the generic op-by-op
    path, same weights and inputs."""
    from mogt_amd.model_mogt import MOGTBlock, MOGTModel, configure_coupled_gate

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = MOGTModel(vocab_size=vocab, d_model=768, num_layers=layers, r=16,
                      ffn_hidden=ffn_hidden).to(dev)
    configure_coupled_gate(model, zero_gate_weight=False)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" not in name and not name.endswith("bias"):
                prm.normal_(0.0, 0.02)
    model.train()
    ids = torch.randint(0, vocab, (1, L), device=dev)
    orig = MOGTBlock.fused_path_ok
    if not fused:
        MOGTBlock.fused_path_ok = lambda self: False

    def step():
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = model(ids)
        loss = out.float().pow(2).mean()
        loss.backward()
        return loss

    try:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            loss = step()
        end.record()
        torch.cuda.synchronize()
    finally:
        MOGTBlock.fused_path_ok = orig
    ms = start.elapsed_time(end) / iters
    assert torch.isfinite(loss)
    del model
    return {"ms": round(ms, 3), "tokens_per_s": round(L * 1000.0 / ms),
            "peak_mem_mb": round(torch.cuda.max_memory_allocated(dev) / 2**20, 1)}


def cpu_baseline(L=32768, D=768):
    """Reference CPU PyTorch scan (sequential bmm loop, fp32 state) on the folded
    R=C=1 workload, on this host's cores."""
    import torch

    from mogt_amd import synthetic
    from oracle import torch_ref

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    a, b = synthetic.cfg2_inputs(L, seed=1)
    U, V = torch_ref.diag_as_affine(torch.from_numpy(a), torch.from_numpy(b))
    U, V = U.contiguous(), V.contiguous()
    torch_ref.affine_scan_sequential_torch(U[:, :256], V[:, :256])   # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch_ref.affine_scan_sequential_torch(U, V)
        times.append(time.perf_counter() - t0)
    t_seq = statistics.median(times)
    t0 = time.perf_counter()
    torch_ref.affine_scan_doubling_torch(U, V)
    t_dbl = time.perf_counter() - t0
    total = L * D * 12
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": total / t_seq / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full workload D=768 L={L} fp32, folded R=C=1 (768 sequences): sequential "
                   f"bmm loop median of 3 = {t_seq * 1e3:.1f} ms; doubling variant "
                   f"{t_dbl * 1e3:.1f} ms; {cpu}; torch {torch.__version__}"),
        "ms": t_seq * 1e3,
        "doubling_ms": t_dbl * 1e3,
    }


def read_traffic(name: str, manifest: dict):
    """HBM bytes per launch of the headline kernel, measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's counter reading) and kept
    as key=value lines in a profile.  The profile names the source hashes of the
    kernel it measured (``kernel_sources=``); the figure is used only when they
    equal the loaded library's, i.e. the profile came from this kernel's build.
    Returns (bytes or None, provenance dict)."""
    path = ROOT / "profiles" / name
    info = {"file": f"profiles/{name}"}
    if not path.exists():
        info["status"] = "missing"
        return None, info
    kv = {}
    for line in path.read_text().splitlines():
        if "=" in line and not line.lstrip().startswith(("#", "|", "`")):
            k, v = line.split("=", 1)
            kv[k.strip()] = v.strip()
    srcs = dict(item.split(":", 1) for item in kv.get("kernel_sources", "").split(",") if ":" in item)
    stale = sorted(k for k, h in srcs.items() if manifest.get(k) != h)
    if not srcs or stale:
        info["status"] = f"refused: profile taken from other sources ({', '.join(stale) or 'none named'})"
        return None, info
    try:
        traffic = float(kv["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        info["status"] = "no hbm_bytes_per_launch"
        return None, info
    info.update(status="matches this build", kernel_sources=kv["kernel_sources"],
                profile_avg_us=float(kv.get("avg_us", "nan")))
    return traffic, info


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the scan is "
              "single-GPU in this build.", file=sys.stderr)
        sys.exit(2)
    import torch

    import mogt_amd
    from mogt_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    lib = mogt_amd._lib.load()
    torch.cuda.init()
    tile = tuple(int(x) for x in args.tile.split(",")) if args.tile else None

    if args.calib_copy:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy of {n} bytes done (x5)")

    if args.sweep:
        for L in (8192, 16384, 32768):
            for dt in (torch.float32, torch.bfloat16):
                for t in mogt_amd._lib.diag_tiles(0 if dt == torch.float32 else 1):
                    r = measure_diag(torch, lib, ops, L, dt, dt, args.steps, args.warmup, tile=t)
                    log(f"sweep L={L} {dt} tile={t}: {r['ms'] * 1e3:.1f} us  {r['gbs']:.0f} GB/s "
                        f"({r['gbs'] / HBM_PEAK_GBS:.1%} of peak)")
            for t in mogt_amd._lib.diag_tiles(2):
                r = measure_coupled(torch, lib, ops, L, args.steps, args.warmup, tile=t)
                log(f"sweep L={L} coupled tile={t}: {r['ms'] * 1e3:.1f} us  {r['gbs']:.0f} GB/s "
                    f"({r['gbs'] / HBM_PEAK_GBS:.1%} of peak)")

    log("headline: diag scan fp32 B=1 D=768 L=32768")
    head = measure_diag(torch, lib, ops, 32768, torch.float32, torch.float32, args.steps,
                        args.warmup, tile=tile)
    log(f"headline: {head['ms'] * 1e3:.1f} us/launch, {head['gbs']:.0f} GB/s")

    extras = {}
    only = args.only
    if not args.no_extras and only != {"diag"}:
        full = "all" in only
        if full:
            for L in (8192, 16384):
                r = measure_diag(torch, lib, ops, L, torch.float32, torch.float32, args.steps,
                                 args.warmup)
                extras[f"diag_fp32_L{L}"] = {"us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                                             "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}
            for L in (8192, 32768):
                r = measure_diag(torch, lib, ops, L, torch.bfloat16, torch.bfloat16, args.steps,
                                 args.warmup)
                extras[f"diag_bf16_L{L}"] = {"us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                                             "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}
            for L in (8192, 32768):
                re_ = measure_diag_op(torch, L, args.steps, args.warmup, graph=False)
                rg_ = measure_diag_op(torch, L, args.steps, args.warmup, graph=True)
                rg16 = measure_diag_op(torch, L, args.steps, args.warmup, graph=True, per_graph=16)
                extras[f"diag_fp32_L{L}_op_level"] = {
                    "eager_us": round(re_["ms"] * 1e3, 2), "graph_us": round(rg_["ms"] * 1e3, 2),
                    "graph_nodes": rg_["graph_nodes"], "graph16_us": round(rg16["ms"] * 1e3, 2),
                    "graph16_nodes": rg16["graph_nodes"],
                    "note": "mogt_amd.diag_scan per call (eager: input checks, output allocation, C-ABI launch; "
                            "the custom-op dispatch is taken only under autograd or tracing), the same call "
                            "captured alone in a HIP graph and replayed (graph_nodes: nodes per captured graph; "
                            "the replay pays the runtime's graph launch), and 16 calls captured in one graph "
                            "(graph16_us: replay time per call)"}
            r = measure_diag_rev(torch, lib, ops, 32768, args.steps, args.warmup)
            extras["diag_rev_fp32_L32768"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "note": "backward reverse scan G_t = dH_t + a_{t+1} G_{t+1} at the headline shape"}
        if full or "coupled" in only:
            log("extras: coupled mixer scan")
            r = measure_coupled(torch, lib, ops, 32768, args.steps, args.warmup)
            extras["coupled_rank_scan_r16c48_L32768"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "note": "z fp32 [1,L,16] + v bf16 [1,L,768] -> h fp32; model-shaped 2' case"}
        if full or "rank1" in only:
            log("extras: rank-1 scan (configs[2])")
            r = measure_rank1(torch, lib, ops, args.steps, args.warmup)
            r3 = measure_rank1(torch, lib, ops, args.steps, args.warmup, path=2)
            extras["rank1_coupled_cfg3_b2_h12_d64_L8192_bf16"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "three_launch_us": round(r3["ms"] * 1e3, 2),
                "note": "BASELINE configs[2]; algorithmic bytes 101.1 MB (f,k,v,q in, y out); us: one launch "
                        "(carries exchanged between work-groups), three_launch_us: summaries, carries, outputs"}
        if full or "dense" in only:
            log("extras: dense scan (core shape, configs[3])")
            r = measure_dense(torch, lib, ops, 1, 32768, 16, 48, max(5, args.steps // 5), 2)
            extras["dense_affine_r16_c48_L32768"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "vs_reference_triton_hybrid_L4_5.48ms": round(REF_TRITON_CORE_MS_L4 / r["ms"], 1),
                "note": "U [1,L,16,16] + V [1,L,16,48] fp32 -> H fp32; the reference's core-operator "
                        "shape (its 5.48 ms was measured on an NVIDIA L4)"}
            r = measure_dense(torch, lib, ops, 8, 16384, 32, 32, max(3, args.steps // 10), 1,
                              cayley=True, sets=2)
            extras["dense_cayley_cfg4_h8_d32_L16384"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(r["tflops"], 2), "frac_fp32_matrix_peak": round(r["tflops"] / 157.3, 4),
                "note": "BASELINE configs[3]: U=gate*Cayley(W) [8,L,32,32], V=v k^T [8,L,32,32] fp32"}
            r = measure_dense(torch, lib, ops, 8, 16384, 32, 32, max(3, args.steps // 10), 1, sets=2, vk=True)
            extras["dense_cayley_cfg4_vk_h8_d32_L16384"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "TFLOP/s": round(r["tflops"], 2), "frac_fp32_matrix_peak": round(r["tflops"] / 157.3, 4),
                "note": "configs[3] with B_t = v_t k_t^T formed in registers (dense_scan(A, v, k)): "
                        "U [8,L,32,32] + v, k [8,L,32] in, S fp32 out"}
        if full or "dense" in only:
            log("extras: dense backward, generic scan")
            r = measure_dense_backward(torch, lib, ops, 1, 32768, 16, 48, max(5, args.steps // 5), 2)
            extras["dense_affine_r16_c48_L32768_backward"] = {
                "reverse_scan_us": round(r["rev_ms"] * 1e3, 2), "reverse_scan_GB/s": round(r["rev_gbs"], 1),
                "reverse_scan_frac": round(r["rev_gbs"] / HBM_PEAK_GBS, 4),
                "grad_us": round(r["grad_ms"] * 1e3, 2), "previous_glue_path_us": round(r["glue_ms"] * 1e3, 2),
                "note": "backward of the core-operator shape: reverse_scan = G_t = dH_t + U_{t+1}^T G_{t+1} "
                        "alone (U, dH in, G out: 7168 B/step); grad = forward recompute + reverse scan + "
                        "dU_t = G_t H_{t-1}^T (affine_scan_grad); previous_glue_path = the reversed-copy "
                        "construction it replaces (cat/flip of U^T and dH, forward scan, flip, batched matmul)"}
            r = measure_generic(torch, lib, ops, 1, 32768, 16, 48, max(3, args.steps // 10), 1)
            extras["generic_affine_f64_r16_c48_L32768"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "note": "float64 state and I/O (affine_scan_sequential(..., state_dtype=torch.float64)) on the "
                        "generic scan; latency-bound (256 + 127 + 256 dependent steps), not an HBM roofline case"}
            r = measure_generic(torch, lib, ops, 24, 2048, 64, 64, max(3, args.steps // 10), 1, f64=False)
            extras["generic_affine_f32_r64_c64_b24_L2048"] = {
                "us": round(r["ms"] * 1e3, 2), "GB/s": round(r["gbs"], 1),
                "note": "R = 64 (above the matrix-core pipeline's 32): fp32 on the generic scan"}
        if full:
            log("extras: connection maps, cross-entropy rows")
            for impl in ("matrix_exp", "cayley"):
                r = measure_connection_map(torch, lib, ops, impl, 32768, 16, args.steps, args.warmup)
                extras[f"connection_map_{impl}_r16_n32768"] = {
                    "us": round(r["ms"] * 1e3, 2), "torch_us": round(r["ms_torch"] * 1e3, 2),
                    "note": "U = f(A) for 32768 skew 16x16 generators (one MOGT layer at L = 32768); "
                            "torch_us: torch.matrix_exp / torch.linalg.solve on the same GPU inputs"}
            r = measure_lm_ce(torch, lib, args.steps, args.warmup)
            extras["lm_ce_rows_4096x32000_fp32"] = {
                "fwd_us": round(r["fwd_ms"] * 1e3, 2), "fwd_GB/s": round(r["fwd_gbs"], 1),
                "fwd_frac": round(r["fwd_gbs"] / HBM_PEAK_GBS, 4),
                "bwd_us": round(r["bwd_ms"] * 1e3, 2), "bwd_GB/s": round(r["bwd_gbs"], 1),
                "bwd_frac": round(r["bwd_gbs"] / HBM_PEAK_GBS, 4),
                "note": "cross-entropy rows of one logits block: forward reads it once (lse, loss), "
                        "backward reads it and writes the softmax gradient"}
            extras["chunked_linear_ce_L32768_d768_v32000_fwd_bwd_ms"] = {
                "ms": round(r["e2e_ms"], 2), "reference_torch_ops_ms": round(r["ref_ms"], 2),
                "note": "chunked_linear_cross_entropy fwd+bwd, chunk 4096, bf16 hidden, fp32 tied weight; "
                        "the GEMMs are the BLAS library's in both; reference = chunked_lm_loss.py's "
                        "torch ops on the same GPU"}
        if full or "swiglu" in only:
            log("extras: fused SwiGLU GEMM")
            r = measure_swiglu(torch, args.steps, args.warmup)
            extras["swiglu_gate_gemm_32768x768_to_3072_bf16"] = {
                "us": round(r["ms"] * 1e3, 2), "TFLOP/s": round(r["tflops"], 1),
                "frac_bf16_mfma_peak": round(r["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                "unfused_us": round(r["ms_unfused"] * 1e3, 2), "library_gemm_only_us": round(r["ms_gemm_only"] * 1e3, 2),
                "one_tile_per_workgroup_us": round(r["ms_one_tile"] * 1e3, 2),
                "note": "FFN gate silu(x w1^T) * (x w2^T) as one GEMM with the gate in its epilogue (persistent "
                        "schedule; one_tile_per_workgroup = the same tiles one per work-group) vs the "
                        "library GEMM against [w1; w2] + the silu_mul row kernel (model_mogt.py:29-30)"}
        if full or "wgrad" in only:
            from mogt_amd import gemm_tuning

            log("extras: weight-gradient GEMMs")
            tuned = gemm_tuning.use_tuned_gemms()
            extras["linear_wgrad_T32768_bf16"] = dict(
                measure_wgrad(torch, args.steps, args.warmup), tuned_gemm_table=tuned,
                note="dW = dY^T X of the training path's linear layers at T = 32768 tokens: the split-K HIP "
                     "GEMM (fp32 partials per token slice, summed in slice order, rounded once) vs the "
                     "library GEMM autograd calls (tuned table)")
            if tuned:
                gemm_tuning.default_gemms()
        if full or "backbone" in only:
            from mogt_amd import gemm_tuning

            # the libraries' default GEMM choice first, then the tuned table
            # (mogt_amd/tuning/gemm_gfx950.csv); both are reported
            log("extras: backbone forward (default GEMMs)")
            d4 = measure_backbone(torch, 4, 3072, 32000, 32768, 10, 3)
            d2 = measure_backbone(torch, 2, None, 4096, 32768, 10, 3)
            log("extras: backbone training step (default GEMMs)")
            dt = measure_backbone_train(torch, 4, 3072, 32000, 32768, 5, 10, fused=True)
            tuned = gemm_tuning.use_tuned_gemms()
            log(f"extras: backbone forward, tuned GEMM table {tuned}")
            r = measure_backbone(torch, 4, 3072, 32000, 32768, 10, 3) if tuned else d4
            extras["mogt_backbone_4layer_d768_L32768_bf16_ms"] = dict(
                r, ffn_hidden=3072, vocab=32000, default_gemms_ms=d4["ms"], tuned_gemm_table=tuned,
                mfma_frac=round(2.174e12 / (r["ms"] * 1e-3) / (MFMA_BF16_PEAK_TFLOPS * 1e12), 4),
                note="BASELINE configs[4]: 4 layers, 4x gated MLP, bf16 autocast; target < 77.56 ms; "
                     "ms with the tuned GEMM table, default_gemms_ms with the libraries' own choice; "
                     "mfma_frac = 2.174 TFLOP of GEMMs / time / 2.5 PFLOP/s")
            r = measure_backbone(torch, 2, None, 4096, 32768, 10, 3) if tuned else d2
            extras["mogt_backbone_2layer_refffn_L32768_bf16_ms"] = dict(
                r, ffn_hidden=2048, vocab=4096, default_gemms_ms=d2["ms"], tuned_gemm_table=tuned,
                note="like-for-like with the reference's 77.56 ms (2 layers, FFN 2048, NVIDIA L4)")
            log("extras: backbone length sweep")
            extras["mogt_backbone_length_sweep"] = {
                "4layer_ffn3072_vocab32000": backbone_lengths(torch, 4, 3072, 32000),
                "2layer_refffn_vocab4096": backbone_lengths(torch, 2, None, 4096),
                "reference_2layer_L4_ms": {"8192": 14.07, "16384": 37.88, "32768": 77.56},
                "tuned_gemm_table": tuned,
                "note": "forward, bf16 autocast, inference mode, B = 1, tuned GEMM table when accepted; "
                        "status 'oom' where the forward runs out of device memory "
                        "(benchmark_backbone_throughput.py:92-131)"}
            # 10 warm-up steps: the first training steps of a process run slow for
            # ~0.2 s of wall time (measured 27 ms/step with 2-5 warm-up steps, 14.5
            # with 10-20), independent of which path runs first
            log("extras: backbone training step (tuned GEMMs, generic path)")
            rf = measure_backbone_train(torch, 4, 3072, 32000, 32768, 5, 10, fused=True) if tuned else dt
            rg = measure_backbone_train(torch, 4, 3072, 32000, 32768, 5, 10, fused=False)
            extras["mogt_backbone_4layer_d768_L32768_bf16_train_step_ms"] = dict(
                rf, default_gemms_ms=dt["ms"], tuned_gemm_table=tuned,
                generic_path_ms=rg["ms"], generic_path_peak_mem_mb=rg["peak_mem_mb"],
                note="forward + backward (mean-square loss on the backbone output, no optimizer), "
                     "bf16 autocast; fused block path, whose linear layers take their weight gradients from "
                     "the split-K HIP GEMM (default_gemms_ms: the libraries' own choice for the other "
                     "GEMMs) vs the generic op-by-op path on the same weights")
            if tuned:
                gemm_tuning.default_gemms()
        log(f"extras: {json.dumps(extras)}")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (reference sequential torch scan restated, host cores)")
        cpu = cpu_baseline()
        log(f"cpu baseline: {cpu['ms']:.0f} ms ({cpu['value']:.3f} GB/s)")

    # every single-pass scan above ran on a cached workspace: a look-back wait
    # that gave up would have poisoned its outputs with NaN; refuse the numbers
    give_ups = ops.workspace_faults()
    if give_ups:
        print(f"bench.py: {give_ups} look-back wait(s) gave up; the measured scans are invalid",
              file=sys.stderr)
        sys.exit(3)

    traffic, traffic_info = read_traffic(HEADLINE_PROFILE, mogt_amd._lib.build_manifest())
    achieved = head["gbs"]
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "tokens_per_s": round(32768 / (head["ms"] * 1e-3)),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded PCG64; a=sigmoid(N(3,1)), b~N(0,0.5))",
        "config": {
            "workload": "diag_affine_scan B=1 D=768 L=32768 fp32 I/O, fp32 state "
                        "(BASELINE configs[1])",
            "batch": 1, "features": 768, "seq_len": 32768,
            "tile": list(tile) if tile else "default",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": ({k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")}
                         if cpu else None),
        "scan_core_us": round(head["ms"] * 1e3, 3),
        "lookback_give_ups": give_ups,
        "build_id": mogt_amd._lib.build_id(),
        "traffic_profile": traffic_info,
        "reference_triton_core_ms_L4": REF_TRITON_CORE_MS_L4,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
