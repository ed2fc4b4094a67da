"""PyTorch custom ops (``torch.ops.mogt.*``) over the HIP C-ABI library.

Each op validates its inputs with the reference's ``ValueError`` conditions,
allocates outputs through the PyTorch caching allocator, and enqueues the HIP
kernel on the current stream.  The native library never allocates: single-pass
scans get a persistent, zero-initialised workspace per (device, stream) that
the kernels leave reusable after every launch.
"""
from __future__ import annotations

import ctypes
import os
import threading
import warnings

import torch
import torch.nn.functional as F

from . import _lib

_DTYPE_CODE = {torch.float32: _lib.MOGT_F32, torch.bfloat16: _lib.MOGT_BF16}

_ws_lock = threading.Lock()
_ws_cache: dict[tuple[int, int, str], torch.Tensor] = {}
# Workspaces replaced by a larger one.  They are kept alive for the life of the
# process: a HIP graph captured earlier still holds their address, and freeing
# them would let the allocator hand the memory to another tensor that the
# graph's replays would then overwrite.  Growth is geometric, so the retired
# buffers together are smaller than the live one.
_ws_retired: list[torch.Tensor] = []
_ws_retired_lookback: list[torch.Tensor] = []   # the look-back family ones among them
# layout of the launches on each look-back workspace, and whether a captured
# graph uses the buffer (pinned to that layout)
_ws_layout: dict[tuple[int, int, str], tuple] = {}
WS_HDR_BYTES = 256   # epoch and give-up counter (common.h); never cleared

# Checked mode: after every single-pass scan, read the workspace's give-up
# counter (a device synchronisation) and raise if it counted a new give-up.
CHECK_WORKSPACE = os.environ.get("MOGT_CHECK_WORKSPACE", "0") not in ("", "0")


class WorkspaceFault(RuntimeError):
    """A single-pass scan's look-back gave up: its output is not valid."""


def dtype_code(dt: torch.dtype, what: str) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"{what}: dtype {dt} not supported (float32 or bfloat16)") from None


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# Workspace families.  "plain" holds data that the kernels read back only in
# launches that wrote it (dense / generic / three-launch rank-1 scans: chunk
# products, carries, states).  The others hold tagged words of the look-back
# protocol, which a launch accepts when their tag carries the workspace's
# current epoch; a family never shares its buffer with plain data, and a
# launch whose layout differs from the buffer's previous one clears everything
# past the header first (or, if a captured graph uses the buffer, takes a new
# one), so a word it reads is either zero, an older tag or its own.
LOOKBACK_FAMILIES = frozenset({"diag", "diag_rev", "coupled", "coupled_rev", "rank1"})


def workspace(nbytes: int, device: torch.device, family: str = "plain", layout: tuple | None = None
              ) -> torch.Tensor:
    """Zero-initialised scratch of at least ``nbytes`` for the current stream.

    One buffer per (device, stream, family) keeps concurrent streams and the
    kernel families apart.  Look-back families (``LOOKBACK_FAMILIES``) pass the
    launch's ``layout`` (its shape, dtypes and tile).  Kernels using the
    look-back protocol leave the buffer reusable after every launch, so
    launches of one layout never clear it; a launch of another layout first
    clears bytes ``[256, nbytes)`` with a fill kernel.  A buffer that a graph
    capture used is pinned to that layout: a later launch of another layout on
    the stream gets a new buffer, and the pinned one stays alive (and
    untouched by other layouts) for the graph's replays.
    """
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           _stream_handle(device), family)
    lookback = family in LOOKBACK_FAMILIES
    if lookback and layout is None:
        raise ValueError(f"workspace family {family!r} needs the launch's layout")
    capturing = lookback and torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        buf = _ws_cache.get(key)
        state = _ws_layout.get(key)          # (layout, pinned) of the buffer's launches
        want = tuple(layout) if lookback else None
        moved = lookback and buf is not None and state is not None and state[0] != want and state[1]
        if buf is None or buf.numel() < nbytes or moved:
            size = max(int(nbytes), 1 << 16)
            if buf is not None:
                if buf.numel() >= nbytes:
                    size = buf.numel()
                else:
                    size = max(size, 2 * buf.numel())
                _ws_retired.append(buf)
                if lookback:
                    _ws_retired_lookback.append(buf)
            # a new buffer starts from epoch 0 with every word zero; it is a
            # normal tensor even when made under inference mode, so that later
            # calls outside that mode may still clear it in place
            with torch.inference_mode(False):
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
            state = None
        if lookback:
            if state is not None and state[0] != want and nbytes > WS_HDR_BYTES:
                buf[WS_HDR_BYTES:nbytes].zero_()
            _ws_layout[key] = (want, capturing or (state is not None and state[0] == want and state[1]))
        return buf


def _faults_of(buf: torch.Tensor) -> int:
    lib = _lib.load()
    count = ctypes.c_uint32(0)
    rc = lib.mogt_workspace_faults(buf.data_ptr(), buf.numel(), ctypes.byref(count),
                                   _stream_handle(buf.device))
    _lib.check(rc, "mogt_workspace_faults")
    return int(count.value)


def workspace_faults() -> int:
    """Number of bounded look-back waits that gave up, summed over every cached
    look-back workspace, live or retired (read through
    ``mogt_workspace_faults``; plain buffers have no header, their first bytes
    are data).  Always 0 unless the protocol was violated, in which case the
    affected outputs also hold NaN.  Synchronises the streams involved."""
    with _ws_lock:
        bufs = [b for k, b in _ws_cache.items() if k[2] in LOOKBACK_FAMILIES] + list(_ws_retired_lookback)
    return sum(_faults_of(b) for b in bufs)


_ws_faults_seen: dict[int, int] = {}


def _new_faults(ws: torch.Tensor) -> int:
    """Give-ups counted on ``ws`` since the last call for it (synchronises)."""
    n = _faults_of(ws)
    with _ws_lock:
        seen = _ws_faults_seen.get(ws.data_ptr(), 0)
        _ws_faults_seen[ws.data_ptr()] = n
    return n - seen


def _checked(ws: torch.Tensor, what: str) -> None:
    """In checked mode (MOGT_CHECK_WORKSPACE=1) raise if the launch that just
    used ``ws`` gave up a look-back wait."""
    if CHECK_WORKSPACE and not torch.cuda.is_current_stream_capturing():
        n = _new_faults(ws)
        if n:
            raise WorkspaceFault(f"{what}: {n} look-back wait(s) gave up; the output is invalid (NaN)")


def _direct(*tensors: torch.Tensor) -> bool:
    """Whether a public op may call its implementation directly: a plain eager
    call on real tensors with no autograd recording and no compiler tracing,
    where the custom-op dispatch would only add host time (about 13 us per
    call, more than a short scan's kernel).  Everything else goes through
    ``torch.ops.mogt.*`` (autograd, fake tensors, torch.compile)."""
    if torch.compiler.is_compiling():
        return False
    grad = torch.is_grad_enabled()
    return all(type(t) is torch.Tensor and not (grad and t.requires_grad) for t in tensors)


def require_cuda(what: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(f"{what} requires CUDA tensors")


# ---------------------------------------------------------------------------
# diag_scan: h_t = a_t * h_{t-1} + b_t over [B, L, D]
# ---------------------------------------------------------------------------
def _diag_scan_launch(a: torch.Tensor, b: torch.Tensor, h: torch.Tensor,
                      prefix: torch.Tensor | None,
                      cfg: tuple[int, int, int, int] | None = None) -> None:
    lib = _lib.load()
    B, L, D = a.shape
    in_code = dtype_code(a.dtype, "diag_scan")
    out_code = dtype_code(h.dtype, "diag_scan")
    if cfg is None:
        nbytes = lib.mogt_diag_scan_workspace_bytes(B, L, D, in_code)
    else:
        nbytes = lib.mogt_diag_scan_workspace_bytes_cfg(B, L, D, *cfg)
    ws = workspace(nbytes, a.device, "diag", (B, L, D, in_code, cfg))
    pre = prefix.data_ptr() if prefix is not None else None
    stream = _stream_handle(a.device)
    if cfg is None:
        rc = lib.mogt_diag_scan_fwd(a.data_ptr(), b.data_ptr(), h.data_ptr(), pre, B, L, D,
                                    in_code, out_code, ws.data_ptr(), ws.numel(), stream)
    else:
        rc = lib.mogt_diag_scan_fwd_cfg(a.data_ptr(), b.data_ptr(), h.data_ptr(), pre, B, L, D,
                                        in_code, out_code, cfg[0], cfg[1], cfg[2], cfg[3],
                                        ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "mogt_diag_scan_fwd")
    _checked(ws, "mogt_diag_scan_fwd")


def _check_diag_inputs(a: torch.Tensor, b: torch.Tensor) -> None:
    require_cuda("diag_scan", a, b)
    if a.ndim != 3 or b.ndim != 3:
        raise ValueError("a and b must be rank-3 tensors [B, L, D]")
    if a.shape != b.shape:
        raise ValueError("a and b must have the same shape [B, L, D]")
    if a.dtype != b.dtype:
        raise ValueError("a and b must have the same dtype")
    dtype_code(a.dtype, "diag_scan")


def _diag_scan_impl(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    a = a.contiguous()
    b = b.contiguous()
    h = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    _diag_scan_launch(a, b, h, None)
    return h


_diag_scan_op = torch.library.custom_op("mogt::diag_scan", _diag_scan_impl, mutates_args=())


@_diag_scan_op.register_fake
def _(a, b, out_dtype):
    return a.new_empty(a.shape, dtype=out_dtype)


def _diag_scan_prefix_impl(a: torch.Tensor, b: torch.Tensor,
                           out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    a = a.contiguous()
    b = b.contiguous()
    h = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    pre = torch.empty(a.shape, dtype=out_dtype, device=a.device)
    _diag_scan_launch(a, b, h, pre)
    return pre, h


_diag_scan_prefix_op = torch.library.custom_op("mogt::diag_scan_prefix", _diag_scan_prefix_impl, mutates_args=())


@_diag_scan_prefix_op.register_fake
def _(a, b, out_dtype):
    return a.new_empty(a.shape, dtype=out_dtype), a.new_empty(a.shape, dtype=out_dtype)


@torch.library.custom_op("mogt::diag_scan_rev", mutates_args=())
def _diag_scan_rev_op(a: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """G_t = g_t + a_{t+1} G_{t+1} (G_L = 0) in fp32: the reverse-time scan of
    the diagonal scan's backward."""
    lib = _lib.load()
    a = a.to(torch.float32).contiguous()
    g = g.to(torch.float32).contiguous()
    B, L, D = a.shape
    out = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    ws = workspace(lib.mogt_diag_scan_workspace_bytes(B, L, D, _lib.MOGT_F32), a.device, "diag_rev", (B, L, D))
    rc = lib.mogt_diag_scan_rev_fwd(a.data_ptr(), g.data_ptr(), out.data_ptr(), B, L, D,
                                    ws.data_ptr(), ws.numel(), _stream_handle(a.device))
    _lib.check(rc, "mogt_diag_scan_rev_fwd")
    _checked(ws, "mogt_diag_scan_rev_fwd")
    return out


@_diag_scan_rev_op.register_fake
def _(a, g):
    return a.new_empty(a.shape, dtype=torch.float32)


def _shift_prev(h: torch.Tensor) -> torch.Tensor:
    """h_{t-1} with h_{-1} = 0 along dim 1."""
    out = torch.zeros_like(h)
    out[:, 1:] = h[:, :-1]
    return out


def _diag_scan_setup(ctx, inputs, output):
    a, b, _ = inputs
    ctx.save_for_backward(a, b)


def _diag_scan_backward(ctx, grad_h):
    """Reverse scan on the GPU (affine_scan.py:65-124 for R = C = 1): G = dH +
    a_{t+1} G_{t+1}; db = G; da_t = G_t h_{t-1}, with h recomputed in fp32 as
    the reference's backward does (triton_scan.py:370-378)."""
    a, b = ctx.saved_tensors
    need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    G = torch.ops.mogt.diag_scan_rev(a, grad_h)
    da = db = None
    if need_a:
        h = torch.ops.mogt.diag_scan(a.float().contiguous(), b.float().contiguous(), torch.float32)
        da = (G * _shift_prev(h)).to(a.dtype)
    if need_b:
        db = G.to(b.dtype)
    return da, db, None


torch.library.register_autograd("mogt::diag_scan", _diag_scan_backward, setup_context=_diag_scan_setup)


def diag_scan(a: torch.Tensor, b: torch.Tensor, *, out_dtype: torch.dtype | None = None,
              return_prefix: bool = False):
    """h_t = a_t * h_{t-1} + b_t (h_0 = 0) over ``[B, L, D]`` on the GPU.

    fp32 state and arithmetic; ``out_dtype`` defaults to ``b.dtype`` (the
    reference's ``output_dtype or V.dtype``, affine_scan.py:34).  With
    ``return_prefix`` also returns ``prod_{s<=t} a_s`` first, like the
    reference's ``(U_prefix, H)`` pair (affine_scan.py:57-62).
    """
    _check_diag_inputs(a, b)
    out_dtype = out_dtype or b.dtype
    dtype_code(out_dtype, "diag_scan")
    if _direct(a, b):
        return _diag_scan_prefix_impl(a, b, out_dtype) if return_prefix else _diag_scan_impl(a, b, out_dtype)
    if return_prefix:
        return torch.ops.mogt.diag_scan_prefix(a, b, out_dtype)
    return torch.ops.mogt.diag_scan(a, b, out_dtype)


# ---------------------------------------------------------------------------
# coupled_rank_scan: MOGT mixer scan with identity connection and rank gate
# ---------------------------------------------------------------------------
def _coupled_rank_scan_impl(z: torch.Tensor, v: torch.Tensor, rank: int, damping: float,
                            out_dtype: torch.dtype) -> torch.Tensor:
    lib = _lib.load()
    z = z.contiguous()
    v = v.contiguous()
    B, L, D = v.shape
    C = D // rank
    h = torch.empty(v.shape, dtype=out_dtype, device=v.device)
    zc = dtype_code(z.dtype, "coupled_rank_scan")
    vc = dtype_code(v.dtype, "coupled_rank_scan")
    oc = dtype_code(out_dtype, "coupled_rank_scan")
    nbytes = lib.mogt_coupled_rank_scan_workspace_bytes(B, L, rank, C, vc)
    ws = workspace(nbytes, v.device, "coupled", ("plain", B, L, rank, C, vc))
    rc = lib.mogt_coupled_rank_scan_fwd(z.data_ptr(), v.data_ptr(), h.data_ptr(), B, L, rank, C,
                                        float(damping), zc, vc, oc, ws.data_ptr(), ws.numel(),
                                        _stream_handle(v.device))
    _lib.check(rc, "mogt_coupled_rank_scan_fwd")
    _checked(ws, "mogt_coupled_rank_scan_fwd")
    return h


_coupled_rank_scan_op = torch.library.custom_op("mogt::coupled_rank_scan", _coupled_rank_scan_impl,
                                                mutates_args=())


@_coupled_rank_scan_op.register_fake
def _(z, v, rank, damping, out_dtype):
    return v.new_empty(v.shape, dtype=out_dtype)


@torch.library.custom_op("mogt::coupled_scan_rev", mutates_args=())
def _coupled_scan_rev_op(z: torch.Tensor, grad_h: torch.Tensor, rank: int, damping: float) -> torch.Tensor:
    """G_t = dH_t + a_{t+1} G_{t+1} with a = damping (1 - sigmoid(z)) per rank,
    the decay formed from the gate logits inside the reverse scan."""
    lib = _lib.load()
    z = z.contiguous()
    g = grad_h.contiguous().to(torch.float32)
    B, L, D = g.shape
    out = torch.empty_like(g)
    nbytes = lib.mogt_coupled_rank_scan_rev_workspace_bytes(B, L, rank, D // rank)
    ws = workspace(nbytes, g.device, "coupled_rev", (B, L, rank, D // rank))
    rc = lib.mogt_coupled_rank_scan_rev_fwd(z.data_ptr(), g.data_ptr(), out.data_ptr(), B, L, rank, D // rank,
                                            float(damping), dtype_code(z.dtype, "coupled_scan_rev"), ws.data_ptr(),
                                            ws.numel(), _stream_handle(g.device))
    _lib.check(rc, "mogt_coupled_rank_scan_rev_fwd")
    _checked(ws, "mogt_coupled_rank_scan_rev_fwd")
    return out


@_coupled_scan_rev_op.register_fake
def _(z, grad_h, rank, damping):
    return grad_h.new_empty(grad_h.shape, dtype=torch.float32)


@torch.library.custom_op("mogt::coupled_grad", mutates_args=())
def _coupled_grad_op(G: torch.Tensor, z: torch.Tensor, v: torch.Tensor, h: torch.Tensor, rank: int,
                     damping: float) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    B, L, D = v.shape
    G = G.contiguous()
    z = z.contiguous().to(torch.float32)
    v = v.contiguous()
    h = h.contiguous().to(torch.float32)
    dv = torch.empty_like(v)
    dz = torch.empty((B, L, rank), dtype=torch.float32, device=v.device)
    rc = lib.mogt_coupled_rank_scan_grad(G.data_ptr(), z.data_ptr(), v.data_ptr(), h.data_ptr(), dv.data_ptr(),
                                         dz.data_ptr(), B, L, rank, D // rank, float(damping),
                                         dtype_code(v.dtype, "coupled_grad"), _stream_handle(v.device))
    _lib.check(rc, "mogt_coupled_rank_scan_grad")
    return dv, dz


@_coupled_grad_op.register_fake
def _(G, z, v, h, rank, damping):
    return torch.empty_like(v), v.new_empty((*v.shape[:2], rank), dtype=torch.float32)


def _coupled_setup(ctx, inputs, output):
    z, v, rank, damping, _ = inputs
    # the fp32 output is the forward state h; the dz term needs it (h_{t-1})
    ctx.save_for_backward(z, v, output if output.dtype == torch.float32 else None)
    ctx.rank = rank
    ctx.damping = damping


def _coupled_backward(ctx, grad_h):
    """Backward of the fused gate + scan.  With g = sigmoid(z), a = damping (1-g)
    (per rank, over its c channels) and v' = v * g:  G = dH + a_{t+1} G_{t+1}
    (GPU reverse scan forming a from z in registers), dv = G * g, and per rank
    dg = sum_c G * v - damping * sum_c G * h_{t-1}, dz = dg * g (1 - g): one HIP
    epilogue kernel (channels a multiple of 4, D <= 4096) over G, z, v and the saved fp32
    forward output h (recomputed in fp32 when the forward rounded it, as the
    reference recomputes, triton_scan.py:370-378).
    The bf16 rounding of v * g (model_mogt.py:180) passes gradients through
    unchanged, as a dtype cast does under autograd."""
    z, v, h = ctx.saved_tensors
    r, damping = ctx.rank, ctx.damping
    B, L, D = v.shape
    c = D // r
    G = torch.ops.mogt.coupled_scan_rev(z, grad_h, r, damping)    # fp32 [B, L, D]
    if c % 4 == 0 and D <= 4096:
        if h is None:   # the forward returned a rounded h: recompute the fp32 state
            h = torch.ops.mogt.coupled_rank_scan(z, v, r, damping, torch.float32)
        dv, dz = torch.ops.mogt.coupled_grad(G, z, v, h, r, damping)
        return (dz.to(z.dtype) if ctx.needs_input_grad[0] else None,
                dv if ctx.needs_input_grad[1] else None, None, None, None)
    g = torch.sigmoid(z.float())                                   # [B, L, r]
    Gr = G.view(B, L, r, c)
    dz = dv = None
    if ctx.needs_input_grad[1]:
        g_io = g.to(v.dtype).float()                               # the gate as multiplied into v
        dv = (Gr * g_io.unsqueeze(-1)).reshape(B, L, D).to(v.dtype)
    if ctx.needs_input_grad[0]:
        if h is None:
            h = torch.ops.mogt.coupled_rank_scan(z, v, r, damping, torch.float32)
        hp = _shift_prev(h).view(B, L, r, c)
        dg = (Gr * v.float().view(B, L, r, c)).sum(-1) - damping * (Gr * hp).sum(-1)
        dz = (dg * g * (1.0 - g)).to(z.dtype)
    return dz, dv, None, None, None


torch.library.register_autograd("mogt::coupled_rank_scan", _coupled_backward, setup_context=_coupled_setup)


STAT_GROUP = 64   # features per column of the coupled scan's row statistics


@torch.library.custom_op("mogt::coupled_rank_scan_stats", mutates_args=())
def _coupled_rank_scan_stats_op(z: torch.Tensor, v: torch.Tensor, rank: int, damping: float,
                                out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    z = z.contiguous().to(torch.float32)
    v = v.contiguous()
    B, L, D = v.shape
    C = D // rank
    h = torch.empty(v.shape, dtype=out_dtype, device=v.device)
    stats = torch.empty((B, L, -(-D // STAT_GROUP)), dtype=torch.float32, device=v.device)
    vc = dtype_code(v.dtype, "coupled_rank_scan_stats")
    ws = workspace(lib.mogt_coupled_rank_scan_workspace_bytes(B, L, rank, C, vc), v.device, "coupled",
                   ("stats", B, L, rank, C, vc))
    rc = lib.mogt_coupled_rank_scan_stats_fwd(z.data_ptr(), v.data_ptr(), h.data_ptr(), stats.data_ptr(), B, L,
                                              rank, C, float(damping), vc,
                                              dtype_code(out_dtype, "coupled_rank_scan_stats"), ws.data_ptr(),
                                              ws.numel(), _stream_handle(v.device))
    _lib.check(rc, "mogt_coupled_rank_scan_stats_fwd")
    _checked(ws, "mogt_coupled_rank_scan_stats_fwd")
    return h, stats


@_coupled_rank_scan_stats_op.register_fake
def _(z, v, rank, damping, out_dtype):
    B, L, D = v.shape
    return v.new_empty(v.shape, dtype=out_dtype), v.new_empty((B, L, -(-D // STAT_GROUP)), dtype=torch.float32)


def coupled_rank_scan_stats(gate_logits: torch.Tensor, v_raw: torch.Tensor, *, damping: float = 1.0,
                            out_dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """``coupled_rank_scan`` that also returns the row statistics of the RMSNorm
    reading its output: ``stats[b, t, k]`` = sum of ``h[b, t, 64k:64k+64]**2`` in
    the fp32 state (before ``out_dtype`` rounding).  No autograd: the
    inference read-out (``add_rmsnorm_rowscale``) consumes them."""
    require_cuda("coupled_rank_scan_stats", gate_logits, v_raw)
    if gate_logits.ndim != 3 or v_raw.ndim != 3:
        raise ValueError("gate_logits must be [B, L, r] and v_raw [B, L, r*c]")
    B, L, r = gate_logits.shape
    if v_raw.shape[:2] != (B, L) or v_raw.shape[2] % r != 0:
        raise ValueError("gate_logits must be [B, L, r] and v_raw [B, L, r*c]")
    return torch.ops.mogt.coupled_rank_scan_stats(gate_logits, v_raw, r, float(damping), out_dtype)


@torch.library.custom_op("mogt::coupled_rank_scan_proj", mutates_args=())
def _coupled_rank_scan_proj_op(proj: torch.Tensor, features: int, gate_prev: bool, gate_const: torch.Tensor | None,
                               rank: int, damping: float) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    proj = proj.contiguous()
    B, L, ld = proj.shape
    D = int(features)
    C = D // rank
    h = torch.empty((B, L, D), dtype=proj.dtype, device=proj.device)
    stats = torch.empty((B, L, -(-D // STAT_GROUP)), dtype=torch.float32, device=proj.device)
    code = dtype_code(proj.dtype, "coupled_rank_scan_proj")
    gc = None
    if gate_const is not None:
        gc = gate_const.to(torch.float32).expand(B, rank).contiguous()
    ws = workspace(lib.mogt_coupled_rank_scan_workspace_bytes(B, L, rank, C, code), proj.device, "coupled",
                   ("proj", B, L, rank, C, code, ld, int(bool(gate_prev))))
    rc = lib.mogt_coupled_rank_scan_proj_fwd(proj.data_ptr(), ld, D, int(bool(gate_prev)),
                                             gc.data_ptr() if gc is not None else None, h.data_ptr(),
                                             stats.data_ptr(), None, B, L, rank, C, float(damping), code, code,
                                             ws.data_ptr(), ws.numel(), _stream_handle(proj.device))
    _lib.check(rc, "mogt_coupled_rank_scan_proj_fwd")
    _checked(ws, "mogt_coupled_rank_scan_proj_fwd")
    return h, stats


@_coupled_rank_scan_proj_op.register_fake
def _(proj, features, gate_prev, gate_const, rank, damping):
    B, L, _ = proj.shape
    return (proj.new_empty((B, L, features)),
            proj.new_empty((B, L, -(-features // STAT_GROUP)), dtype=torch.float32))


def coupled_rank_scan_proj(proj: torch.Tensor, features: int, *, rank: int, gate_prev: bool,
                           gate_const: torch.Tensor | None = None,
                           damping: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """The coupled scan fed by one projection ``proj [B, L, features + rank *
    (1 + gate_prev)]``: ``v = proj[..., :features]`` and the value gate's logit
    ``z_t = proj_t[features + i] + proj_{t-1}[features + rank + i] (if
    gate_prev, t > 0) + gate_const[b, i]``.  Returns ``h`` in proj's dtype and
    the row statistics of ``coupled_rank_scan_stats``.  No autograd."""
    require_cuda("coupled_rank_scan_proj", proj)
    if proj.ndim != 3 or features % rank != 0 or proj.shape[-1] < features + rank * (1 + int(gate_prev)):
        raise ValueError("proj must be [B, L, features + rank * (1 + gate_prev)]")
    if gate_const is not None:
        require_cuda("coupled_rank_scan_proj", gate_const)
        if gate_const.shape[-1] != rank or gate_const.ndim > 2:
            raise ValueError("gate_const must be [rank] or [B, rank]")
    return torch.ops.mogt.coupled_rank_scan_proj(proj, int(features), bool(gate_prev), gate_const, int(rank),
                                                 float(damping))


@torch.library.custom_op("mogt::coupled_proj_scan", mutates_args=())
def _coupled_proj_scan_op(proj: torch.Tensor, gate_const: torch.Tensor | None, features: int, rank: int,
                          gate_prev: bool, damping: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Training form of the projection-fed scan: fp32 h and the assembled
    fp32 logits z (kept for the backward)."""
    lib = _lib.load()
    proj = proj.contiguous()
    B, L, ld = proj.shape
    D = int(features)
    C = D // rank
    h = torch.empty((B, L, D), dtype=torch.float32, device=proj.device)
    z = torch.empty((B, L, rank), dtype=torch.float32, device=proj.device)
    code = dtype_code(proj.dtype, "coupled_proj_scan")
    gc = gate_const.to(torch.float32).contiguous() if gate_const is not None else None
    ws = workspace(lib.mogt_coupled_rank_scan_workspace_bytes(B, L, rank, C, code), proj.device, "coupled",
                   ("proj", B, L, rank, C, code, ld, int(bool(gate_prev))))
    rc = lib.mogt_coupled_rank_scan_proj_fwd(proj.data_ptr(), ld, D, int(bool(gate_prev)),
                                             gc.data_ptr() if gc is not None else None, h.data_ptr(), None,
                                             z.data_ptr(), B, L, rank, C, float(damping), code, _lib.MOGT_F32,
                                             ws.data_ptr(), ws.numel(), _stream_handle(proj.device))
    _lib.check(rc, "mogt_coupled_rank_scan_proj_fwd")
    _checked(ws, "mogt_coupled_rank_scan_proj_fwd")
    return h, z


@_coupled_proj_scan_op.register_fake
def _(proj, gate_const, features, rank, gate_prev, damping):
    B, L, _ = proj.shape
    return (proj.new_empty((B, L, features), dtype=torch.float32),
            proj.new_empty((B, L, rank), dtype=torch.float32))


@torch.library.custom_op("mogt::coupled_proj_grad", mutates_args=())
def _coupled_proj_grad_op(G: torch.Tensor, z: torch.Tensor, proj: torch.Tensor, h: torch.Tensor, features: int,
                          rank: int, gate_prev: bool, damping: float) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    G, z, proj, h = G.contiguous(), z.contiguous(), proj.contiguous(), h.contiguous()
    B, L, ld = proj.shape
    D = int(features)
    dproj = torch.empty_like(proj)
    dz = torch.empty((B, L, rank), dtype=torch.float32, device=proj.device)
    rc = lib.mogt_coupled_rank_scan_proj_grad(G.data_ptr(), z.data_ptr(), proj.data_ptr(), ld, int(bool(gate_prev)),
                                              h.data_ptr(), dproj.data_ptr(), dz.data_ptr(), B, L, rank, D // rank,
                                              float(damping), dtype_code(proj.dtype, "coupled_proj_grad"),
                                              _stream_handle(proj.device))
    _lib.check(rc, "mogt_coupled_rank_scan_proj_grad")
    return dproj, dz


@_coupled_proj_grad_op.register_fake
def _(G, z, proj, h, features, rank, gate_prev, damping):
    B, L, _ = proj.shape
    return torch.empty_like(proj), proj.new_empty((B, L, rank), dtype=torch.float32)


def _coupled_proj_setup(ctx, inputs, output):
    proj, gate_const, features, rank, gate_prev, damping = inputs
    h, z = output
    ctx.save_for_backward(proj, z, h)
    ctx.args = (int(features), int(rank), bool(gate_prev), float(damping))
    # the logits output is saved for the backward, not differentiated
    ctx.set_materialize_grads(False)


def _coupled_proj_backward(ctx, grad_h, grad_z):
    """G = dH + a_{t+1} G_{t+1} (reverse scan, decay from the saved logits),
    then one epilogue writes the projection's gradient (dv and the logit
    gradient in the current / previous-token gate columns); the per-sequence
    logit term gets the logit gradient summed over time."""
    proj, z, h = ctx.saved_tensors
    features, rank, gate_prev, damping = ctx.args
    if grad_h is None:
        return None, None, None, None, None, None
    G = torch.ops.mogt.coupled_scan_rev(z, grad_h, rank, damping)
    dproj, dz = torch.ops.mogt.coupled_proj_grad(G, z, proj, h, features, rank, gate_prev, damping)
    dconst = dz.sum(1) if ctx.needs_input_grad[1] else None
    return dproj, dconst, None, None, None, None


torch.library.register_autograd("mogt::coupled_proj_scan", _coupled_proj_backward, setup_context=_coupled_proj_setup)


def coupled_proj_scan(proj: torch.Tensor, features: int, *, rank: int, gate_prev: bool,
                      gate_const: torch.Tensor | None = None, damping: float = 1.0) -> torch.Tensor:
    """Differentiable projection-fed coupled scan: ``v = proj[..., :features]``,
    logits ``z_t = proj_t[features + i] + proj_{t-1}[features + rank + i]`` (if
    ``gate_prev``, t > 0) ``+ gate_const[b, i]`` (``[B, rank]`` fp32 or None);
    returns the fp32 state ``h [B, L, features]``.  Needs ``features / rank``
    and the projection's row length to be multiples of 4."""
    require_cuda("coupled_proj_scan", proj)
    B, L, ld = proj.shape
    if features % rank != 0 or ld != features + rank * (1 + int(gate_prev)):
        raise ValueError("proj must be [B, L, features + rank * (1 + gate_prev)]")
    if gate_const is not None and tuple(gate_const.shape) != (B, rank):
        raise ValueError("gate_const must be [B, rank]")
    h, _ = torch.ops.mogt.coupled_proj_scan(proj, gate_const, int(features), int(rank), bool(gate_prev),
                                            float(damping))
    return h


def coupled_proj_scan_supported(features: int, rank: int, gate_prev: bool) -> bool:
    c = features // rank
    return (features % rank == 0 and c % 4 == 0 and features <= 4096
            and (features + rank * (1 + int(gate_prev))) % 4 == 0)


def coupled_rank_scan(gate_logits: torch.Tensor, v_raw: torch.Tensor, *, damping: float = 1.0,
                      out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Fused gate + scan of the coupled write-forget MOGT mixer.

    ``gate_logits`` is ``[B, L, r]`` (the pre-sigmoid output of
    ``phi_value_gate``), ``v_raw`` is ``[B, L, r*c]`` (``phi_val`` output,
    feature ``d = i*c + j``).  Returns ``H`` flattened to ``[B, L, r*c]`` with
    ``H_t = damping*(1-g_t) * H_{t-1} + g_t * v_t`` per rank
    (model_mogt.py:166-203, identity connection, coupled gate).
    """
    require_cuda("coupled_rank_scan", gate_logits, v_raw)
    if gate_logits.ndim != 3 or v_raw.ndim != 3:
        raise ValueError("gate_logits must be [B, L, r] and v_raw [B, L, r*c]")
    B, L, r = gate_logits.shape
    if v_raw.shape[:2] != (B, L) or v_raw.shape[2] % r != 0:
        raise ValueError("gate_logits must be [B, L, r] and v_raw [B, L, r*c]")
    if _direct(gate_logits, v_raw):
        return _coupled_rank_scan_impl(gate_logits, v_raw, r, float(damping), out_dtype)
    return torch.ops.mogt.coupled_rank_scan(gate_logits, v_raw, r, float(damping), out_dtype)


# ---------------------------------------------------------------------------
# dense affine scan: H_t = U_t H_{t-1} + V_t (U [B,L,R,R], V/H [B,L,R,C])
# ---------------------------------------------------------------------------
MFMA_MAX_RANK = 32        # the matrix-core pipeline (dense_scan.hip)
GENERIC_MAX_RANK = 1024   # the generic scan (generic_scan.hip)
STATE_DTYPES = (torch.float32, torch.float64)
_GENERIC_CODE = {torch.float32: _lib.MOGT_F32, torch.bfloat16: _lib.MOGT_BF16,
                 torch.float64: _lib.MOGT_F64, torch.float16: _lib.MOGT_F16}


def check_affine_shapes(U: torch.Tensor, V: torch.Tensor) -> tuple[int, int, int, int]:
    """The reference's shape checks (affine_scan.py:26-32, triton_scan.py:193-199)."""
    if U.ndim != 4 or V.ndim != 4:
        raise ValueError("U and V must be rank-4 tensors")
    B, L, R, R2 = U.shape
    Bv, Lv, Rv, C = V.shape
    if (B, L, R) != (Bv, Lv, Rv) or R != R2:
        raise ValueError("U must be [B, L, R, R] and V must be [B, L, R, C]")
    if R > GENERIC_MAX_RANK:
        raise ValueError(f"R = {R} not supported by the MI355X scan (R <= {GENERIC_MAX_RANK})")
    return B, L, R, C


def check_mfma_rank(R: int, what: str) -> None:
    if R > MFMA_MAX_RANK:
        raise ValueError(f"{what}: R = {R} not supported by the MI355X scan (R <= {MFMA_MAX_RANK})")


def _affine_launch(U: torch.Tensor, V: torch.Tensor | None, H: torch.Tensor | None,
                   P: torch.Tensor | None) -> None:
    lib = _lib.load()
    B, L, R, _ = U.shape
    C = V.shape[-1] if V is not None else 0
    vc = dtype_code(V.dtype, "affine_scan") if V is not None else _lib.MOGT_F32
    out = H if H is not None else P
    oc = dtype_code(out.dtype, "affine_scan")
    stream = _stream_handle(U.device)
    if V is None:
        nbytes = lib.mogt_fused_scan_workspace_bytes(B, L, R)
        ws = workspace(nbytes, U.device)
        rc = lib.mogt_fused_scan_fwd(U.data_ptr(), P.data_ptr(), B, L, R, oc, ws.data_ptr(),
                                     ws.numel(), stream)
        _lib.check(rc, "mogt_fused_scan_fwd")
        return
    nbytes = lib.mogt_affine_scan_workspace_bytes(B, L, R, C)
    ws = workspace(nbytes, U.device)
    rc = lib.mogt_affine_scan_fwd(U.data_ptr(), V.data_ptr(), H.data_ptr(),
                                  P.data_ptr() if P is not None else None, B, L, R, C, vc, oc,
                                  ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "mogt_affine_scan_fwd")


def _prep_uv(U: torch.Tensor, V: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    U = U.contiguous()
    if U.dtype != torch.float32:
        U = U.to(torch.float32)   # the reference up-casts U (triton_scan.py:203)
    V = V.contiguous()
    if V.dtype not in _DTYPE_CODE:
        V = V.to(torch.float32)
    return U, V


@torch.library.custom_op("mogt::affine_scan", mutates_args=())
def _affine_scan_op(U: torch.Tensor, V: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    U, V = _prep_uv(U, V)
    H = torch.empty(V.shape, dtype=out_dtype, device=V.device)
    _affine_launch(U, V, H, None)
    return H


@_affine_scan_op.register_fake
def _(U, V, out_dtype):
    return V.new_empty(V.shape, dtype=out_dtype)


@torch.library.custom_op("mogt::affine_scan_prefix", mutates_args=())
def _affine_scan_prefix_op(U: torch.Tensor, V: torch.Tensor,
                           out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    U, V = _prep_uv(U, V)
    H = torch.empty(V.shape, dtype=out_dtype, device=V.device)
    P = torch.empty(U.shape, dtype=out_dtype, device=U.device)
    _affine_launch(U, V, H, P)
    return P, H


@_affine_scan_prefix_op.register_fake
def _(U, V, out_dtype):
    return U.new_empty(U.shape, dtype=out_dtype), V.new_empty(V.shape, dtype=out_dtype)


@torch.library.custom_op("mogt::affine_scan_generic", mutates_args=())
def _affine_scan_generic_op(U: torch.Tensor, V: torch.Tensor, state_dtype: torch.dtype,
                            out_dtype: torch.dtype, with_prefix: bool,
                            reverse: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """The generic scan (any R <= 1024, fp32 or fp64 state): returns
    ``(U_prefix, H)``, ``U_prefix`` empty unless ``with_prefix``; ``reverse``
    runs the backward's recursion H_t = V_t + U_{t+1}^T H_{t+1}."""
    lib = _lib.load()
    Us = U.to(state_dtype).contiguous()        # U_work = U.to(state_dtype), affine_scan.py:35
    Vc = (V if V.dtype in _GENERIC_CODE else V.to(state_dtype)).contiguous()
    B, L, R, _ = U.shape
    C = V.shape[-1]
    H = torch.empty(V.shape, dtype=out_dtype, device=V.device)
    P = torch.empty(U.shape if with_prefix else (0,), dtype=out_dtype, device=U.device)
    sc = _GENERIC_CODE[state_dtype]
    ws = workspace(lib.mogt_affine_scan_generic_workspace_bytes(B, L, R, C, int(with_prefix), sc), U.device)
    rc = lib.mogt_affine_scan_generic_fwd(
        Us.data_ptr(), Vc.data_ptr() if Vc.numel() else None, H.data_ptr() if H.numel() else None,
        P.data_ptr() if with_prefix and P.numel() else None, B, L, R, C, _GENERIC_CODE[Vc.dtype], sc,
        _GENERIC_CODE[out_dtype], int(reverse), ws.data_ptr(), ws.numel(), _stream_handle(U.device))
    _lib.check(rc, "mogt_affine_scan_generic_fwd")
    return P, H


@_affine_scan_generic_op.register_fake
def _(U, V, state_dtype, out_dtype, with_prefix, reverse):
    return (U.new_empty(U.shape if with_prefix else (0,), dtype=out_dtype),
            V.new_empty(V.shape, dtype=out_dtype))


def _use_mfma(R: int, state_dtype: torch.dtype, output_dtype: torch.dtype) -> bool:
    return state_dtype == torch.float32 and R <= MFMA_MAX_RANK and output_dtype in _DTYPE_CODE


def _forward_state(U: torch.Tensor, V: torch.Tensor, state_dtype: torch.dtype, prefix: bool):
    """H (and U_prefix) kept in the state dtype, as the backward needs them."""
    if _use_mfma(U.shape[-1], state_dtype, state_dtype):
        if prefix:
            return torch.ops.mogt.affine_scan_prefix(U, V, state_dtype)
        return torch.ops.mogt.affine_scan(U, V, state_dtype)
    P, H = torch.ops.mogt.affine_scan_generic(U, V, state_dtype, state_dtype, prefix, False)
    return (P, H) if prefix else H


@torch.library.custom_op("mogt::affine_scan_rev", mutates_args=())
def _affine_scan_rev_op(U: torch.Tensor, X: torch.Tensor) -> torch.Tensor:
    """G_t = X_t + U_{t+1}^T G_{t+1} on the matrix-core pipeline (fp32, R <= 32):
    time walked backwards and U_{t+1} read transposed inside the kernels."""
    lib = _lib.load()
    U, X = U.contiguous(), X.contiguous()
    B, L, R, C = X.shape
    G = torch.empty_like(X)
    ws = workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), X.device)
    rc = lib.mogt_affine_scan_rev_fwd(U.data_ptr(), X.data_ptr(), G.data_ptr(), B, L, R, C, ws.data_ptr(),
                                      ws.numel(), _stream_handle(X.device))
    _lib.check(rc, "mogt_affine_scan_rev_fwd")
    return G


@_affine_scan_rev_op.register_fake
def _(U, X):
    return torch.empty_like(X)


@torch.library.custom_op("mogt::affine_scan_grad_u", mutates_args=())
def _affine_scan_grad_u_op(G: torch.Tensor, H: torch.Tensor, P: torch.Tensor | None) -> torch.Tensor:
    """dU_t = G_t M_{t-1}^T with M = H or [H | P], M_{-1} = [0 | I] (fp32)."""
    lib = _lib.load()
    G, H = G.contiguous(), H.contiguous()
    P = P.contiguous() if P is not None else None
    B, L, R, C = H.shape
    dU = torch.empty(B, L, R, R, dtype=torch.float32, device=G.device)
    rc = lib.mogt_affine_scan_grad_u(G.data_ptr(), H.data_ptr(), P.data_ptr() if P is not None else None,
                                     dU.data_ptr(), B, L, R, C, _stream_handle(G.device))
    _lib.check(rc, "mogt_affine_scan_grad_u")
    return dU


@_affine_scan_grad_u_op.register_fake
def _(G, H, P):
    B, L, R, _ = H.shape
    return H.new_empty(B, L, R, R)


def _reverse_scan(U: torch.Tensor, X: torch.Tensor, state_dtype: torch.dtype) -> torch.Tensor:
    """G_t = X_t + U_{t+1}^T G_{t+1}, G_{L-1} = X_{L-1}, in the state dtype
    (the carry recursion of affine_scan.py:110-118): the matrix-core
    pipeline's reverse mode for fp32 and R <= 32, the generic scan's
    otherwise."""
    R = U.shape[-1]
    if _use_mfma(R, state_dtype, state_dtype):
        return torch.ops.mogt.affine_scan_rev(U.to(torch.float32), X.to(torch.float32))
    _, G = torch.ops.mogt.affine_scan_generic(U, X, state_dtype, state_dtype, False, True)
    return G


def affine_scan_grad(U: torch.Tensor, V: torch.Tensor, grad_H: torch.Tensor | None,
                     grad_P: torch.Tensor | None = None, *, state_dtype: torch.dtype = torch.float32,
                     need_grad_u: bool = True, need_grad_v: bool = True):
    """Gradients of H_t = U_t H_{t-1} + V_t (affine_scan_sequential_backward,
    affine_scan.py:65-124) and, with ``grad_P``, of U_prefix_t = U_t U_prefix_{t-1}:
    the augmented state M = [H | U_prefix] gets G = [dH | dP] + U_{t+1}^T G_{t+1}
    (one reverse scan), dV = G[..., :C] and dU_t = G_t M_{t-1}^T with
    M_{-1} = [0 | I].  Computed in ``state_dtype``, returned in U's / V's dtypes."""
    B, L, R, C = V.shape
    X = (grad_H.to(state_dtype) if grad_H is not None
         else torch.zeros(V.shape, dtype=state_dtype, device=V.device))
    if grad_P is not None:
        X = torch.cat([X, grad_P.to(state_dtype)], dim=-1)
    G = _reverse_scan(U, X.contiguous(), state_dtype)
    grad_v = G[..., :C].to(V.dtype) if need_grad_v else None
    grad_u = None
    if need_grad_u:
        if _use_mfma(R, state_dtype, state_dtype):
            # dU from the recomputed forward state read in place (shifted by a step)
            if grad_P is not None:
                P, H = _forward_state(U, V, state_dtype, True)
                grad_u = torch.ops.mogt.affine_scan_grad_u(G, H, P)
            else:
                grad_u = torch.ops.mogt.affine_scan_grad_u(G, _forward_state(U, V, state_dtype, False), None)
            return grad_u.to(U.dtype), grad_v
        zeros = torch.zeros(B, 1, R, C, dtype=state_dtype, device=V.device)
        if grad_P is not None:
            P, H = _forward_state(U, V, state_dtype, True)
            M = torch.cat([H, P], dim=-1)
            eye = torch.eye(R, dtype=state_dtype, device=V.device).expand(B, 1, R, R)
            M0 = torch.cat([zeros, eye], dim=-1)
        else:
            M = _forward_state(U, V, state_dtype, False)
            M0 = zeros
        M_prev = torch.cat([M0, M[:, :-1]], dim=1)
        grad_u = torch.matmul(G, M_prev.transpose(-2, -1).contiguous()).to(U.dtype)
    return grad_u, grad_v


def _affine_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1])


def _affine_backward(ctx, grad_H):
    U, V = ctx.saved_tensors
    gu, gv = affine_scan_grad(U, V, grad_H, None, state_dtype=torch.float32,
                              need_grad_u=ctx.needs_input_grad[0], need_grad_v=ctx.needs_input_grad[1])
    return gu, gv, None


def _affine_prefix_backward(ctx, grad_P, grad_H):
    U, V = ctx.saved_tensors
    gu, gv = affine_scan_grad(U, V, grad_H, grad_P, state_dtype=torch.float32,
                              need_grad_u=ctx.needs_input_grad[0], need_grad_v=ctx.needs_input_grad[1])
    return gu, gv, None


def _generic_setup(ctx, inputs, output):
    U, V, state_dtype, _out_dtype, with_prefix, reverse = inputs
    ctx.state_dtype = state_dtype
    ctx.with_prefix = with_prefix
    ctx.reverse = reverse
    ctx.save_for_backward(U, V)


def _generic_backward(ctx, grad_P, grad_H):
    if ctx.reverse:
        raise RuntimeError("the reverse affine scan (a backward pass) is not differentiable")
    U, V = ctx.saved_tensors
    gu, gv = affine_scan_grad(U, V, grad_H, grad_P if ctx.with_prefix else None,
                              state_dtype=ctx.state_dtype, need_grad_u=ctx.needs_input_grad[0],
                              need_grad_v=ctx.needs_input_grad[1])
    return gu, gv, None, None, None, None


torch.library.register_autograd("mogt::affine_scan", _affine_backward, setup_context=_affine_setup)
torch.library.register_autograd("mogt::affine_scan_prefix", _affine_prefix_backward,
                                setup_context=_affine_setup)
torch.library.register_autograd("mogt::affine_scan_generic", _generic_backward,
                                setup_context=_generic_setup)


def affine_scan(U: torch.Tensor, V: torch.Tensor, *, output_dtype: torch.dtype | None = None,
                return_prefix: bool = False, state_dtype: torch.dtype = torch.float32):
    """H_t = U_t H_{t-1} + V_t on the GPU, the state kept in ``state_dtype``
    (float32 or float64), ``output_dtype`` defaulting to ``V.dtype``; with
    ``return_prefix`` returns ``(U_prefix, H)`` (affine_scan.py:14-62
    semantics).  Differentiable in U and V.  fp32 state with R <= 32 and
    fp32 / bf16 output runs on the matrix-core pipeline, everything else on the
    generic scan."""
    require_cuda("affine_scan", U, V)
    _, _, R, _ = check_affine_shapes(U, V)
    output_dtype = output_dtype or V.dtype
    if state_dtype not in STATE_DTYPES:
        raise ValueError(f"state dtype {state_dtype} not supported (float32 or float64)")
    if output_dtype not in _GENERIC_CODE:
        raise ValueError(f"output dtype {output_dtype} not supported (float32, bfloat16, float16, float64)")
    if _use_mfma(R, state_dtype, output_dtype):
        if return_prefix:
            return torch.ops.mogt.affine_scan_prefix(U, V, output_dtype)
        return torch.ops.mogt.affine_scan(U, V, output_dtype)
    P, H = torch.ops.mogt.affine_scan_generic(U, V, state_dtype, output_dtype, return_prefix, False)
    return (P, H) if return_prefix else H


# ---------------------------------------------------------------------------
# dense_scan: the matrix scan with B_t given densely or as a rank-1 write v k^T
# ---------------------------------------------------------------------------
def check_vk_shapes(U: torch.Tensor, v: torch.Tensor, k: torch.Tensor) -> tuple[int, int, int, int]:
    if U.ndim != 4 or v.ndim != 3 or k.ndim != 3:
        raise ValueError("U must be [B, L, R, R], v [B, L, R] and k [B, L, C]")
    B, L, R, R2 = U.shape
    if R != R2 or tuple(v.shape) != (B, L, R) or tuple(k.shape[:2]) != (B, L):
        raise ValueError("U must be [B, L, R, R], v [B, L, R] and k [B, L, C]")
    if R > GENERIC_MAX_RANK:
        raise ValueError(f"R = {R} not supported by the MI355X scan (R <= {GENERIC_MAX_RANK})")
    return B, L, R, k.shape[-1]


@torch.library.custom_op("mogt::affine_scan_vk", mutates_args=())
def _affine_scan_vk_op(U: torch.Tensor, v: torch.Tensor, k: torch.Tensor,
                       out_dtype: torch.dtype) -> torch.Tensor:
    B, L, R, C = check_vk_shapes(U, v, k)
    U = U.contiguous()
    if U.dtype != torch.float32:
        U = U.to(torch.float32)
    if v.dtype not in _DTYPE_CODE or k.dtype != v.dtype:
        wide = torch.float32 if v.dtype not in _DTYPE_CODE else v.dtype
        v, k = v.to(wide), k.to(wide)
    v, k = v.contiguous(), k.contiguous()
    H = torch.empty((B, L, R, C), dtype=out_dtype, device=U.device)
    lib = _lib.load()
    ws = workspace(lib.mogt_affine_scan_workspace_bytes(B, L, R, C), U.device)
    rc = lib.mogt_affine_scan_vk_fwd(U.data_ptr(), v.data_ptr(), k.data_ptr(), H.data_ptr(), None,
                                     B, L, R, C, dtype_code(v.dtype, "dense_scan"),
                                     dtype_code(out_dtype, "dense_scan"), ws.data_ptr(), ws.numel(),
                                     _stream_handle(U.device))
    _lib.check(rc, "mogt_affine_scan_vk_fwd")
    return H


@_affine_scan_vk_op.register_fake
def _(U, v, k, out_dtype):
    return U.new_empty((*v.shape, k.shape[-1]), dtype=out_dtype)


def dense_scan(A: torch.Tensor, Bm: torch.Tensor | None = None, *, v: torch.Tensor | None = None,
               k: torch.Tensor | None = None, output_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``S_t = A_t S_{t-1} + B_t``, ``S_0 = 0`` (fp32 state) with either a dense
    ``Bm [B, L, R, C]`` or a rank-1 write ``B_t = v_t k_t^T`` from ``v [B, L, R]``
    and ``k [B, L, C]``, which is formed in registers and never written to
    memory (configs[3]'s ``B_t = v_t k_t^T``).  ``output_dtype`` defaults to the
    dtype of ``Bm`` (or ``v``)."""
    if (Bm is None) == (v is None and k is None) or (Bm is None and (v is None or k is None)):
        raise ValueError("dense_scan takes either Bm or both v and k")
    if Bm is not None:
        return affine_scan(A, Bm, output_dtype=output_dtype)
    require_cuda("dense_scan", A, v, k)
    _, _, R, _ = check_vk_shapes(A, v, k)
    output_dtype = output_dtype or v.dtype
    if output_dtype not in _DTYPE_CODE:
        raise ValueError(f"output dtype {output_dtype} not supported (float32 or bfloat16)")
    if R > MFMA_MAX_RANK:
        # above the matrix-core pipeline's rank: B_t = v_t k_t^T formed as fp32
        # products (as the in-register form does) and scanned by the generic kernel
        Bm = v.to(torch.float32).unsqueeze(-1) * k.to(torch.float32).unsqueeze(-2)
        return affine_scan(A, Bm, output_dtype=output_dtype)
    return torch.ops.mogt.affine_scan_vk(A, v, k, output_dtype)


@torch.library.custom_op("mogt::fused_scan", mutates_args=())
def _fused_scan_op(U: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    Uf = U.contiguous().to(torch.float32)
    Y = torch.empty(U.shape, dtype=out_dtype, device=U.device)
    _affine_launch(Uf, None, None, Y)
    return Y


@_fused_scan_op.register_fake
def _(U, out_dtype):
    return U.new_empty(U.shape, dtype=out_dtype)


def fused_scan(U: torch.Tensor, *, output_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Transport-only prefix product Y_t = U_t Y_{t-1}, Y_0 = I (triton_scan.py:13-51)."""
    require_cuda("fused_scan", U)
    if U.ndim != 4 or U.shape[2] != U.shape[3]:
        raise ValueError("U must be [B, L, R, R]")
    B, L, R, _ = U.shape
    if R > GENERIC_MAX_RANK:
        raise ValueError(f"R = {R} not supported by the MI355X scan (R <= {GENERIC_MAX_RANK})")
    output_dtype = output_dtype or U.dtype
    if output_dtype not in _GENERIC_CODE:
        raise ValueError(f"output dtype {output_dtype} not supported (float32, bfloat16, float16, float64)")
    if R <= MFMA_MAX_RANK and output_dtype in _DTYPE_CODE:
        return torch.ops.mogt.fused_scan(U, output_dtype)
    # the generic scan's prefix columns with no channels: Y_t = U_t Y_{t-1}, Y_0 = I
    Y, _ = torch.ops.mogt.affine_scan_generic(U, U.new_empty((B, L, R, 0), dtype=torch.float32),
                                              torch.float32, output_dtype, True, False)
    return Y


@torch.library.custom_op("mogt::affine_local_scan", mutates_args=())
def _affine_local_scan_op(U: torch.Tensor, V: torch.Tensor, block_size: int
                          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    U, V = _prep_uv(U, V)
    B, L, R, _ = U.shape
    C = V.shape[-1]
    nb = (L + block_size - 1) // block_size
    f32 = dict(dtype=torch.float32, device=U.device)
    Up = torch.empty(U.shape, **f32)
    Hp = torch.empty(V.shape, **f32)
    Us = torch.empty((B, nb, R, R), **f32)
    Hs = torch.empty((B, nb, R, C), **f32)
    rc = lib.mogt_affine_local_scan(U.data_ptr(), V.data_ptr(), Up.data_ptr(), Hp.data_ptr(),
                                    Us.data_ptr(), Hs.data_ptr(), B, L, R, C, block_size,
                                    dtype_code(V.dtype, "affine_local_scan"),
                                    _stream_handle(U.device))
    _lib.check(rc, "mogt_affine_local_scan")
    return Up, Hp, Us, Hs


@_affine_local_scan_op.register_fake
def _(U, V, block_size):
    B, L, R, _ = U.shape
    C = V.shape[-1]
    nb = (L + block_size - 1) // block_size
    f = dict(dtype=torch.float32)
    return (U.new_empty(U.shape, **f), V.new_empty(V.shape, **f),
            U.new_empty((B, nb, R, R), **f), V.new_empty((B, nb, R, C), **f))


@torch.library.custom_op("mogt::affine_local_scan_generic", mutates_args=())
def _affine_local_scan_generic_op(U: torch.Tensor, V: torch.Tensor, block_size: int
                                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The block-local scan on the generic kernel (R > 32), fp32 like the
    matrix-core pass; summaries are the prefixes at each block's last step
    (the identity padding of the tail block changes neither)."""
    lib = _lib.load()
    Us = U.to(torch.float32).contiguous()
    Vc = (V if V.dtype in _GENERIC_CODE else V.to(torch.float32)).contiguous()
    B, L, R, _ = U.shape
    C = V.shape[-1]
    Up = torch.empty(U.shape, dtype=torch.float32, device=U.device)
    Hp = torch.empty(V.shape, dtype=torch.float32, device=V.device)
    rc = lib.mogt_affine_local_scan_generic(
        Us.data_ptr(), Vc.data_ptr() if Vc.numel() else None, Up.data_ptr(), Hp.data_ptr() if Hp.numel() else None,
        B, L, R, C, block_size, _GENERIC_CODE[Vc.dtype], _lib.MOGT_F32, _lib.MOGT_F32, _stream_handle(U.device))
    _lib.check(rc, "mogt_affine_local_scan_generic")
    ends = torch.clamp(torch.arange(1, (L + block_size - 1) // block_size + 1, device=U.device) * block_size,
                       max=L) - 1
    return Up, Hp, Up[:, ends].contiguous(), Hp[:, ends].contiguous()


@_affine_local_scan_generic_op.register_fake
def _(U, V, block_size):
    B, L, R, _ = U.shape
    C = V.shape[-1]
    nb = (L + block_size - 1) // block_size
    f = dict(dtype=torch.float32)
    return (U.new_empty(U.shape, **f), V.new_empty(V.shape, **f),
            U.new_empty((B, nb, R, R), **f), V.new_empty((B, nb, R, C), **f))


def affine_local_scan(U: torch.Tensor, V: torch.Tensor, *, block_size: int = 256):
    """Block-local prefixes and per-block summaries (triton_scan.py:178-229),
    fp32; R <= 32 on the matrix-core pass, larger R on the generic kernel."""
    require_cuda("affine_local_scan", U, V)
    _, _, R, _ = check_affine_shapes(U, V)
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if R > MFMA_MAX_RANK:
        return torch.ops.mogt.affine_local_scan_generic(U, V, int(block_size))
    return torch.ops.mogt.affine_local_scan(U, V, int(block_size))


# ---------------------------------------------------------------------------
# row-wise block kernels: rmsnorm, residual-add + rmsnorm, silu-mul
# ---------------------------------------------------------------------------
@torch.library.custom_op("mogt::rmsnorm", mutates_args=())
def _rmsnorm_op(x: torch.Tensor, weight: torch.Tensor, eps: float,
                out_dtype: torch.dtype) -> torch.Tensor:
    lib = _lib.load()
    x = x.contiguous()
    w = weight.contiguous().to(torch.float32)
    D = x.shape[-1]
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rc = lib.mogt_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), out.data_ptr(), x.numel() // D, D,
                              float(eps), dtype_code(x.dtype, "rmsnorm"),
                              dtype_code(out_dtype, "rmsnorm"), _stream_handle(x.device))
    _lib.check(rc, "mogt_rmsnorm_fwd")
    return out


@_rmsnorm_op.register_fake
def _(x, weight, eps, out_dtype):
    return x.new_empty(x.shape, dtype=out_dtype)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
            out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """RMSNorm.forward (model_mogt.py:15-20) in one pass; ``out_dtype`` defaults
    to float32 (the dtype of ``normalised.type_as(x) * fp32 weight``)."""
    require_cuda("rmsnorm", x, weight)
    return torch.ops.mogt.rmsnorm(x, weight, float(eps), out_dtype or torch.float32)


@torch.library.custom_op("mogt::add_rmsnorm", mutates_args=())
def _add_rmsnorm_op(x: torch.Tensor, z: torch.Tensor, scale: float, weight: torch.Tensor, eps: float,
                    out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    x = x.contiguous()
    z = z.contiguous()
    w = weight.contiguous().to(torch.float32)
    D = x.shape[-1]
    x_out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rc = lib.mogt_add_rmsnorm_fwd(x.data_ptr(), z.data_ptr(), float(scale), w.data_ptr(),
                                  x_out.data_ptr(), out.data_ptr(), x.numel() // D, D, float(eps),
                                  dtype_code(z.dtype, "add_rmsnorm"),
                                  dtype_code(out_dtype, "add_rmsnorm"), _stream_handle(x.device))
    _lib.check(rc, "mogt_add_rmsnorm_fwd")
    return x_out, out


@_add_rmsnorm_op.register_fake
def _(x, z, scale, weight, eps, out_dtype):
    return x.new_empty(x.shape, dtype=torch.float32), x.new_empty(x.shape, dtype=out_dtype)


def add_rmsnorm(x: torch.Tensor, z: torch.Tensor, scale: float, weight: torch.Tensor,
                eps: float = 1e-6, out_dtype: torch.dtype = torch.float32):
    """``x' = x + scale * z`` (fp32 residual stream) and ``rmsnorm(x') * weight``."""
    require_cuda("add_rmsnorm", x, z, weight)
    if x.dtype != torch.float32:
        raise ValueError("add_rmsnorm keeps the residual stream in float32")
    if x.shape != z.shape:
        raise ValueError("x and z must have the same shape")
    return torch.ops.mogt.add_rmsnorm(x, z, float(scale), weight, float(eps), out_dtype)


@torch.library.custom_op("mogt::add_rmsnorm_final", mutates_args=())
def _add_rmsnorm_final_op(x: torch.Tensor, z: torch.Tensor, scale: float, weight: torch.Tensor, eps: float,
                          out_dtype: torch.dtype) -> torch.Tensor:
    lib = _lib.load()
    x = x.contiguous()
    z = z.contiguous()
    w = weight.contiguous().to(torch.float32)
    D = x.shape[-1]
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rc = lib.mogt_add_rmsnorm_fwd(x.data_ptr(), z.data_ptr(), float(scale), w.data_ptr(), None, out.data_ptr(),
                                  x.numel() // D, D, float(eps), dtype_code(z.dtype, "add_rmsnorm_final"),
                                  dtype_code(out_dtype, "add_rmsnorm_final"), _stream_handle(x.device))
    _lib.check(rc, "mogt_add_rmsnorm_fwd")
    return out


@_add_rmsnorm_final_op.register_fake
def _(x, z, scale, weight, eps, out_dtype):
    return x.new_empty(x.shape, dtype=out_dtype)


def add_rmsnorm_final(x: torch.Tensor, z: torch.Tensor, scale: float, weight: torch.Tensor, eps: float = 1e-6,
                      out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``rmsnorm(x + scale * z) * weight`` without writing the updated residual
    stream (the last norm of the backbone).  No autograd."""
    require_cuda("add_rmsnorm_final", x, z, weight)
    if x.dtype != torch.float32 or x.shape != z.shape:
        raise ValueError("add_rmsnorm_final: x float32 and z of the same shape")
    return torch.ops.mogt.add_rmsnorm_final(x, z, float(scale), weight, float(eps), out_dtype)


@torch.library.custom_op("mogt::add_rmsnorm_rowscale", mutates_args=())
def _add_rmsnorm_rowscale_op(x: torch.Tensor, z: torch.Tensor, stats: torch.Tensor, stat_eps: float, scale: float,
                             weight: torch.Tensor, eps: float, out_dtype: torch.dtype
                             ) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    x = x.contiguous()
    z = z.contiguous()
    stats = stats.contiguous()
    w = weight.contiguous().to(torch.float32)
    D = x.shape[-1]
    rows = x.numel() // D
    x_out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rc = lib.mogt_add_rmsnorm_rowscale_fwd(x.data_ptr(), z.data_ptr(), stats.data_ptr(), stats.shape[-1],
                                           float(stat_eps), float(scale), w.data_ptr(), x_out.data_ptr(),
                                           out.data_ptr(), rows, D, float(eps),
                                           dtype_code(z.dtype, "add_rmsnorm_rowscale"),
                                           dtype_code(out_dtype, "add_rmsnorm_rowscale"), _stream_handle(x.device))
    _lib.check(rc, "mogt_add_rmsnorm_rowscale_fwd")
    return x_out, out


@_add_rmsnorm_rowscale_op.register_fake
def _(x, z, stats, stat_eps, scale, weight, eps, out_dtype):
    return x.new_empty(x.shape, dtype=torch.float32), x.new_empty(x.shape, dtype=out_dtype)


def add_rmsnorm_rowscale(x: torch.Tensor, z: torch.Tensor, stats: torch.Tensor, scale: float,
                         weight: torch.Tensor, *, stat_eps: float = 1e-6, eps: float = 1e-6,
                         out_dtype: torch.dtype = torch.float32):
    """``add_rmsnorm`` whose residual term is normalised per row first:
    ``Z = z * rsqrt(sum(stats[row]) / D + stat_eps)`` (rounded to z's dtype),
    ``x' = x + scale * Z``, ``out = rmsnorm(x') * weight``.  For ``z = h @ (W
    diag(w_out))^T`` and ``stats`` from ``coupled_rank_scan_stats`` it equals
    ``theta_read(norm_out(h))`` added to the residual stream.  No autograd."""
    require_cuda("add_rmsnorm_rowscale", x, z, stats, weight)
    if x.dtype != torch.float32:
        raise ValueError("add_rmsnorm_rowscale keeps the residual stream in float32")
    if x.shape != z.shape or stats.shape[:-1] != x.shape[:-1] or stats.dtype != torch.float32:
        raise ValueError("x and z must have the same shape and stats must be float32 [..., n_stats]")
    return torch.ops.mogt.add_rmsnorm_rowscale(x, z, stats, float(stat_eps), float(scale), weight, float(eps),
                                               out_dtype)


@torch.library.custom_op("mogt::silu_mul", mutates_args=())
def _silu_mul_op(y: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    y = y.contiguous()
    H2 = y.shape[-1]
    out = torch.empty((*y.shape[:-1], H2 // 2), dtype=y.dtype, device=y.device)
    rc = lib.mogt_silu_mul_fwd(y.data_ptr(), out.data_ptr(), y.numel() // H2, H2 // 2,
                               dtype_code(y.dtype, "silu_mul"), _stream_handle(y.device))
    _lib.check(rc, "mogt_silu_mul_fwd")
    return out


@_silu_mul_op.register_fake
def _(y):
    return y.new_empty((*y.shape[:-1], y.shape[-1] // 2))


@torch.library.custom_op("mogt::swiglu_gate", mutates_args=())
def _swiglu_gate_op(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    x = x if x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 else x.contiguous()
    w_gate = w_gate.contiguous()
    w_up = w_up.contiguous()
    H, K = w_gate.shape
    y = torch.empty((x.shape[0], H), dtype=x.dtype, device=x.device)
    rc = lib.mogt_swiglu_gate_fwd(x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), y.data_ptr(), x.shape[0], K, H,
                                  x.stride(0), y.stride(0), dtype_code(x.dtype, "swiglu_gate"),
                                  _stream_handle(x.device))
    _lib.check(rc, "mogt_swiglu_gate_fwd")
    return y


@_swiglu_gate_op.register_fake
def _(x, w_gate, w_up):
    return x.new_empty((x.shape[0], w_gate.shape[0]))


SWIGLU_GATE_K_MULTIPLE = 32
SWIGLU_GATE_H_MULTIPLE = 128


def swiglu_gate_supported(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> bool:
    """Whether ``swiglu_gate`` takes these operands: bf16 CUDA tensors, the
    input dimension a multiple of 32 and the hidden size of 128."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and w_gate.dtype == torch.bfloat16
            and w_up.dtype == torch.bfloat16 and w_gate.shape == w_up.shape and w_gate.ndim == 2
            and x.shape[-1] == w_gate.shape[1] and w_gate.shape[1] % SWIGLU_GATE_K_MULTIPLE == 0
            and w_gate.shape[0] % SWIGLU_GATE_H_MULTIPLE == 0)


def swiglu_gate(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """``silu(x @ w_gate.T) * (x @ w_up.T)`` in bf16 as one GEMM whose
    epilogue applies the gate (model_mogt.py:29-30); each linear output and
    the silu are rounded to bf16 as in the unfused expression.  x ``[..., K]``,
    weights ``[H, K]``.  No autograd."""
    require_cuda("swiglu_gate", x, w_gate, w_up)
    if not swiglu_gate_supported(x, w_gate, w_up):
        raise ValueError("swiglu_gate needs bf16 x [..., K] and weights [H, K] with K % 32 == 0, H % 128 == 0")
    lead = x.shape[:-1]
    y = torch.ops.mogt.swiglu_gate(x.reshape(-1, x.shape[-1]), w_gate, w_up)
    return y.reshape(*lead, w_gate.shape[0])


# weight gradient of the training path's linear layers ---------------------
WGRAD_MULTIPLE = 8   # d_out, d_in and row strides of mogt_linear_wgrad


def _wgrad_rows(t: torch.Tensor) -> torch.Tensor:
    """``t`` as [tokens, features] rows the kernel takes (unit column stride,
    row stride a multiple of 8, 16-byte aligned), copying only if needed."""
    r = t.reshape(-1, t.shape[-1])
    if r.stride(-1) != 1 or r.stride(0) % WGRAD_MULTIPLE != 0 or r.data_ptr() % 16 != 0 or r.stride(0) < r.shape[1]:
        r = r.contiguous()
    return r


def _linear_wgrad_impl(dy: torch.Tensor, x: torch.Tensor, out_dtype: torch.dtype, splits: int = 0) -> torch.Tensor:
    lib = _lib.load()
    d2, x2 = _wgrad_rows(dy), _wgrad_rows(x)
    T, O = d2.shape
    I = x2.shape[1]
    dw = torch.empty((O, I), dtype=out_dtype, device=dy.device)
    nbytes = int(lib.mogt_linear_wgrad_workspace_bytes(T, O, I, splits, 0))
    ws = workspace(nbytes, dy.device)
    rc = lib.mogt_linear_wgrad(d2.data_ptr(), x2.data_ptr(), dw.data_ptr(), T, O, I, d2.stride(0), x2.stride(0),
                               dw.stride(0), splits, dtype_code(out_dtype, "linear_wgrad"), ws.data_ptr(), ws.numel(),
                               _stream_handle(dy.device))
    _lib.check(rc, "mogt_linear_wgrad")
    return dw


@torch.library.custom_op("mogt::linear_wgrad", mutates_args=())
def _linear_wgrad_op(dy: torch.Tensor, x: torch.Tensor, out_dtype: torch.dtype, splits: int = 0) -> torch.Tensor:
    """dW = dY^T X over the flattened leading dimensions."""
    return _linear_wgrad_impl(dy, x, out_dtype, splits)


@_linear_wgrad_op.register_fake
def _(dy, x, out_dtype, splits=0):
    return dy.new_empty((dy.shape[-1], x.shape[-1]), dtype=out_dtype)


def linear_wgrad_supported(dy: torch.Tensor, x: torch.Tensor) -> bool:
    """Whether ``linear_wgrad`` takes these operands: bf16 CUDA tensors with
    the same leading shape and both feature sizes multiples of 8."""
    return (dy.is_cuda and x.is_cuda and dy.dtype == torch.bfloat16 and x.dtype == torch.bfloat16
            and dy.ndim >= 1 and dy.shape[:-1] == x.shape[:-1] and dy.shape[-1] % WGRAD_MULTIPLE == 0
            and x.shape[-1] % WGRAD_MULTIPLE == 0 and dy.shape[-1] > 0 and x.shape[-1] > 0)


def linear_wgrad(dy: torch.Tensor, x: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16,
                 splits: int = 0) -> torch.Tensor:
    """``dy.reshape(-1, O).T @ x.reshape(-1, I)``, the weight gradient of a
    bias-free linear layer ``y = x @ W.T`` (model_mogt.py:25-27, 57, 61), as
    the HIP split-K GEMM: fp32 partials per token slice, summed in slice order
    and rounded once to ``out_dtype`` (bf16 or float32).  ``splits`` <= 0
    picks the slice count that gives every CU one work-group.  No autograd."""
    require_cuda("linear_wgrad", dy, x)
    if not linear_wgrad_supported(dy, x):
        raise ValueError("linear_wgrad needs bf16 dy [..., O] and x [..., I] with equal leading shapes and "
                         "O % 8 == 0, I % 8 == 0")
    if _direct(dy, x):
        return _linear_wgrad_impl(dy, x, out_dtype, int(splits))
    return torch.ops.mogt.linear_wgrad(dy, x, out_dtype, int(splits))


class _Linear(torch.autograd.Function):
    """``y = x @ w.T`` (a bias-free nn.Linear, F.linear's own GEMM); backward:
    ``dx = dy @ w`` with the same library GEMM autograd would call, and ``dw``
    by the split-K weight-gradient kernel in ``w``'s dtype."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        dx = g.matmul(w) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            dw = torch.ops.mogt.linear_wgrad(g, x, w.dtype, 0) if linear_wgrad_supported(g, x) \
                else g.reshape(-1, g.shape[-1]).t().mm(x.reshape(-1, x.shape[-1]))
        return dx, dw


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, w)`` whose weight gradient, when ``w`` needs one and the
    operands are bf16 on the GPU with feature sizes that are multiples of 8,
    comes from ``linear_wgrad`` instead of the library GEMM (whose d_out x
    d_in output has too few tiles to fill the GPU at the model's widths)."""
    if (torch.is_grad_enabled() and w.requires_grad and x.is_cuda and x.dtype == torch.bfloat16
            and w.dtype == torch.bfloat16 and w.ndim == 2 and x.shape[-1] == w.shape[1]
            and w.shape[0] % WGRAD_MULTIPLE == 0 and w.shape[1] % WGRAD_MULTIPLE == 0):
        return _Linear.apply(x, w)
    return F.linear(x, w)


# token embedding with a deterministic HIP backward -------------------------
EMBEDDING_BLOCK = 16   # sorted positions per block of mogt_embedding_bwd


def _rows_for_embedding_bwd(grad: torch.Tensor, D: int) -> torch.Tensor:
    g = grad.reshape(-1, D)
    if g.stride(-1) != 1 or g.stride(0) % 4 != 0 or g.data_ptr() % 16 != 0:
        g = g.contiguous()
    return g


@torch.library.custom_op("mogt::embedding_bwd", mutates_args=())
def _embedding_bwd_op(grad: torch.Tensor, ids: torch.Tensor, vocab: int, grad2: torch.Tensor | None = None,
                      ids2: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [vocab, D] gradient of the table from the rows of ``grad`` at
    ``ids`` and, optionally, those of ``grad2`` at ``ids2`` (a second lookup
    into the same table), summed per id in position order."""
    lib = _lib.load()
    D = grad.shape[-1]
    g = _rows_for_embedding_bwd(grad, D)
    flat = ids.reshape(-1).to(torch.int64)
    n1 = flat.numel()
    g2 = None
    if grad2 is not None:
        g2 = _rows_for_embedding_bwd(grad2.to(g.dtype), D)
        flat = torch.cat([flat, ids2.reshape(-1).to(torch.int64)])
    sorted_ids, positions = torch.sort(flat, stable=True)
    n = flat.numel()
    dw = torch.zeros((int(vocab), D), dtype=torch.float32, device=grad.device)
    parts = torch.empty((max(1, -(-n // EMBEDDING_BLOCK)) * 2, D), dtype=torch.float32, device=grad.device)
    rc = lib.mogt_embedding_bwd(g.data_ptr(), g.stride(0), g2.data_ptr() if g2 is not None else None,
                                g2.stride(0) if g2 is not None else 0, n1, dtype_code(g.dtype, "embedding_bwd"),
                                sorted_ids.data_ptr(), positions.data_ptr(), n, D, int(vocab), dw.data_ptr(),
                                parts.data_ptr(), _stream_handle(grad.device))
    _lib.check(rc, "mogt_embedding_bwd")
    return dw


@_embedding_bwd_op.register_fake
def _(grad, ids, vocab, grad2=None, ids2=None):
    return grad.new_empty((int(vocab), grad.shape[-1]), dtype=torch.float32)


class _Embedding(torch.autograd.Function):
    """F.embedding forward (one or two lookups into the same table); the
    weight's gradient from mogt_embedding_bwd, one table for both lookups."""

    @staticmethod
    def forward(ctx, weight, ids, ids2=None):
        ctx.save_for_backward(ids, ids2)
        ctx.vocab = weight.shape[0]
        ctx.wdtype = weight.dtype
        if ids2 is None:
            return F.embedding(ids, weight)
        return F.embedding(ids, weight), F.embedding(ids2, weight)

    @staticmethod
    def backward(ctx, grad_out, grad_out2=None):
        ids, ids2 = ctx.saved_tensors
        if grad_out is None:
            grad_out, ids = grad_out2, ids2
            grad_out2 = None
        if grad_out is None:
            return None, None, None
        dw = torch.ops.mogt.embedding_bwd(grad_out, ids, ctx.vocab, grad_out2, ids2 if grad_out2 is not None else None)
        return dw.to(ctx.wdtype), None, None


def _plain_embedding(module: torch.nn.Embedding) -> bool:
    w = module.weight
    plain = (module.padding_idx is None and module.max_norm is None and not module.scale_grad_by_freq
             and not module.sparse)
    return (plain and w.is_cuda and w.dim() == 2 and w.shape[1] % 4 == 0 and w.shape[1] <= 4096
            and w.dtype in (torch.float32, torch.bfloat16))


def embedding_pair(ids: torch.Tensor, ids2: torch.Tensor,
                   module: torch.nn.Embedding) -> tuple[torch.Tensor, torch.Tensor]:
    """``(module(ids), module(ids2))`` whose backward writes one gradient table
    for both lookups (the second lookup's rows join the first's in the same
    position-ordered sums) instead of a full-size table per lookup and their
    sum."""
    if not _plain_embedding(module):
        return module(ids), module(ids2)
    return _Embedding.apply(module.weight, ids, ids2)


def embedding(ids: torch.Tensor, module: torch.nn.Embedding) -> torch.Tensor:
    """``module(ids)`` with the weight's gradient summed by the HIP kernel in
    position order (deterministic, one pass over the gradient rows).  Plain
    embeddings only (no padding index, norm clipping, frequency scaling or
    sparse gradients); others go through ``module`` itself."""
    if not _plain_embedding(module):
        return module(ids)
    return _Embedding.apply(module.weight, ids)


# GEMM operands of a training step, cast in one pass -------------------------
class _CastGroups(torch.autograd.Function):
    """Each group of parameters concatenated along dim 0 and cast to ``dtype``
    (the casts autocast, or an explicit ``.to``, would make one tensor at a
    time, after a concatenation) with one multi-tensor copy; backward: every
    parameter's gradient, its rows of the group's gradient cast back to the
    parameter's dtype, with one multi-tensor copy."""

    @staticmethod
    def forward(ctx, dtype, sizes, *params):
        ctx.sizes = sizes
        ctx.meta = [(p.shape, p.dtype) for p in params]
        ctx.set_materialize_grads(False)   # an unused operand gives its parameters no gradient
        outs, dst = [], []
        i = 0
        for n in sizes:
            grp = params[i:i + n]
            out = torch.empty((sum(p.shape[0] for p in grp), *grp[0].shape[1:]), dtype=dtype,
                              device=grp[0].device)
            outs.append(out)
            dst.extend(out.split([p.shape[0] for p in grp], dim=0))
            i += n
        torch._foreach_copy_(dst, [p.contiguous() for p in params])
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        res = [None] * len(ctx.meta)
        src, dst = [], []
        i = 0
        for n, g in zip(ctx.sizes, grads):
            if g is not None:
                parts = g.split([ctx.meta[k][0][0] for k in range(i, i + n)], dim=0)
                for k, part in zip(range(i, i + n), parts):
                    res[k] = torch.empty(ctx.meta[k][0], dtype=ctx.meta[k][1], device=part.device)
                    src.append(part)
                    dst.append(res[k])
            i += n
        if dst:
            torch._foreach_copy_(dst, src)
        return (None, None, *res)


def cast_groups(groups: list, dtype: torch.dtype) -> list:
    """For each group (parameters with equal trailing shape), the parameters
    concatenated along dim 0 in ``dtype``, differentiable.  All the casts, and
    their gradients' casts back, run as one multi-tensor copy each way instead
    of a kernel per tensor plus the concatenations."""
    params = [p for grp in groups for p in grp]
    return list(_CastGroups.apply(dtype, [len(grp) for grp in groups], *params))


# backward of the row kernels -------------------------------------------------
RMSNORM_BWD_WAVES_PER_GROUP = 4   # mogt_rmsnorm_bwd writes one dw partial per feature and 4-wave work-group


def _rows_per_wave(rows: int) -> int:
    # about 2048 waves, at least 4 rows each: the dw partials stay a few MB
    return max(4, -(-rows // 2048))


def _rmsnorm_bwd_launch(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, dres: torch.Tensor | None,
                        eps: float, dz: torch.Tensor | None, dz_scale: float):
    lib = _lib.load()
    x = x.contiguous()
    dy = dy.contiguous()
    w = weight.contiguous().to(torch.float32)
    D = x.shape[-1]
    rows = x.numel() // D
    rpw = _rows_per_wave(rows)
    dx = torch.empty_like(x)
    groups = -(-(-(-rows // rpw)) // RMSNORM_BWD_WAVES_PER_GROUP)
    parts = torch.empty((D, max(1, groups)), dtype=torch.float32, device=x.device)
    if dres is not None:
        dres = dres.contiguous().to(torch.float32)
    rc = lib.mogt_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), dy.data_ptr(),
                              dres.data_ptr() if dres is not None else None, dx.data_ptr(),
                              parts.data_ptr(), rows, D, float(eps), rpw, dtype_code(x.dtype, "rmsnorm_bwd"),
                              dtype_code(dy.dtype, "rmsnorm_bwd"), dz.data_ptr() if dz is not None else None,
                              float(dz_scale), dtype_code(dz.dtype, "rmsnorm_bwd") if dz is not None else 0,
                              _stream_handle(x.device))
    _lib.check(rc, "mogt_rmsnorm_bwd")
    dw = parts.sum(1) if rows > 0 else torch.zeros(D, dtype=torch.float32, device=x.device)
    return dx, dw


@torch.library.custom_op("mogt::rmsnorm_bwd", mutates_args=())
def _rmsnorm_bwd_op(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, dres: torch.Tensor | None,
                    eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return _rmsnorm_bwd_launch(x, weight, dy, dres, eps, None, 0.0)


@_rmsnorm_bwd_op.register_fake
def _(x, weight, dy, dres, eps):
    return torch.empty_like(x), x.new_empty(x.shape[-1], dtype=torch.float32)


@torch.library.custom_op("mogt::add_rmsnorm_bwd", mutates_args=())
def _add_rmsnorm_bwd_op(x_out: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, dres: torch.Tensor | None,
                        eps: float, scale: float, z_dtype: torch.dtype
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of add_rmsnorm in one pass: dx (the residual stream), dz =
    (dx * scale) in z's dtype, and dw."""
    dz = torch.empty(x_out.shape, dtype=z_dtype, device=x_out.device)
    dx, dw = _rmsnorm_bwd_launch(x_out, weight, dy, dres, eps, dz, scale)
    return dx, dz, dw


@_add_rmsnorm_bwd_op.register_fake
def _(x_out, weight, dy, dres, eps, scale, z_dtype):
    return (torch.empty_like(x_out), x_out.new_empty(x_out.shape, dtype=z_dtype),
            x_out.new_empty(x_out.shape[-1], dtype=torch.float32))


def _rmsnorm_setup(ctx, inputs, output):
    x, weight, eps, out_dtype = inputs
    ctx.save_for_backward(x, weight)
    ctx.eps = eps


def _rmsnorm_backward(ctx, g):
    x, weight = ctx.saved_tensors
    dx, dw = torch.ops.mogt.rmsnorm_bwd(x, weight, g, None, ctx.eps)
    return dx, dw.to(weight.dtype), None, None


torch.library.register_autograd("mogt::rmsnorm", _rmsnorm_backward, setup_context=_rmsnorm_setup)


def _add_rmsnorm_setup(ctx, inputs, output):
    x, z, scale, weight, eps, out_dtype = inputs
    ctx.save_for_backward(output[0], weight)
    ctx.scale = scale
    ctx.eps = eps
    ctx.z_dtype = z.dtype
    # an unused output gets no gradient tensor (not a materialised zero one)
    ctx.set_materialize_grads(False)


def _add_rmsnorm_backward(ctx, g_xout, g_out):
    x_out, weight = ctx.saved_tensors
    if g_out is None:
        if g_xout is None:
            return None, None, None, None, None, None
        # only the residual stream's own gradient: the norm adds nothing
        dx = g_xout.to(x_out.dtype)
        dz = (dx * float(ctx.scale)).to(ctx.z_dtype)
        dw = torch.zeros(x_out.shape[-1], dtype=weight.dtype, device=x_out.device)
        return dx, dz, None, dw, None, None
    dx, dz, dw = torch.ops.mogt.add_rmsnorm_bwd(x_out, weight, g_out, g_xout, ctx.eps, float(ctx.scale),
                                                ctx.z_dtype)
    return dx, dz, None, dw.to(weight.dtype), None, None


torch.library.register_autograd("mogt::add_rmsnorm", _add_rmsnorm_backward, setup_context=_add_rmsnorm_setup)


@torch.library.custom_op("mogt::silu_mul_bwd", mutates_args=())
def _silu_mul_bwd_op(y: torch.Tensor, dout: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    y = y.contiguous()
    dout = dout.contiguous().to(y.dtype)
    H2 = y.shape[-1]
    dy = torch.empty_like(y)
    rc = lib.mogt_silu_mul_bwd(y.data_ptr(), dout.data_ptr(), dy.data_ptr(), y.numel() // H2, H2 // 2,
                               dtype_code(y.dtype, "silu_mul_bwd"), _stream_handle(y.device))
    _lib.check(rc, "mogt_silu_mul_bwd")
    return dy


@_silu_mul_bwd_op.register_fake
def _(y, dout):
    return torch.empty_like(y)


def _silu_mul_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])


def _silu_mul_backward(ctx, g):
    (y,) = ctx.saved_tensors
    return torch.ops.mogt.silu_mul_bwd(y, g)


torch.library.register_autograd("mogt::silu_mul", _silu_mul_backward, setup_context=_silu_mul_setup)


def silu_mul(y: torch.Tensor) -> torch.Tensor:
    """``silu(y[..., :H]) * y[..., H:]`` for the fused ``[w1; w2]`` projection."""
    require_cuda("silu_mul", y)
    if y.shape[-1] % 8 != 0:
        raise ValueError("silu_mul needs an even hidden size that is a multiple of 4")
    return torch.ops.mogt.silu_mul(y)


# ---------------------------------------------------------------------------
# connection map of the transport: U = damping * f(scale * A), A skew
# ---------------------------------------------------------------------------
_CONN_IMPL = {"matrix_exp": _lib.MOGT_CONN_EXP, "cayley": _lib.MOGT_CONN_CAYLEY}


def _connection_map_reference(A: torch.Tensor, impl: int, scale: float, damping: float) -> torch.Tensor:
    """The same map with torch's library routines (model_mogt.py:79-102); used
    to differentiate the HIP forward."""
    X = A.to(torch.float32) * scale
    if impl == _lib.MOGT_CONN_EXP:
        U = torch.matrix_exp(X)
    else:
        eye = torch.eye(A.shape[-1], dtype=X.dtype, device=X.device)
        U = torch.linalg.solve(eye - 0.5 * X, eye + 0.5 * X)
    return U * damping


@torch.library.custom_op("mogt::connection_map", mutates_args=())
def _connection_map_op(A: torch.Tensor, impl: int, scale: float, damping: float,
                       out_dtype: torch.dtype) -> torch.Tensor:
    lib = _lib.load()
    A32 = A.to(torch.float32).contiguous()
    r = A.shape[-1]
    n = A32.numel() // (r * r) if r else 0
    U = torch.empty(A.shape, dtype=out_dtype, device=A.device)
    rc = lib.mogt_connection_map_fwd(A32.data_ptr(), U.data_ptr(), n, r, float(scale), float(damping),
                                     int(impl), dtype_code(out_dtype, "connection_map"),
                                     _stream_handle(A.device))
    _lib.check(rc, "mogt_connection_map_fwd")
    return U


@_connection_map_op.register_fake
def _(A, impl, scale, damping, out_dtype):
    return A.new_empty(A.shape, dtype=out_dtype)


def _connection_map_setup(ctx, inputs, output):
    A, impl, scale, damping, _ = inputs
    ctx.save_for_backward(A)
    ctx.args = (impl, scale, damping)


def _connection_map_backward(ctx, grad_u):
    (A,) = ctx.saved_tensors
    with torch.enable_grad():
        Ad = A.detach().requires_grad_()
        U = _connection_map_reference(Ad, *ctx.args)
        (gA,) = torch.autograd.grad(U, Ad, grad_u.to(U.dtype))
    return gA.to(A.dtype), None, None, None, None


torch.library.register_autograd("mogt::connection_map", _connection_map_backward,
                                setup_context=_connection_map_setup)


def connection_map(A: torch.Tensor, impl: str, *, scale: float = 1.0, damping: float = 1.0,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``U = damping * f(scale * A)`` for skew-symmetric ``A [..., r, r]`` (r <= 32)
    with ``f`` = ``matrix_exp`` or ``cayley`` (``(I - S/2)^{-1} (I + S/2)``),
    the transport maps of model_mogt.py:79-102, on the HIP kernels; gradients
    come from torch's routines on the same inputs."""
    require_cuda("connection_map", A)
    if impl not in _CONN_IMPL:
        raise ValueError(f"Unsupported connection_impl: {impl}")
    if A.ndim < 2 or A.shape[-1] != A.shape[-2]:
        raise ValueError("A must be [..., r, r]")
    if A.shape[-1] > 32:
        raise ValueError(f"r = {A.shape[-1]} not supported by the MI355X connection map (r <= 32)")
    return torch.ops.mogt.connection_map(A, _CONN_IMPL[impl], float(scale), float(damping), out_dtype)


# ---------------------------------------------------------------------------
# rank-1 coupled write-forget scan with readout
# ---------------------------------------------------------------------------
RANK1_PATHS = {"auto": 0, "single": 1, "three": 2}
# path 3 of the C entry point: the one-launch kernel with super-chunk 0
# withholding its aggregate and short bounded waits (a test of the give-up
# handling and of the fallback below); not a public choice
_RANK1_GIVEUP_TEST = 3
R1_SUPER = 256        # steps per super-chunk
R1_SINGLE_MAX = 64    # super-chunks per sequence the one-launch kernel takes
R1_GROUPS_PER_CU = 3  # one-launch work-groups resident per compute unit


def _rank1_single(path: int, B: int, L: int, H: int, kvq: torch.dtype, device: torch.device) -> bool:
    """Whether the C entry point runs the one-launch kernel for this call (the
    rule of mogt_rank1_coupled_scan_fwd_cfg: bf16 k, v, q, at most
    R1_SINGLE_MAX super-chunks per sequence, and every work-group resident at
    once, R1_GROUPS_PER_CU per compute unit)."""
    if path in (1, _RANK1_GIVEUP_TEST):
        return True
    nsc = -(-L // R1_SUPER)
    if path != 0 or kvq != torch.bfloat16 or nsc > R1_SINGLE_MAX:
        return False
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return B * H * nsc <= R1_GROUPS_PER_CU * cus


def _rank1_launch(f, k, v, q, y, path: int) -> torch.Tensor:
    lib = _lib.load()
    B, L, H, d = k.shape
    single = _rank1_single(path, B, L, H, k.dtype, k.device)
    nbytes = lib.mogt_rank1_coupled_scan_workspace_bytes(B, L, H, d)
    ws = workspace(nbytes, k.device, "rank1", (B, L, H)) if single else workspace(nbytes, k.device)
    rc = lib.mogt_rank1_coupled_scan_fwd_cfg(f.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr(),
                                             y.data_ptr(), B, L, H, d,
                                             dtype_code(f.dtype, "rank1_coupled_scan"),
                                             dtype_code(k.dtype, "rank1_coupled_scan"),
                                             dtype_code(y.dtype, "rank1_coupled_scan"),
                                             ws.data_ptr(), ws.numel(), int(path), _stream_handle(k.device))
    _lib.check(rc, "mogt_rank1_coupled_scan_fwd_cfg")
    return ws if single else None


def _rank1_impl(f: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
                out_dtype: torch.dtype, path: int) -> torch.Tensor:
    f, k, v, q = (t.contiguous() for t in (f, k, v, q))
    y = torch.empty(k.shape, dtype=out_dtype, device=k.device)
    ws = _rank1_launch(f, k, v, q, y, path)
    if ws is not None and CHECK_WORKSPACE and not torch.cuda.is_current_stream_capturing():
        # the one-launch kernel needs every super-chunk of a sequence resident
        # at once; if work on another stream held the GPU its waits gave up
        # and y holds NaN: take the three-launch path, which waits on nothing
        n = _new_faults(ws)
        if n:
            warnings.warn(f"rank1_coupled_scan: {n} wait(s) of the one-launch kernel gave up; "
                          "recomputed with the three-launch path", RuntimeWarning, stacklevel=2)
            _rank1_launch(f, k, v, q, y, RANK1_PATHS["three"])
    return y


_rank1_op = torch.library.custom_op("mogt::rank1_coupled_scan", _rank1_impl, mutates_args=())


@_rank1_op.register_fake
def _(f, k, v, q, out_dtype, path):
    return k.new_empty(k.shape, dtype=out_dtype)


def rank1_coupled_scan(f: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor, *,
                       out_dtype: torch.dtype | None = None, path: str = "auto") -> torch.Tensor:
    """``y_t = S_t q_t`` with ``S_t = f_t S_{t-1} + (1 - f_t) v_t k_t^T`` per
    (batch, head); f ``[B, L, H]``, k/v/q ``[B, L, H, 64]``.  Products on bf16
    MFMA (inputs rounded to bf16), fp32 state; ``out_dtype`` defaults to
    ``q.dtype``.  ``path``: "auto" (one launch for bf16 k, v, q when
    L <= 16384 and the B * H * ceil(L / 256) work-groups fit the GPU at three
    per compute unit; three launches otherwise), "single" or "three" to force
    one."""
    if path not in RANK1_PATHS:
        raise ValueError(f"path must be one of {sorted(RANK1_PATHS)}")
    require_cuda("rank1_coupled_scan", f, k, v, q)
    if k.ndim != 4 or k.shape != v.shape or k.shape != q.shape:
        raise ValueError("k, v and q must be [B, L, H, d] of the same shape")
    if f.shape != k.shape[:3]:
        raise ValueError("f must be [B, L, H]")
    if k.dtype != v.dtype or k.dtype != q.dtype:
        raise ValueError("k, v and q must share a dtype")
    if k.shape[-1] != 64:
        raise ValueError(f"head dim {k.shape[-1]} not supported (64)")
    if _direct(f, k, v, q):
        return _rank1_impl(f, k, v, q, out_dtype or q.dtype, RANK1_PATHS[path])
    return torch.ops.mogt.rank1_coupled_scan(f, k, v, q, out_dtype or q.dtype, RANK1_PATHS[path])


# ---------------------------------------------------------------------------
# cross-entropy rows of the chunked tied-head loss (chunked_lm_loss.py:5-80)
# ---------------------------------------------------------------------------
def _check_ce_rows(logits: torch.Tensor, labels: torch.Tensor, what: str) -> None:
    require_cuda(what, logits, labels)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError(f"{what}: logits must be [rows, vocab] with contiguous rows")
    if labels.dim() != 1 or labels.shape[0] != logits.shape[0] or labels.dtype != torch.int64:
        raise ValueError(f"{what}: labels must be int64 [rows]")
    dtype_code(logits.dtype, what)


@torch.library.custom_op("mogt::lm_ce_fwd", mutates_args=())
def _lm_ce_fwd_op(logits: torch.Tensor, labels: torch.Tensor,
                  ignore_index: int) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    labels = labels.contiguous()
    rows, vocab = logits.shape
    loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
    lse = torch.empty(rows, dtype=torch.float32, device=logits.device)
    rc = lib.mogt_lm_ce_fwd(logits.data_ptr(), logits.stride(0), dtype_code(logits.dtype, "lm_ce_fwd"),
                            labels.data_ptr(), rows, vocab, int(ignore_index), loss.data_ptr(),
                            lse.data_ptr(), _stream_handle(logits.device))
    _lib.check(rc, "mogt_lm_ce_fwd")
    return loss, lse


@_lm_ce_fwd_op.register_fake
def _(logits, labels, ignore_index):
    rows = logits.shape[0]
    return logits.new_empty(rows, dtype=torch.float32), logits.new_empty(rows, dtype=torch.float32)


def lm_ce_forward(logits: torch.Tensor, labels: torch.Tensor, *, ignore_index: int = -100):
    """Per-row cross-entropy of a logits block: ``(loss_rows, lse_rows)``, both
    fp32 [rows]; ``loss = logsumexp(logits) - logits[label]`` (0 where the label
    is ``ignore_index``), as F.cross_entropy(..., reduction="none")."""
    _check_ce_rows(logits, labels, "lm_ce_forward")
    return torch.ops.mogt.lm_ce_fwd(logits, labels, int(ignore_index))


@torch.library.custom_op("mogt::lm_ce_bwd_", mutates_args=("logits",))
def _lm_ce_bwd_op(logits: torch.Tensor, labels: torch.Tensor, lse: torch.Tensor, scale: torch.Tensor,
                  ignore_index: int) -> None:
    lib = _lib.load()
    labels = labels.contiguous()
    lse = lse.contiguous()
    rows, vocab = logits.shape
    code = dtype_code(logits.dtype, "lm_ce_bwd")
    rc = lib.mogt_lm_ce_bwd(logits.data_ptr(), logits.stride(0), code, labels.data_ptr(), lse.data_ptr(),
                            rows, vocab, int(ignore_index), scale.data_ptr(), logits.data_ptr(),
                            logits.stride(0), code, _stream_handle(logits.device))
    _lib.check(rc, "mogt_lm_ce_bwd")


@_lm_ce_bwd_op.register_fake
def _(logits, labels, lse, scale, ignore_index):
    return None


@torch.library.custom_op("mogt::lm_ce_grad", mutates_args=())
def _lm_ce_grad_op(logits: torch.Tensor, labels: torch.Tensor, lse: torch.Tensor, scale: torch.Tensor,
                   ignore_index: int) -> torch.Tensor:
    lib = _lib.load()
    labels = labels.contiguous()
    lse = lse.contiguous()
    rows, vocab = logits.shape
    grad = torch.empty((rows, vocab), dtype=torch.float32, device=logits.device)
    rc = lib.mogt_lm_ce_bwd(logits.data_ptr(), logits.stride(0), dtype_code(logits.dtype, "lm_ce_grad"),
                            labels.data_ptr(), lse.data_ptr(), rows, vocab, int(ignore_index), scale.data_ptr(),
                            grad.data_ptr(), vocab, _lib.MOGT_F32, _stream_handle(logits.device))
    _lib.check(rc, "mogt_lm_ce_bwd")
    return grad


@_lm_ce_grad_op.register_fake
def _(logits, labels, lse, scale, ignore_index):
    return logits.new_empty(logits.shape, dtype=torch.float32)


def lm_ce_grad(logits: torch.Tensor, labels: torch.Tensor, lse: torch.Tensor, scale: torch.Tensor, *,
               ignore_index: int = -100) -> torch.Tensor:
    """``scale * (softmax(logits) - onehot(labels))`` as a new fp32 block (zero
    rows where the label is ``ignore_index``), for fp32 or bf16 logits."""
    _check_ce_rows(logits, labels, "lm_ce_grad")
    if lse.shape != labels.shape or lse.dtype != torch.float32:
        raise ValueError("lm_ce_grad: lse must be float32 [rows]")
    if scale.numel() != 1 or scale.dtype != torch.float32 or scale.device != logits.device:
        raise ValueError("lm_ce_grad: scale must be a one-element float32 tensor on the logits' device")
    return torch.ops.mogt.lm_ce_grad(logits, labels, lse, scale.reshape(1).contiguous(), int(ignore_index))


def lm_ce_backward_(logits: torch.Tensor, labels: torch.Tensor, lse: torch.Tensor,
                    scale: torch.Tensor, *, ignore_index: int = -100) -> torch.Tensor:
    """Overwrite a logits block with ``scale * (softmax(logits) - onehot(labels))``
    (zero rows where the label is ``ignore_index``); ``scale`` is a one-element
    fp32 device tensor (``grad_output / tokens``), read by the kernel."""
    _check_ce_rows(logits, labels, "lm_ce_backward_")
    if lse.shape != labels.shape or lse.dtype != torch.float32:
        raise ValueError("lm_ce_backward_: lse must be float32 [rows]")
    if scale.numel() != 1 or scale.dtype != torch.float32 or scale.device != logits.device:
        raise ValueError("lm_ce_backward_: scale must be a one-element float32 tensor on the logits' device")
    torch.ops.mogt.lm_ce_bwd_(logits, labels, lse, scale.reshape(1).contiguous(), int(ignore_index))
    return logits
