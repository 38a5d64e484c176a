"""The Loopback depth-attention read on MI355X: a drop-in for yancyou/Loopback's `fused_dattn.py`.

Same names, signatures and gradient conventions as the reference module (fused_dattn.py:185-793); the compute runs
in hand-written HIP kernels for gfx950 behind the C ABI of `include/loopback_read.h` (loaded by `_lib`). There is no
Triton, no CUDA path and no fallback: a missing library fails at import, a bad argument raises RuntimeError.

One read at destination s has n = s + 1 sources v_i (the raw block updates) and computes (fused_dattn.py:3-27)

    z_i  = r_i (q . v_i) / sqrt(d),  r_i = rsqrt(mean(v_i^2) + eps)
    p    = softmax_i(z_i + lc_i),  p0 = softmax_i(lc_i),  lc_i = log max(c0_i, 1e-8),  M = sum_i c0_i
    tc_i = c0_i + M (p_i - p0_i)                         (the installed coefficients, returned)
    out  = base + sum_i (tc_i - cbar_i) v_i              (fp32 accumulation, one rounding to the update dtype)

Backward (g = dL/dout, gt = dL/dtc): gd_i = g.v_i, gp_i = M (gd_i + gt_i), Sacc = sum_i p_i gp_i,
dz_i = p_i (gp_i - Sacc), dq = sum_tok sum_i dz_i r_i v_i / sqrt(d), dv_i = (tc_i - cbar_i) g + dz_i r_i q / sqrt(d),
dr_i = dz_i z_i / r_i, dcbar_i = -gd_i, dbase = g.

Layouts:
  * list layout (FusedDattnRead, FusedDattnReadAcc): one tensor per source; the kernels take the n source addresses
    by value in their arguments (no device pointer array, no host-to-device copy);
  * stacked layout (DattnStack, FusedDattnReadStk): the updates of a pass in V[n_steps, b, t, d]. With the read
    queries, each write also stores the update's scores against every later read query, DOTS[j, i, tok]
    (query-major, then source, then token: coalesced for both the write and the read), and the reads form their
    softmax from them; without them (and in the list layout) a read forms the scores as it streams the sources,
    with an online softmax, in one pass. The stacked backward does not read-modify-write a gradient stack per read: each read's
    backward keeps its output gradient g_s and its per-(source, token) scalars (w, dz r / sqrt(d)); the gradient of
    update i is formed once, when its scale's backward runs (after every read of it), as
    sum_s (w_si g_s + dzr_si q_s) + the scale's term, in fp32 with one rounding. Same gradients, at least as
    accurate as the per-read bf16 adds, and about a quarter less HBM traffic over a pass. With
    LOOP_DATTN_GRAD_ROUNDING=per_read the same kernel rounds each read's share and adds them in the update dtype from
    the last read to the first, then the scale's term: the list layout's gradients bit for bit, as the reference's
    stack (which read-modify-writes a bf16 gradient stack) promises;
  * FusedCombineStk (this module's extension, no reference counterpart): the stacked read with the caller's glue
    (LoopDeltaAttnRes.combine's iteration-end blend and coefficient bookkeeping) inside the kernels, and the
    gradient hand-offs that spare autograd's own glue (one query gradient per pass, the proposal's gradient added
    by the update-gradient kernel, h0's blend gradients summed once).
"""
from __future__ import annotations

import ctypes
import os
import weakref

import torch

from . import _lib as L

__all__ = ["rstd_ref", "rstd", "fused_read_supported", "FusedDattnRead", "DattnGradAccum", "FusedDattnReadAcc",
           "DattnStack", "FusedDattnReadStk", "FusedCombineStk", "_alias"]

_LIB = L.LIB
MAX_SOURCES = L.MAX_SOURCES
ANY_MAX_SOURCES = L.ANY_MAX_SOURCES


# ---------------------------------------------------------------------------------------------------------------
# plumbing
# ---------------------------------------------------------------------------------------------------------------
def _p(t: torch.Tensor | None):
    """A tensor's device address for a pointer argument (an int; None is NULL)."""
    return None if t is None else t.data_ptr()


_raw_stream = torch._C._cuda_getCurrentRawStream   # the device's current hipStream_t, as an int


def _stream(dev: torch.device):
    """The current stream of `dev` (the launch stream of every entry point)."""
    return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())


_DTYPES = {torch.bfloat16: L.BF16, torch.float16: L.F16, torch.float32: L.F32}


def _dtype_code(dtype: torch.dtype) -> int:
    """The library's code of an update dtype: bf16, fp16 (the reference's kernels load any float dtype and round
    back to it) or fp32."""
    code = _DTYPES.get(dtype)
    if code is None:
        raise RuntimeError(f"delta_attnres HIP read: updates must be bfloat16, float16 or float32, got {dtype}")
    return code


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"delta_attnres HIP read: {what} must be a GPU (HIP) tensor, got device {t.device}")


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _f32(t: torch.Tensor) -> torch.Tensor:
    """t as a contiguous fp32 tensor for a kernel argument (t itself when it already is one)."""
    if t.dtype is torch.float32 and t.is_contiguous():
        return t.detach()
    return t.detach().float().contiguous()


def _inv_sqrt(d: int) -> float:
    return 1.0 / (d ** 0.5)


def grad_rounding() -> str:
    """LOOP_DATTN_GRAD_ROUNDING (this build's switch, read when a stack is made): 'once' (default) forms each update's
    gradient as one fp32 sum rounded once; 'per_read' rounds each read's share and adds them in the update dtype in
    the order autograd adds the list layout's per-read gradients, so the stacked gradients are the list layout's."""
    mode = os.environ.get("LOOP_DATTN_GRAD_ROUNDING", "once")
    if mode not in ("once", "per_read"):
        raise ValueError(f"LOOP_DATTN_GRAD_ROUNDING must be 'once' or 'per_read', got {mode!r}")
    return mode


def _fast(d: int, n: int, *rows) -> bool:
    """Whether the row-layout entry points take a call: width d a multiple of 8 up to MAX_WIDTH, at most
    MAX_SOURCES sources, every row tensor 16-byte aligned. Other calls go to the any-shape entry points (rows of any
    width at element alignment, up to ANY_MAX_SOURCES sources, per-source addresses in device arrays)."""
    if d % 8 or d > L.MAX_WIDTH or n > MAX_SOURCES:
        return False
    for t in rows:
        if t is not None and t.data_ptr() % 16:
            return False
    return True


def _dev_addrs(addrs, dev: torch.device) -> torch.Tensor:
    """A device array of addresses for an any-shape entry point, copied on the current stream from pinned host
    memory (torch keeps the host buffer until the copy has run; the device array is freed in stream order). Not
    under HIP graph capture: a replay would copy from a host buffer torch may since have reused."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("delta_attnres HIP read: shapes the row-layout kernels do not take (d not a multiple of 8 "
                           "or above 8192, more than 64 sources, unaligned rows) cannot be captured in a HIP graph")
    host = torch.tensor(list(addrs), dtype=torch.int64).pin_memory()
    return host.to(dev, non_blocking=True)


def _b1_parts(n_tok: int, d: int) -> int:
    """Rows of backward pass 1's query-gradient partials: the row-layout kernel's workgroups (which the any-shape
    kernel then also uses), or for widths that layout does not take one per 64 tokens, up to 512."""
    p = L.bwd1_parts(n_tok, d)
    return p if p > 0 else max(1, min(512, -(-n_tok // 64)))


class _Src:
    """The sources of one read: host address arrays (v, r; dr for the scale gradients) for the row-layout entry
    points when `fast`, else device address arrays for the any-shape ones."""
    __slots__ = ("fast", "v", "r", "dr")

    def __init__(self, fast: bool, v, r, dr=None):
        self.fast, self.v, self.r, self.dr = fast, v, r, dr

    @staticmethod
    def of(fast: bool, values, rstds, dev, drs=None):
        addrs = (lambda ts: L.u64_array(t.data_ptr() for t in ts)) if fast else \
                (lambda ts: _dev_addrs((t.data_ptr() for t in ts), dev))
        return _Src(fast, addrs(values), addrs(rstds), None if drs is None else addrs(drs))

    def ptrs(self):
        """(v, r) as entry-point arguments: host arrays, or the device arrays' addresses."""
        return (self.v, self.r) if self.fast else (self.v.data_ptr(), self.r.data_ptr())

    def dr_ptr(self):
        return self.dr if self.fast else self.dr.data_ptr()


def _read(src: _Src, n: int, q, dots, stored: bool, base, h0, beta: float, cbar, cols: int, c0, lam: float, out, tc,
          prob, next_prior, n_tok: int, d: int, dt: int, st) -> None:
    """One read forward from stored raw scores (stored: dots[i, tok]) or with the scores formed from the fp32 query q
    and kept in dots: the row-layout kernels when src.fast, else the any-shape kernel. cols: n (cbar, c0 as the read
    takes them) or n - 1 (the previous read's coefficients and prior, scaled by lam, the newest entry implied)."""
    v, r = src.ptrs()
    tail = (_p(base), _p(h0), float(beta), _p(cbar), cols, _p(c0), cols, float(lam), _inv_sqrt(d), _p(out), _p(tc),
            _p(prob), _p(next_prior), n_tok, d, dt, st)
    if not src.fast:
        _run("read_fwd_any", v, r, n, None if stored else _p(q), _p(dots), n_tok, *tail)
    elif stored:
        _run("read_fwd", v, r, n, _p(dots), n_tok, *tail)
    else:
        _run("read_fwd_online", v, r, n, _p(q), _p(dots), n_tok, *tail)


# Optional launch observer: a callable name -> context manager, entered around every library call (the bench uses it
# to bracket each kernel with HIP events on the launch stream). None in normal use.
_TIMER = None


# the entry points, bound once (name without the ldr_ prefix -> ctypes function with its signature)
_FN = {name[4:]: getattr(_LIB, name) for name in L.SIGNATURES}


def _run(name: str, *args) -> None:
    fn = _FN[name]
    if _TIMER is None:
        code = fn(*args)
    else:
        with _TIMER(name):
            code = fn(*args)
    if code:
        L.check(code, name)


# ---------------------------------------------------------------------------------------------------------------
# the RMS scale of a source (fused_dattn.py:197-261)
# ---------------------------------------------------------------------------------------------------------------
def rstd_ref(delta: torch.Tensor, eps: float) -> torch.Tensor:
    """The RMSNorm scale of a source as a torch expression, (b, t, 1) fp32 (fused_dattn.py:197-199). Part of the
    module's interface for callers, and what rstd returns for a tensor that is not on the GPU; the HIP path does not
    use it."""
    return torch.rsqrt(delta.float().pow(2).mean(-1, keepdim=True) + eps)


class _Rstd(torch.autograd.Function):
    """r = rsqrt(sum x^2 / d + eps) per token; backward gx = gr (-r^3) / d x (fused_dattn.py:232-254)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, eps: float):
        xc = x.contiguous()
        d = xc.shape[-1]
        n_tok = xc.numel() // d
        r = torch.empty(xc.shape[:-1] + (1,), device=xc.device, dtype=torch.float32)
        _run("rstd_fwd", _p(xc), _p(r), n_tok, d, float(eps), _dtype_code(xc.dtype), _stream(xc.device))
        ctx.save_for_backward(xc, r)
        return r

    @staticmethod
    def backward(ctx, gr: torch.Tensor):
        xc, r = ctx.saved_tensors
        d = xc.shape[-1]
        n_tok = xc.numel() // d
        gx = torch.empty_like(xc)
        grc = gr.float().contiguous()
        _run("rstd_bwd", _p(xc), _p(r), _p(grc), _p(gx), n_tok, d, _dtype_code(xc.dtype), _stream(xc.device))
        return gx, None


def rstd(delta: torch.Tensor, eps: float) -> torch.Tensor:
    """The RMSNorm scale of a source, (b, t, 1) fp32, differentiable (fused_dattn.py:257-261): the HIP kernels for a
    GPU tensor; for any other tensor rstd_ref, as the reference module returns there. That keeps the reference's
    callers working on CPU tensors: `combine` takes the scales from rstd before asking fused_read_supported, which is
    False off the GPU, and then runs its own read (looped_transformer.py:395-404). No read of this module runs on the
    CPU."""
    if delta.is_cuda:
        return _Rstd.apply(delta, float(eps))
    return rstd_ref(delta, eps)


# ---------------------------------------------------------------------------------------------------------------
# list layout (fused_dattn.py:264-395)
# ---------------------------------------------------------------------------------------------------------------
def fused_read_supported(base, values, rstds, cbar) -> bool:
    """The reference's gate (fused_dattn.py:379-395) -- GPU, contiguous, same-shape same-dtype bf16/fp32 sources and
    base, contiguous fp32 (b, t, 1) rstds, contiguous fp32 (b, t, n) cbar -- plus the kernels' source count (at most
    ANY_MAX_SOURCES) and one device; fp16 sources are taken too (the stacked layout's kernels, which the reference
    runs on any float dtype). Any width and alignment: rows the row-layout kernels do not take go to the any-shape
    kernels."""
    v0 = values[0]
    if not v0.is_cuda or v0.dtype not in _DTYPES:
        return False
    shape = v0.shape
    if shape[-1] < 1 or len(values) > ANY_MAX_SOURCES or len(rstds) != len(values):
        return False
    if base.dtype != v0.dtype or base.shape != shape or base.device != v0.device:
        return False
    for v in values:
        if v.dtype != v0.dtype or v.shape != shape or not v.is_contiguous() or v.device != v0.device:
            return False
    rshape = shape[:-1] + (1,)
    for r in rstds:
        if r.dtype != torch.float32 or r.shape != rshape or not r.is_contiguous():
            return False
    return cbar.dtype == torch.float32 and cbar.shape == shape[:-1] + (len(values),) and cbar.is_contiguous()


def _check_list(base, values, rstds, cbar) -> None:
    if not fused_read_supported(base, values, rstds, cbar):
        raise RuntimeError("delta_attnres HIP read: unsupported inputs (see fused_read_supported)")


def _forward_impl(ctx, q, base, cbar, c0, srcs):
    n = len(srcs) // 2
    values, rstds = srcs[:n], srcs[n:]
    _check_list(base, values, rstds, cbar)
    v0 = values[0]
    d = v0.shape[-1]
    n_tok = v0.numel() // d
    dev = v0.device
    dt = _dtype_code(v0.dtype)
    st = _stream(dev)
    qc = _f32(q)
    c0c = _f32(c0)
    cbar_c = _f32(cbar)
    base_c = base.detach().contiguous()
    out = torch.empty_like(base_c)
    tc = torch.empty((n_tok, n), device=dev, dtype=torch.float32)
    grad = any(ctx.needs_input_grad)      # else no backward: the probabilities are not stored
    prob = torch.empty((n_tok, n), device=dev, dtype=torch.float32) if grad else None
    dots = torch.empty((n, n_tok), device=dev, dtype=torch.float32)
    src = _Src.of(_fast(d, n, base_c, qc, *values), values, rstds, dev)
    _read(src, n, qc, dots, False, base_c, None, 0.0, cbar_c, n, c0c, 1.0, out, tc, prob, None, n_tok, d, dt, st)
    if grad:
        ctx.save_for_backward(qc, cbar_c, c0c, prob, dots, tc, *values, *rstds)
    ctx.n, ctx.q_dtype, ctx.base_shape = n, q.dtype, base.shape
    return out, tc.view(*base.shape[:-1], n)


def _bwd1(src: _Src, n, g, gt, prob, dots, tc, cbar_c, c0c, dr_accum, wz, wz_stride, n_tok, d,
          dtype, dev, cols=None, lam=1.0, g_prop=None, g_h0=None, beta=0.0, dq=None, part=None):
    """Pass 1 of the backward plus the dq reduction; returns (dq fp32, dcbar [n_tok, cols]). src: the sources with the
    scale gradients' addresses (src.dr), on the row-layout kernel when src.fast (chosen with g among its rows;
    g_prop and g_h0 are fresh, aligned allocations), else on the any-shape kernel. prob and dots are the
    forward's probabilities [n_tok, n] and raw scores [n, >= n_tok] (row stride dots.stride(0)). cols = n: cbar_c and c0c
    are the read's own; cols = n - 1: they are the previous read's coefficients and prior (scaled by lam, the newest
    entry implied) and dcbar is the gradient of those coefficients. g_prop / g_h0 receive the iteration-end blend's
    gradients when given. dq: an fp32 row of d to reduce the query gradient into (else a new one). part: a
    [bwd1_parts, d] view (any row stride) that takes the per-workgroup partials instead, left for the caller to
    reduce (dq is then None)."""
    st = _stream(dev)
    cols = n if cols is None else cols
    gt_c = None if gt is None else gt.reshape(n_tok, n).float().contiguous()
    dcbar = torch.empty((n_tok, cols), device=dev, dtype=torch.float32)
    parts = _b1_parts(n_tok, d) if part is None else part.shape[0]
    dq_part = torch.empty((parts, d), device=dev, dtype=torch.float32) if part is None else part
    v, r = src.ptrs()
    head = (v, r, n, _p(g), _p(gt_c), _p(prob), _p(dots), dots.stride(0), _p(tc), _p(cbar_c), cols, _p(c0c), cols,
            float(lam), _inv_sqrt(d), _p(dcbar), cols, src.dr_ptr(), int(dr_accum), _p(wz), wz_stride, _p(dq_part))
    tail = (_p(g_prop), _p(g_h0), float(beta), n_tok, d, dtype, st)
    if src.fast:
        if not _fast(d, n, g, g_prop, g_h0):   # the caller chose src with g among its rows
            raise RuntimeError("delta_attnres HIP read: host source tables with rows the row-layout kernels refuse")
        _run("read_bwd1", *head, dq_part.stride(0), *tail)
    else:
        _run("read_bwd1_any", *head, parts, dq_part.stride(0), *tail)
    if part is not None:
        return None, dcbar
    dq = torch.empty(d, device=dev, dtype=torch.float32) if dq is None else dq
    if n_tok > 0:
        _run("reduce_rows", _p(dq_part), parts, d, _p(dq), st)
    else:
        dq.zero_()
    return dq, dcbar


def _backward_impl(ctx, g, gt, dv, accum):
    """dv: one gradient buffer per source, written (accum False) or added into (accum True) by the kernel."""
    qc, cbar_c, c0c, prob, dots, tc, *rest = ctx.saved_tensors
    n = ctx.n
    values, rstds = rest[:n], rest[n:]
    v0 = values[0]
    d = v0.shape[-1]
    n_tok = v0.numel() // d
    dev = v0.device
    dt = _dtype_code(v0.dtype)
    g = g.to(v0.dtype).contiguous()
    dr = torch.empty((n, n_tok), device=dev, dtype=torch.float32)
    wz = torch.empty((n, n_tok, 2), device=dev, dtype=torch.float32)
    fast = _fast(d, n, g, qc, *values, *dv)
    src = _Src.of(fast, values, rstds, dev, drs=[dr[i] for i in range(n)])
    dq, dcbar = _bwd1(src, n, g, gt, prob, dots, tc, cbar_c, c0c, False, wz, n_tok, n_tok, d, dt, dev)
    for t in dv:
        if t.dtype != v0.dtype or not t.is_contiguous() or t.numel() != v0.numel():
            raise RuntimeError("delta_attnres HIP read: gradient buffers must match the sources")
    if fast:
        _run("read_bwd2_list", L.u64_array(t.data_ptr() for t in dv), n, int(bool(accum)), _p(g), _p(qc), _p(wz),
             n_tok, n_tok, d, dt, _stream(dev))
    else:
        dvt = _dev_addrs((t.data_ptr() for t in dv), dev)
        _run("read_bwd2_list_any", _p(dvt), n, int(bool(accum)), _p(g), _p(qc), _p(wz), n_tok, n_tok, d, dt,
             _stream(dev))
    return dq.to(ctx.q_dtype), g, dcbar.view(*ctx.base_shape[:-1], n), [dr[i].view_as(rstds[i]) for i in range(n)]


class FusedDattnRead(torch.autograd.Function):
    """(out, tc) = FusedDattnRead.apply(q, base, cbar, c0, *values, *rstds) (fused_dattn.py:321-334); backward
    returns (dq, g, dcbar, None, *dv, *dr)."""

    @staticmethod
    def forward(ctx, q: torch.Tensor, base: torch.Tensor, cbar: torch.Tensor, c0: torch.Tensor, *srcs: torch.Tensor):
        return _forward_impl(ctx, q, base, cbar, c0, srcs)

    @staticmethod
    def backward(ctx, g: torch.Tensor, gt: torch.Tensor | None):
        n = ctx.n
        values = ctx.saved_tensors[6:6 + n]
        dv = [torch.empty_like(v) for v in values]   # one tensor per source: autograd releases each as soon as it can
        dq, g_out, dcbar_v, dr = _backward_impl(ctx, g, gt, dv, accum=False)
        return (dq, g_out, dcbar_v, None, *dv, *dr)


class DattnGradAccum:
    """Per-forward-pass state of the list layout's in-kernel gradient accumulation (fused_dattn.py:337-350): the first
    backward of a pass allocates one gradient buffer per source, later backwards add into them inside the kernel
    (prev + round(dv), rounded: autograd's own bf16 accumulation), and read i (read 1 for source 0) returns the
    finished buffer."""
    __slots__ = ("bufs",)

    def __init__(self):
        self.bufs = {}


class FusedDattnReadAcc(torch.autograd.Function):
    """FusedDattnRead with in-kernel gradient accumulation: apply(acc, step, q, base, cbar, c0, *values, *rstds)
    (fused_dattn.py:353-376)."""

    @staticmethod
    def forward(ctx, acc: DattnGradAccum, step: int, q, base, cbar, c0, *srcs):
        out = _forward_impl(ctx, q, base, cbar, c0, srcs)
        ctx.acc, ctx.step = acc, int(step)
        return out

    @staticmethod
    def backward(ctx, g: torch.Tensor, gt: torch.Tensor | None):
        acc, step, n = ctx.acc, ctx.step, ctx.n
        values = ctx.saved_tensors[6:6 + n]
        first = not acc.bufs
        if first:
            for i in range(n):
                acc.bufs[i] = torch.empty_like(values[i])
        elif any(i not in acc.bufs for i in range(n)):
            raise RuntimeError("delta_attnres gradient accumulation: a source without a buffer (reads out of order?)")
        dv = [acc.bufs[i] for i in range(n)]
        dq, g_out, dcbar_v, dr = _backward_impl(ctx, g, gt, dv, accum=not first)
        final = [i == step or (step == 1 and i == 0) for i in range(n)]
        ctx.acc = None                    # release the buffers from this node
        return (None, None, dq, g_out, dcbar_v, None, *[dv[i] if final[i] else None for i in range(n)], *dr)


# ---------------------------------------------------------------------------------------------------------------
# stacked layout (fused_dattn.py:629-793)
# ---------------------------------------------------------------------------------------------------------------
def _alias(stack_tensor: torch.Tensor, s: int) -> torch.Tensor:
    """Slice s of a stack as a tensor that shares its storage but is not an autograd view of it (fused_dattn.py:
    629-636): later slices are written in place, and autograd forbids a custom Function to return a view whose base
    is then modified."""
    sl = stack_tensor[s]
    out = torch.empty(0, dtype=stack_tensor.dtype, device=stack_tensor.device)
    out.set_(stack_tensor.untyped_storage(), sl.storage_offset(), sl.shape, sl.stride())
    return out


def _pair(s: int, i: int) -> int:
    """Row of the (read s >= 1, source i <= s) pair in DattnStack.WZ: reads in order, sources in order."""
    return s * (s + 1) // 2 - 1 + i


class DattnStack:
    """The stacked storage of one forward pass (fused_dattn.py:639-676): V[n_steps, b, t, d] (the updates) and
    R[n_steps, b, t, 1] (their RMS scales). Given `query` (the read queries, (n_steps - 1, d); read s uses row s - 1)
    each write also stores the update's scores against the queries of the reads still to come,
    DOTS[query j, source i, token] fp32, and the reads use them.

    Backward state: dR [n_steps, b, t, 1] (the scales' gradients, accumulated by the reads' backwards, zeroed on the
    first), WZ [pairs, b*t, 2] (per (read, source) pair and token: w = tc - cbar and dz r / sqrt(d)), and per read
    whose backward ran, its output gradient and query with their addresses (`bwd`). The updates' gradients are assembled from those by the
    scales' backwards; dV stays None (no gradient stack is read-modified-written). QT is None (the reference's
    transposed operand for its tensor-core product); QB holds the queries' bf16 parts in the order the write's
    matrix-core product loads them."""
    __slots__ = ("V", "R", "dV", "dR", "n_steps", "n_tok", "d", "eps", "Q", "QT", "QB", "DOTS", "r_done", "WZ", "bwd",
                 "assembled", "neg", "dq_parts", "dq_rows", "wh", "gadd", "h0_ref", "h0_steps", "h0_g", "vptr",
                 "rptr", "drptr", "wout", "fast_d", "src_fast", "src_any", "per_read")

    def __init__(self, n_steps: int, shape, dtype, device, query=None, eps: float = 1e-6):
        b, t, d = shape
        n_steps = int(n_steps)
        if dtype not in _DTYPES:
            raise RuntimeError(f"delta_attnres stacked read: dtype must be bfloat16, float16 or float32, got {dtype}")
        if d < 1 or n_steps < 1 or n_steps > ANY_MAX_SOURCES:
            raise RuntimeError(f"delta_attnres stacked read: unsupported shape d={d} n_steps={n_steps} (d >= 1, "
                               f"1 to {ANY_MAX_SOURCES} steps)")
        self.n_steps, self.n_tok, self.d = n_steps, b * t, d
        # rows the row-layout kernels take (the slices of V are then 16-byte aligned); other widths, and reads of
        # more than MAX_SOURCES sources, run on the any-shape kernels
        self.fast_d = d % 8 == 0 and d <= L.MAX_WIDTH
        self.src_fast = self.src_any = None
        # the updates' gradients: one fp32 sum rounded once (default), or rounded per read as the list layout's
        # per-read gradients are when autograd adds them (LOOP_DATTN_GRAD_ROUNDING=per_read: bitwise the list layout)
        self.per_read = grad_rounding() == "per_read"
        self.V = torch.empty((n_steps, b, t, d), dtype=dtype, device=device)
        self.R = torch.empty((n_steps, b, t, 1), dtype=torch.float32, device=device)
        _require_gpu(self.V, "the stack")
        # the slices' addresses, once: a read over sources 0..n-1 passes these tables (the kernels take n entries)
        self.vptr = _slice_table(self.V)
        self.rptr = _slice_table(self.R)
        self.drptr = None
        self.dV = self.dR = None
        self.WZ = None
        self.bwd = {}
        self.assembled = set()
        self.neg = {}         # s -> (gradient of the write's h, of its x, the added proposal gradient or None),
                              # handed from a separate scale node (_RstdStk) to _WriteDelta
        self.wout = {}        # s -> (weak reference to the write's update, its scale output), until rstd(s) takes it
        self.dq_parts = None  # the fused combines' query-gradient partials, [part][read][d] fp32, and the reads
        self.dq_rows = set()  # whose backward wrote theirs; summed once, by read 1's backward (the pass's last)
        self.wh = {}          # s -> weak reference to the write's h (a fused combine that takes it as its proposal
        self.gadd = {}        # hands its proposal gradient, gadd[s] = (g, beta), to the update's gradient kernel)
        self.h0_ref = None    # the fused iteration-end reads: a weak reference to their h0, their steps, and the
        self.h0_steps = []    # output gradients {step: g} of those whose backward ran -- h0's gradient from the
        self.h0_g = {}        # blends is summed once, by the first of them (the last to run backward)
        self.eps = float(eps)
        self.r_done = [False] * self.n_steps      # R[s] (and the scores of update s) written by the write of s
        self.Q = self.QT = self.QB = self.DOTS = None
        if query is not None:
            self.Q = _f32(query)
            nq = self.Q.shape[0]
            if self.Q.dim() != 2 or self.Q.shape[-1] != d:
                raise RuntimeError(f"delta_attnres stacked read: query must be (n_steps - 1, {d}), "
                                   f"got {tuple(self.Q.shape)}")
        # the write kernel stores the scores of rows it takes against up to MAX_QUERIES queries; otherwise the reads
        # form their scores as they read (the same read, as with LOOP_DATTN_DOTS=0)
        if query is not None and self.fast_d and nq <= L.MAX_QUERIES:
            self.DOTS = torch.empty((max(1, nq), n_steps, b * t), dtype=torch.float32, device=device)
            if nq > 0:   # the queries' bf16 parts: the write's matrix-core operand (every update dtype)
                self.QB = torch.empty(int(L.LIB.ldr_query_parts_elems(nq, d)), dtype=torch.bfloat16, device=device)
                _run("split_queries", _p(self.Q), nq, d, _p(self.QB), _stream(self.Q.device))

    def write(self, s: int, h: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """V[s] = h - x, returned as the update tensor (an alias of the stack's slice, with the autograd edge to
        h and x). The write also stores the update's scale R[s], which rstd(s, ...) then returns."""
        v, r = _WriteDelta.apply(self, s, h, x)
        self.wout[s] = (weakref.ref(v), r)
        return v

    def rstd(self, s: int, delta: torch.Tensor, eps: float) -> torch.Tensor:
        """R[s] = the RMS scale of V[s], returned as an alias of the stack (differentiable through `delta`): the
        scale the write of `delta` stored with it, or computed here for another update or eps."""
        w = self.wout.pop(s, None)
        if w is not None and w[0]() is delta and float(eps) == self.eps:
            return w[1]
        return _RstdStk.apply(self, s, delta, float(eps))

    def src(self, n: int, *rows) -> _Src:
        """The stack's sources for a read of n of them (with the scale gradients' addresses once the backward state
        exists): the host tables for the row-layout kernels when they take the read (n <= MAX_SOURCES, the other
        rows 16-byte aligned), else device arrays of the same addresses, made on first use."""
        if self.fast_d and _fast(self.d, n, *rows):
            if self.src_fast is None or (self.src_fast.dr is None and self.drptr is not None):
                self.src_fast = _Src(True, self.vptr, self.rptr, self.drptr)
            return self.src_fast
        if self.src_any is None or (self.src_any.dr is None and self.dR is not None):
            dev = self.V.device
            self.src_any = _Src(False, _dev_addrs(self.vptr, dev), _dev_addrs(self.rptr, dev),
                                None if self.dR is None else _dev_addrs(self.drptr, dev))
        return self.src_any

    def grads(self):
        """Allocate the backward state on the first backward of the pass; False then, True afterwards."""
        if self.dR is None:
            self.dR = torch.zeros_like(self.R)
            self.drptr = _slice_table(self.dR)
            pairs = self.n_steps * (self.n_steps + 1) // 2 - 1
            self.WZ = torch.empty((max(1, pairs), self.n_tok, 2), dtype=torch.float32, device=self.V.device)
            return False
        return True


def _slice_table(t: torch.Tensor):
    """Device addresses of t[0], t[1], ... (a stack's slices), as the kernels' per-source tables."""
    step = t.stride(0) * t.element_size()
    return L.u64_array(t.data_ptr() + i * step for i in range(t.shape[0]))


def _proposal_grad(added):
    """The proposal gradient a fused combine handed over as (g, beta): g itself, or for an iteration-end blend its
    share round(g - round(beta g)) -- the value the update-gradient kernel adds (torch ops, for the rare paths where
    that kernel did not take it)."""
    g, beta = added
    return g - (g * beta).to(g.dtype) if beta else g


def _assemble(stack: DattnStack, s: int, gr):
    """The finished gradient of update s -- every read of it has run its backward -- formed by one kernel from the
    reads' output gradients and (w, dz r / sqrt(d)) pairs, the scale's gradient gr (dR[s], or None) and, when a read
    took the write's h as its proposal, that read's proposal gradient (added as autograd would add it). Returns
    (dv for the write's h, -dv without the proposal's share for its x, the added (g, beta) or None)."""
    # the reads of update s whose backward ran; rounding per read, from the last read to the first (the order in which
    # autograd adds the list layout's per-read gradients), which puts read s last
    reads = sorted((k for k in stack.bwd if k >= max(s, 1)), reverse=stack.per_read)
    if s in reads:   # read s last: when its output gradient is also the added one, the kernel loads it once
        reads.remove(s)
        reads.append(s)
    v = stack.V[s]
    dv = torch.empty_like(v)
    dv_neg = torch.empty_like(v)
    grc = None if gr is None else gr.float().contiguous()
    added = stack.gadd.pop(s, None)       # (g, beta): the combine that took the write's h as its proposal
    if added is not None and (added[0].shape != v.shape or added[0].dtype != v.dtype
                              or not added[0].is_contiguous()):
        added = (added[0].to(v.dtype).contiguous().view(v.shape), added[1])
    bwd = stack.bwd
    fast = stack.fast_d and _fast(stack.d, len(reads), None if added is None else added[0],
                                  *[bwd[k][0] for k in reads], *[bwd[k][1] for k in reads])
    tables = None
    if reads:
        wz0, wz_row = stack.WZ.data_ptr(), stack.WZ.stride(0) * stack.WZ.element_size()
        tables = ([bwd[k][2] for k in reads], [wz0 + _pair(k, s) * wz_row for k in reads], [bwd[k][3] for k in reads])
    args = (len(reads), _p(v), _p(stack.R[s]), _p(grc), _p(None if added is None else added[0]),
            0.0 if added is None else float(added[1]), int(stack.per_read), _p(dv), _p(dv_neg), stack.n_tok, stack.d,
            _dtype_code(v.dtype), _stream(v.device))
    if fast:
        _run("dv_assemble", *([L.u64_array(t) for t in tables] if tables else [None] * 3), *args)
    else:
        dev_tabs = [_dev_addrs(t, v.device) for t in tables] if tables else None
        _run("dv_assemble_any", *([t.data_ptr() for t in dev_tabs] if dev_tabs else [None] * 3), *args)
    stack.assembled.add(s)
    for k in [k for k in bwd if all(j in stack.assembled for j in range(k + 1))]:
        del bwd[k]                        # every update read by read k has its gradient: drop g_k
    return dv, dv_neg, added


class _WriteDelta(torch.autograd.Function):
    """V[s] = round(h - x), R[s] from the rounded update and the scores against the later read queries, in one pass
    (fused_dattn.py:679-695); a plain subtraction into the slice (and the scale kernel) for layouts the kernel does
    not take. Outputs the update and its scale as aliases of the stack: the scale is what DattnStack.rstd hands the
    reads (the reference's separate _RstdStk node, one autograd node fewer per step).

    Backward: every read of update s takes its scale, so this runs after all of them; the update's gradient is
    assembled here once (_assemble) and returned as (dv, -dv) to (h, x), with any gradient other consumers of the
    update gave it added. When the update's gradient was already assembled by a separate scale node (_RstdStk, for
    a scale of another eps), its (dv, -dv) pair comes from there."""

    @staticmethod
    def forward(ctx, stack: DattnStack, s: int, h: torch.Tensor, x: torch.Tensor):
        ctx.stack, ctx.s = stack, s
        stack.wh[s] = weakref.ref(h)
        out = _alias(stack.V, s)
        r = _alias(stack.R, s)
        V = stack.V
        if (stack.fast_d and h.is_cuda and h.is_contiguous() and x.is_contiguous() and h.dtype == V.dtype == x.dtype
                and h.numel() == x.numel() == stack.n_tok * stack.d and h.shape[-1] == stack.d
                and _aligned(h) and _aligned(x)):
            nq, j_lo, dptr, jstride = 0, 0, None, stack.n_steps * stack.n_tok
            if stack.DOTS is not None:
                nq = stack.Q.shape[0]
                j_lo = min(max(0, s - 1), nq)         # read s' >= s uses query s' - 1: queries j_lo .. nq - 1
                if j_lo < nq:
                    dptr = stack.DOTS[j_lo, s]
            _run("write_dots", _p(h), _p(x), _p(out), _p(r), _p(stack.Q), _p(stack.QB), nq, j_lo, _p(dptr),
                 stack.n_tok, stack.d, jstride, stack.eps, _dtype_code(V.dtype), _stream(V.device))
            stack.r_done[s] = True
        else:
            torch.sub(h, x, out=out)
            _run("rstd_fwd", _p(out), _p(r), stack.n_tok, stack.d, stack.eps, _dtype_code(V.dtype), _stream(V.device))
            stack.r_done[s] = False           # the update has no scores (the reads form them online)
        ctx.set_materialize_grads(False)
        return out, r

    @staticmethod
    def backward(ctx, g: torch.Tensor | None, gr: torch.Tensor | None):
        stack, s = ctx.stack, ctx.s
        ctx.stack = None
        if s not in stack.assembled:         # the update's gradient, from every read of it and its scale
            dh, dx, _ = _assemble(stack, s, gr)
            if g is not None:                # other consumers of the update: their gradient joins both inputs'
                dh, dx = dh + g, dx - g
            return None, None, dh, dx
        prep = stack.neg.pop(s, None)        # (gradient of h, gradient of x, the added proposal gradient or None)
        left = stack.gadd.pop(s, None)       # a proposal gradient no update-gradient kernel took
        if g is None:
            return None, None, None, None
        if prep is not None:
            dh, dx, added = prep
            if (g.data_ptr() == dh.data_ptr() and g.shape == dh.shape and g.stride() == dh.stride()
                    and g.dtype == dh.dtype):
                return None, None, g, dx
            # other consumers of the update added to its gradient: h takes all of it, x all but the proposal's
            return None, None, g, -(g - _proposal_grad(added)) if added is not None else -g
        return None, None, (g if left is None else g + _proposal_grad(left)), -g


class _RstdStk(torch.autograd.Function):
    """The scale of update s as a separate node, for a scale DattnStack.rstd cannot take from the write (an update
    that is not the write's output, or another eps; fused_dattn.py:698-722). Forward: R[s] (the kernel skipped when
    the write stored it with this eps). Backward: the finished gradient of update s (_assemble) -- every read of it
    has run its backward by then -- returned as the update's one gradient."""

    @staticmethod
    def forward(ctx, stack: DattnStack, s: int, x: torch.Tensor, eps: float):
        r = _alias(stack.R, s)
        if not (stack.r_done[s] and eps == stack.eps):      # else the write already stored R[s]
            xc = x.contiguous()
            if xc.numel() != stack.n_tok * stack.d or xc.dtype != stack.V.dtype:
                raise RuntimeError("delta_attnres stacked read: the scale's input must be the stack's update")
            _run("rstd_fwd", _p(xc), _p(r), stack.n_tok, stack.d, float(eps), _dtype_code(xc.dtype),
                 _stream(xc.device))
        ctx.stack, ctx.s, ctx.x = stack, s, x
        return r

    @staticmethod
    def backward(ctx, gr: torch.Tensor):
        stack, s, x = ctx.stack, ctx.s, ctx.x
        if stack.dR is None:
            raise RuntimeError("delta_attnres stacked read: the scale's backward ran before any read's backward")
        dv, dv_neg, added = _assemble(stack, s, gr)
        if dv.shape == x.shape:
            stack.neg[s] = (dv, dv_neg, added)   # the write's backward returns dv_neg for its x input
        ctx.stack = ctx.x = None          # release the stack from this node
        return None, None, dv.view(x.shape), None


class FusedDattnReadStk(torch.autograd.Function):
    """(out, tc) = apply(stack, step, q, base, cbar, c0, *updates, *scales) (fused_dattn.py:725-793): the updates and
    scales are the stack's slices 0..step (inputs only for autograd's bookkeeping; the kernels read the stack).
    Backward returns (None, None, dq, g, dcbar, None, None x n, dR alias for the scales whose last read this is) --
    except that when the base is the write's h of this step (the caller's proposal, as the trainer passes it at every
    read that is not an iteration end) the base's gradient g is added by the update's gradient kernel instead, which
    then returns h's whole gradient, the same bits (its None here)."""

    @staticmethod
    def forward(ctx, stack: DattnStack, step: int, q, base, cbar, c0, *srcs):
        n = len(srcs) // 2
        d, n_tok, dev = stack.d, stack.n_tok, stack.V.device
        if base.dtype != stack.V.dtype or not base.is_contiguous() or base.shape[:-1] != stack.V.shape[1:3]:
            raise RuntimeError("delta_attnres stacked read: base must be contiguous, the stack's dtype and shape")
        if not 1 <= n <= stack.n_steps:
            raise RuntimeError(f"delta_attnres stacked read: {n} sources for a stack of {stack.n_steps}")
        if base.shape[-1] != d:
            raise RuntimeError(f"delta_attnres stacked read: base must have width {d}")
        dt = _dtype_code(stack.V.dtype)
        st = _stream(dev)
        qc = _f32(q)
        c0c = _f32(c0)
        cbar_c = _f32(cbar)
        if cbar_c.numel() != n_tok * n or c0c.numel() != n:
            raise RuntimeError("delta_attnres stacked read: cbar must be (b, t, n) and c0 (n,)")
        out = torch.empty_like(base)
        tc = torch.empty((n_tok, n), device=dev, dtype=torch.float32)
        grad = any(ctx.needs_input_grad)
        prob = torch.empty((n_tok, n), device=dev, dtype=torch.float32) if grad else None
        src = stack.src(n, base, qc)
        stored = stack.DOTS is not None and step >= 1 and all(stack.r_done[:n]) and step - 1 < stack.Q.shape[0]
        # the stored scores of query step - 1 [source, token], else formed (and kept for the backward) as it reads
        dots = stack.DOTS[step - 1] if stored else torch.empty((n, n_tok), device=dev, dtype=torch.float32)
        _read(src, n, qc, dots, stored, base, None, 0.0, cbar_c, n, c0c, 1.0, out, tc, prob, None, n_tok, d, dt, st)
        if grad:
            ctx.save_for_backward(qc, cbar_c, c0c, prob, dots, tc)
        ctx.stack, ctx.step, ctx.n, ctx.q_dtype, ctx.base_shape = stack, int(step), n, q.dtype, base.shape
        # the base is the write's h of this step (the caller's proposal, no blend) and the newest scale comes from
        # that update's scale node, whose backward runs after this one: the base's gradient then goes to the update's
        # gradient kernel, which adds it as autograd would (round(round(dv) + g)), instead of autograd's own add
        wr = stack.wh.get(int(step))
        scale = srcs[-1]
        ctx.linked = (step >= 1 and base.requires_grad and wr is not None and wr() is base and scale.grad_fn is not None
                      and type(scale.grad_fn).__name__ in ("_WriteDeltaBackward", "_RstdStkBackward"))
        return out, tc.view(*base.shape[:-1], n)

    @staticmethod
    def backward(ctx, g: torch.Tensor, gt: torch.Tensor | None):
        qc, cbar_c, c0c, prob, dots, tc = ctx.saved_tensors
        stack, step, n = ctx.stack, ctx.step, ctx.n
        d, n_tok, dev = stack.d, stack.n_tok, stack.V.device
        stack.grads()
        g = g.to(stack.V.dtype).contiguous()
        wz = stack.WZ[_pair(step, 0):_pair(step, 0) + n]
        dq, dcbar = _bwd1(stack.src(n, g), n, g, gt, prob, dots, tc, cbar_c, c0c, True, wz, n_tok, n_tok, d,
                          _dtype_code(stack.V.dtype), dev)
        # for the updates' gradients, formed once per update (the tensors, and their addresses for the kernel tables)
        stack.bwd[step] = (g, qc, g.data_ptr(), qc.data_ptr())
        final = [i == step or (step == 1 and i == 0) for i in range(n)]   # the last read of scale i, in backward order
        gbase = g
        if ctx.linked and ctx.needs_input_grad[3]:
            stack.gadd[step] = (g, 0.0)
            gbase = None
        grads = (None, None, dq.to(ctx.q_dtype), gbase, dcbar.view(*ctx.base_shape[:-1], n), None,
                 *[None] * n, *[_alias(stack.dR, i) if final[i] else None for i in range(n)])
        # Release the stack from this node: ctx attributes live as long as the graph node, and a training loop that
        # keeps each micro-batch's loss until the optimizer step would otherwise keep each micro-batch's stack.
        ctx.stack = None
        return grads


# ---------------------------------------------------------------------------------------------------------------
# extension (no counterpart in the reference module): the caller's glue fused into the stacked read
# ---------------------------------------------------------------------------------------------------------------
class FusedCombineStk(torch.autograd.Function):
    """One read of `LoopDeltaAttnRes.combine` (modeling_looped_transformer.py:148-169) for step >= 1 on the stacked
    layout, with the caller's glue inside the kernels: the iteration-end blend base = proposal + beta (h0 - proposal)
    (rounded step by step as the caller's ops round), the bookkeeping cbar = lam [coeffs, 1], c0 = lam [prior, 1]
    (lam = 1 - beta at an iteration end, else 1), and next_prior = c0 written by the read. The read itself is
    FusedDattnReadStk's. Backward: the blend's gradients (g - beta g to the proposal, beta g to h0) and the
    coefficients' gradient lam (-g.v) come out of backward pass 1; no separate glue kernels. The query is the whole
    (n_steps - 1, d) parameter (read `step` uses row step - 1): each backward reduces its row straight into the stack's
    fp32 query gradient, which the last backward of the pass (read 1) returns -- one gradient tensor per pass instead
    of a zero-filled one per read.

    (out, tc, next_prior) = apply(stack, step, query, proposal, h0, coeffs, prior, beta, at_boundary, *scales) with
    coeffs (b, t, n-1) and prior (n-1,) the previous read's outputs and scales the n sources' scales (DattnStack.rstd:
    the reads' autograd edges to the updates' gradient nodes; the updates themselves are read from the stack);
    next_prior carries no gradient (the prior is a constant of the schedule, as in the reference)."""

    @staticmethod
    def forward(ctx, stack: DattnStack, step: int, query, proposal, h0, coeffs, prior, beta: float, at_boundary: bool,
                *scales):
        n = len(scales)
        d, n_tok, dev = stack.d, stack.n_tok, stack.V.device
        if (proposal.dtype != stack.V.dtype or not proposal.is_contiguous() or proposal.shape[:-1] != stack.V.shape[1:3]
                or proposal.shape[-1] != d):
            raise RuntimeError("delta_attnres fused combine: proposal must be contiguous, the stack's dtype and shape")
        if at_boundary and (h0 is None or h0.dtype != proposal.dtype or h0.shape != proposal.shape
                            or not h0.is_contiguous()):
            raise RuntimeError("delta_attnres fused combine: h0 must match the proposal at an iteration end")
        if not 2 <= n <= stack.n_steps or n != step + 1:
            raise RuntimeError(f"delta_attnres fused combine: {n} sources at step {step} of a stack of {stack.n_steps}")
        if query.dim() != 2 or query.shape[-1] != d or not 1 <= step <= query.shape[0]:
            raise RuntimeError(f"delta_attnres fused combine: query must be (n_steps - 1, {d}) with a row for step {step}")
        dt = _dtype_code(stack.V.dtype)
        st = _stream(dev)
        lam = 1.0 - float(beta) if at_boundary else 1.0
        qc = _f32(query[step - 1])
        coeffs_c = _f32(coeffs)
        prior_c = _f32(prior)
        if coeffs_c.numel() != n_tok * (n - 1) or prior_c.numel() != n - 1:
            raise RuntimeError("delta_attnres fused combine: coeffs must be (b, t, n-1) and prior (n-1,)")
        out = torch.empty_like(proposal)
        tc = torch.empty((n_tok, n), device=dev, dtype=torch.float32)
        grad = any(ctx.needs_input_grad)      # else no backward: the probabilities are not stored
        prob = torch.empty((n_tok, n), device=dev, dtype=torch.float32) if grad else None
        next_prior = torch.empty(n, device=dev, dtype=torch.float32)
        h0b = h0 if at_boundary else None
        src = stack.src(n, proposal, h0b, qc)
        stored = stack.DOTS is not None and all(stack.r_done[:n]) and step - 1 < stack.Q.shape[0]
        dots = stack.DOTS[step - 1] if stored else torch.empty((n, n_tok), device=dev, dtype=torch.float32)
        _read(src, n, qc, dots, stored, proposal, h0b, beta, coeffs_c, n - 1, prior_c, lam, out, tc, prob, next_prior,
              n_tok, d, dt, st)
        if grad:
            ctx.save_for_backward(qc, coeffs_c, prior_c, prob, dots, tc)
        ctx.stack, ctx.step, ctx.n, ctx.shape = stack, int(step), n, proposal.shape
        ctx.q_shape, ctx.q_dtype = query.shape, query.dtype
        ctx.beta, ctx.at_boundary, ctx.lam = float(beta), bool(at_boundary), lam
        # the proposal is the write's h of this step and the newest scale comes from that update's scale node: the
        # proposal's gradient then goes to the update's gradient kernel, which adds it (no separate add)
        wr = stack.wh.get(step)
        scale = scales[step]
        ctx.linked = (proposal.requires_grad and wr is not None and wr() is proposal and scale.grad_fn is not None
                      and type(scale.grad_fn).__name__ in ("_WriteDeltaBackward", "_RstdStkBackward"))
        # an iteration end with the pass's h0: its share of h0's gradient is summed with the other ends' at the
        # first of them (the last to run backward) instead of being written here and added by autograd
        ctx.h0_sum = False
        if at_boundary and h0.requires_grad and (stack.h0_ref is None or stack.h0_ref() is h0):
            stack.h0_ref = weakref.ref(h0)
            stack.h0_steps.append(int(step))
            ctx.h0_sum = True
        ctx.mark_non_differentiable(next_prior)
        ctx.set_materialize_grads(False)
        return out, tc.view(*proposal.shape[:-1], n), next_prior

    @staticmethod
    def backward(ctx, g: torch.Tensor | None, gt: torch.Tensor | None, gnp):
        qc, coeffs_c, prior_c, prob, dots, tc = ctx.saved_tensors
        stack, step, n = ctx.stack, ctx.step, ctx.n
        d, n_tok, dev = stack.d, stack.n_tok, stack.V.device
        stack.grads()
        nq = ctx.q_shape[0]
        parts = _b1_parts(n_tok, d)
        if stack.dq_parts is None or stack.dq_parts.shape != (parts, nq, d):
            # every read's dq partials, interleaved [part][read][d]: one reduction at the pass's last read
            stack.dq_parts = torch.empty((parts, nq, d), device=dev, dtype=torch.float32)
            stack.dq_rows = set()
        g = torch.zeros(ctx.shape, device=dev, dtype=stack.V.dtype) if g is None else g.to(stack.V.dtype).contiguous()
        # the blend's gradients are written only where no later kernel forms them from g
        need_prop, need_h0 = ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        g_prop = torch.empty_like(g) if ctx.at_boundary and not ctx.linked and need_prop else None
        g_h0 = torch.empty_like(g) if ctx.at_boundary and not ctx.h0_sum and need_h0 else None
        wz = stack.WZ[_pair(step, 0):_pair(step, 0) + n]
        _, dcoeffs = _bwd1(stack.src(n, g), n, g, gt, prob, dots, tc, coeffs_c, prior_c, True, wz, n_tok, n_tok, d,
                           _dtype_code(stack.V.dtype), dev, cols=n - 1, lam=ctx.lam, g_prop=g_prop, g_h0=g_h0,
                           beta=ctx.beta, part=stack.dq_parts[:, step - 1, :])
        stack.dq_rows.add(step - 1)
        stack.bwd[step] = (g, qc, g.data_ptr(), qc.data_ptr())
        final = [i == step or (step == 1 and i == 0) for i in range(n)]
        dquery = None
        if step == 1:   # read 1's backward is the pass's last: every read's partials, summed in one launch
            for j in set(range(nq)) - stack.dq_rows:   # reads with no backward in this pass (none, normally)
                stack.dq_parts[:, j, :].zero_()
            dq = torch.empty((nq, d), device=dev, dtype=torch.float32)
            if n_tok > 0:
                _run("reduce_rows", _p(stack.dq_parts), parts, nq * d, _p(dq), _stream(dev))
            else:
                dq.zero_()
            dquery = dq.to(ctx.q_dtype)
            stack.dq_parts, stack.dq_rows = None, set()
        dprop = (g_prop if ctx.at_boundary else g) if need_prop else None
        if ctx.linked:
            stack.gadd[step] = (g, ctx.beta if ctx.at_boundary else 0.0)
            dprop = None
        dh0 = g_h0
        if ctx.h0_sum:
            stack.h0_g[step] = g
            if step == min(stack.h0_steps):   # every other iteration end ran its backward: their sum, once
                # rounding per read: from the last iteration end to the first, as autograd adds the blends' shares
                gs = [stack.h0_g[k] for k in sorted(stack.h0_g, reverse=stack.per_read)]
                dh0 = torch.empty_like(g)
                tail = (len(gs), ctx.beta, int(stack.per_read), _p(dh0), n_tok, d, _dtype_code(stack.V.dtype),
                        _stream(dev))
                if stack.fast_d and _fast(d, len(gs), dh0, *gs):
                    _run("blend_sum", L.u64_array(x.data_ptr() for x in gs), *tail)
                else:
                    gt_ = _dev_addrs((x.data_ptr() for x in gs), dev)
                    _run("blend_sum_any", gt_.data_ptr(), *tail)
                stack.h0_g, stack.h0_steps = {}, []
                dh0 = dh0.view(ctx.shape)
        grads = (None, None, dquery, dprop, dh0,
                 dcoeffs.view(*ctx.shape[:-1], n - 1), None, None, None,
                 *[_alias(stack.dR, i) if final[i] else None for i in range(n)])
        ctx.stack = None
        return grads
