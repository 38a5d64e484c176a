"""The HIP read (list layout, the caller's FusedDattnRead path) against the oracle -- the restated reference read
LoopDeltaAttnRes.combine -- on the same seeded inputs; mirrors tests/test_fused_dattn.py:87-125 of the reference.

  1. fp32: out, tc and every gradient (the query row, each delta through its value and its RMS scale, proposal and
     h0 through base, the previous coefficients) within max-abs 1e-5 x RMS of the reference read evaluated exactly
     (the fp64 oracle on the same fp32 inputs), and within 2e-5 x RMS of the fp32 oracle (two fp32 evaluations,
     each with its own round-off), over ragged token counts, 2..20 sources, boundary and in-iteration reads,
     d in {768, 1024, 1536, 3072};
  2. bf16: against the reference read evaluated exactly (the fp64 oracle on the same bf16-rounded inputs): max-abs
     error <= 1e-2 x max |ref| for what the kernels compute (out, tc, dq, dv, dcbar), and for everything no worse
     than the reference read's own bf16 error (<= 2 err_ref + 2e-3) -- dproposal / dh0 come from the caller's
     bf16 torch glue, the same ops as the reference's; against the bf16 reference read itself (whose gradients
     round every per-source term to bf16): norm-relative <= 1e-2 for outputs and all gradients;
     fp16 to the bf16 bars 8 times tighter (2^-11 against 2^-8 rounding);
  3. zero query, cbar == prior: out == base and tc == c0 bitwise, fp32, bf16 and fp16;
  4. the layout's extremes in fp32: one token, d = 8, 40, 2056, 8192, 64 sources; extreme values (a saturated
     softmax, priors under the clamp, large updates beside an all-zero one).
"""
import pytest
import torch

from gpu_helpers import DEV, err_max, err_norm, err_rms, lib_dtype, lowp, make, ulp_rel
from oracle.reference_read import OracleCell

pytestmark = pytest.mark.gpu


def run_hip(d, n, args, boundary, beta=0.75):
    from loopback_amd.cell import LoopDeltaAttnRes
    deltas, proposal, h0, q, prior, coeffs, up, up2 = [
        [x.to(DEV).requires_grad_() for x in a] if isinstance(a, list) else a.to(DEV) for a in args]
    proposal.requires_grad_()
    h0.requires_grad_()
    nb = n if boundary else n + 1
    cell = LoopDeltaAttnRes(d, num_loops=2, num_blocks=nb, beta=beta, eps=1e-6).to(DEV)
    with torch.no_grad():
        cell.query[n - 2].copy_(q)
    cf = coeffs.detach().clone().requires_grad_()
    out, tc, _ = cell.combine(proposal, h0, deltas, cf, prior, 0, n - 1)
    ((out.float() * up).sum() + (tc * up2).sum()).backward()
    torch.cuda.synchronize()
    return dict(out=out.detach(), tc=tc.detach(), dq=cell.query.grad[n - 2], dv=[x.grad for x in deltas],
                dprop=proposal.grad, dh0=h0.grad, dcoef=cf.grad)


def run_oracle(d, n, args, boundary, beta=0.75, dtype=None):
    deltas, proposal, h0, q, prior, coeffs, up, up2 = args
    cast = (lambda x: x.to(dtype)) if dtype is not None else (lambda x: x)
    deltas = [cast(x).detach().clone().requires_grad_() for x in deltas]
    proposal = cast(proposal).detach().clone().requires_grad_()
    h0 = cast(h0).detach().clone().requires_grad_()
    f = (lambda x: x.double()) if dtype == torch.float64 else (lambda x: x)
    nb = n if boundary else n + 1
    query = torch.zeros(2 * nb - 1, d, dtype=torch.float64 if dtype == torch.float64 else torch.float32)
    query[n - 2] = f(q)
    query.requires_grad_()
    cf = f(coeffs).detach().clone().requires_grad_()
    cell = OracleCell(d, 2, nb, beta, 1e-6, query)
    out, tc, _ = cell.combine(proposal, h0, deltas, cf, f(prior), 0, n - 1)
    ((out.to(f(up).dtype) * f(up)).sum() + (tc * f(up2)).sum()).backward()
    return dict(out=out.detach(), tc=tc.detach(), dq=query.grad[n - 2], dv=[x.grad for x in deltas],
                dprop=proposal.grad, dh0=h0.grad, dcoef=cf.grad)


def compare(a, b, fn):
    e = {k: fn(a[k], b[k]) for k in ("out", "tc", "dq", "dprop", "dcoef")}
    e["dv"] = max(fn(x, y) for x, y in zip(a["dv"], b["dv"]))
    e["dh0"] = fn(a["dh0"], b["dh0"]) if b["dh0"] is not None and b["dh0"].abs().max() > 0 else 0.0
    return e


SHAPES_FP32 = [(2, 64, 768), (2, 37, 1024), (1, 50, 1536), (1, 9, 3072)]


@pytest.mark.parametrize("b,t,d", SHAPES_FP32)
@pytest.mark.parametrize("n", [2, 3, 8, 16, 20])
@pytest.mark.parametrize("boundary", [False, True])
def test_fp32_matches_reference_read(b, t, d, n, boundary):
    args = make(b, t, d, n, torch.float32, seed=1000 * n + d + int(boundary))
    print(f"case fp32 b{b} t{t} d{d} n{n} boundary={boundary}", flush=True)
    hip = run_hip(d, n, args, boundary)
    ref = run_oracle(d, n, args, boundary)
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    e32 = compare(hip, ref, err_rms)
    assert max(e64.values()) <= 1e-5, e64
    assert max(e32.values()) <= 2e-5, e32


@pytest.mark.parametrize("b,t,d,n", [(1, 1, 8, 2), (1, 3, 40, 5), (1, 17, 8192, 3), (2, 5, 64, 64), (1, 33, 2056, 7)])
@pytest.mark.parametrize("boundary", [False, True])
def test_fp32_edge_shapes(b, t, d, n, boundary):
    """The extremes of the layout: one token, the narrowest row (d = 8), rows that are no power of two of vectors
    (d = 40, 2056), the widest row (d = 8192: 256 lanes x 4 vectors), the most sources a read takes (64)."""
    args = make(b, t, d, n, torch.float32, seed=31 * n + d + int(boundary))
    print(f"case fp32 edge b{b} t{t} d{d} n{n} boundary={boundary}", flush=True)
    hip = run_hip(d, n, args, boundary)
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    assert max(e64.values()) <= 1e-5, e64


@pytest.mark.parametrize("boundary", [False, True])
def test_fp32_extreme_inputs(boundary):
    """Conditions the reference read meets at the edges of training: a query large enough to saturate the softmax
    (logits ~ +-50), priors below the 1e-8 clamp, updates of magnitude 1e3 next to an all-zero update (its scale is
    rsqrt(eps) = 1000 and its score 0). No inf / nan, and against the exact read the 1e-5 x RMS fp32 bar -- or, where
    the problem's conditioning puts the reference read itself in fp32 above it (the updates' gradients here, ~5e-5),
    no worse than that reference read."""
    b, t, d, n = 2, 33, 512, 6
    deltas, proposal, h0, q, prior, coeffs, up, up2 = make(b, t, d, n, torch.float32, seed=77)
    deltas = [x * 1e3 for x in deltas[:-2]] + [torch.zeros_like(deltas[-2]), deltas[-1]]
    q = q * 60.0
    prior = prior.clone()
    prior[0], prior[2] = 1e-12, 3e-9
    coeffs = prior.view(1, 1, -1) + 0.2 * torch.randn(b, t, n - 1, generator=torch.Generator().manual_seed(78))
    args = (deltas, proposal, h0, q, prior, coeffs, up, up2)
    print(f"case fp32 extreme boundary={boundary}", flush=True)
    hip = run_hip(d, n, args, boundary)
    for k, v in hip.items():
        for x in (v if isinstance(v, list) else [v]):
            assert x is None or torch.isfinite(x).all(), k
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    er = compare(run_oracle(d, n, args, boundary), ref64, err_rms)
    assert all(e64[k] <= max(1e-5, er[k]) for k in e64), (e64, er)


@pytest.mark.parametrize("b,t,d", [(2, 256, 1024), (2, 128, 1536), (4, 128, 768)])
@pytest.mark.parametrize("n", [4, 16, 20])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_16bit_against_fp64(b, t, d, n, dtype):
    """bf16 to the bars of the module docstring; fp16 (the stacked layout's dtype under fp16 mixed precision) to the
    same bars 8 times tighter (fp16 rounds to 2^-11, bf16 to 2^-8)."""
    args = make(b, t, d, n, dtype, seed=7 * n + d)
    print(f"case {dtype} b{b} t{t} d{d} n{n}", flush=True)
    hip = run_hip(d, n, args, boundary=True)
    ref_lp = run_oracle(d, n, args, boundary=True)
    ref64 = run_oracle(d, n, args, boundary=True, dtype=torch.float64)
    eb = compare(hip, ref_lp, err_norm)
    ef = compare(hip, ref64, err_max)
    er = compare(ref_lp, ref64, err_max)
    assert max(eb.values()) <= lowp(1e-2, dtype), eb
    assert max(ef[k] for k in ("out", "tc", "dq", "dv", "dcoef")) <= lowp(1e-2, dtype), ef
    assert all(ef[k] <= 2.0 * er[k] + lowp(2e-3, dtype) for k in er), (ef, er)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [2, 9, 16])
@pytest.mark.parametrize("boundary", [False, True])
def test_zero_query_identity_bitwise(dtype, n, boundary):
    from loopback_amd import fused_dattn as FD
    b, t, d = 2, 40, 768
    deltas, proposal, h0, q, prior, coeffs, up, up2 = make(b, t, d, n, dtype, seed=n, zero_query=True)
    deltas = [x.to(DEV) for x in deltas]
    proposal, h0, q, prior = proposal.to(DEV), h0.to(DEV), q.to(DEV), prior.to(DEV)
    coeffs = prior.view(1, 1, -1).expand(b, t, -1).contiguous()
    base = proposal + 0.75 * (h0 - proposal) if boundary else proposal
    base_coeffs = torch.cat((coeffs, torch.ones(b, t, 1, device=DEV)), -1)
    next_prior = torch.cat((prior, torch.ones(1, device=DEV)), -1)
    if boundary:
        base_coeffs, next_prior = 0.25 * base_coeffs, 0.25 * next_prior
    rstds = [FD.rstd(x, 1e-6) for x in deltas]
    with torch.no_grad():
        out, tc = FD.FusedDattnRead.apply(q, base, base_coeffs, next_prior, *deltas, *rstds)
    assert torch.equal(out, base)
    assert torch.equal(tc, next_prior.view(1, 1, -1).expand(b, t, -1))


@pytest.mark.parametrize("shape,offset", [((3, 33, 1536), 0), ((2, 17, 100), 0), ((1, 9, 7), 0), ((2, 5, 8200), 0),
                                          ((2, 11, 768), 1)])
def test_rstd_matches_reference_scale(shape, offset):
    """rstd and its backward against fp64 autograd of the torch expression. As the reference's masked kernels, any
    width, alignment and float dtype: the vector rows (bf16 and fp32, d a multiple of 8, aligned) and the scalar rows
    (d = 100, 7, 8200 above the widest vector row, rows one element off 16-byte alignment, and fp16)."""
    from loopback_amd import fused_dattn as FD
    from oracle.reference_read import rstd_ref
    b, t, d = shape
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        flat = (torch.randn(b * t * d + offset, generator=torch.Generator().manual_seed(4)) * 1.7).to(dtype)
        fg = flat.to(DEV).requires_grad_()
        xg = fg[offset:].view(b, t, d)   # contiguous; offset 1 leaves it off 16-byte alignment
        print(f"case rstd {shape} offset={offset} {dtype}", flush=True)
        r = FD.rstd(xg, 1e-6)
        gr = torch.randn(b, t, 1, generator=torch.Generator().manual_seed(5))
        (r * gr.to(DEV)).sum().backward()
        xc = flat[offset:].view(b, t, d).double().requires_grad_()
        rr = rstd_ref(xc, 1e-6)
        (rr * gr.double()).sum().backward()
        assert err_rms(r.detach(), rr.detach()) <= 1e-6
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        assert err_max(fg.grad[offset:].view(b, t, d), xc.grad) <= tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,d,n", [(300, 2048, 31), (77, 768, 9), (41, 64, 64), (50, 1024, 3), (33, 3072, 5)])
@pytest.mark.parametrize("boundary", [False, True])
@pytest.mark.parametrize("q_std", [0.0, 0.05, 30.0])
def test_one_pass_online_read_matches_two_passes(dtype, T, d, n, boundary, q_std):
    """ldr_read_fwd_online (scores formed as the sources stream, an online softmax against a running maximum) against
    ldr_dots_online + ldr_read_fwd on the same inputs, through the C ABI: the stored raw scores bitwise; tc and p to
    fp32 round-off (their softmax is the same function over the same logits, spread over other lanes); out to the
    fp32 bar (1e-5 x RMS; bf16, fp16: one rounding of an fp32 sum, so within 1 ulp at |out|); a zero query gives
    the two-pass out and tc bitwise (no online sum is formed; tc == c0). q_std 30 saturates the softmax (rescales of the running
    sums); d = 3072 takes two passes inside the call (rows wider than a wave)."""
    from loopback_amd import _lib as L
    gen = torch.Generator().manual_seed(T * 7 + d + n + int(boundary) + int(q_std))
    dt = lib_dtype(dtype)
    vs = [torch.randn(T, d, generator=gen).to(dtype).to(DEV) for _ in range(n)]
    rs = [torch.rsqrt(v.float().pow(2).mean(-1) + 1e-6).contiguous() for v in vs]
    q = (torch.randn(d, generator=gen) * q_std).to(DEV)
    base = torch.randn(T, d, generator=gen).to(dtype).to(DEV)
    h0 = torch.randn(T, d, generator=gen).to(dtype).to(DEV) if boundary else None
    cols = n - 1 if boundary else n
    cbar = (torch.rand(T, cols, generator=gen) + 0.1).to(DEV)
    c0 = (torch.rand(cols, generator=gen) + 0.1).to(DEV)
    lam = 0.25 if boundary else 1.0
    vp = L.u64_array(v.data_ptr() for v in vs)
    rp = L.u64_array(r.data_ptr() for r in rs)
    st = torch.cuda.current_stream().cuda_stream
    res = []
    for one_pass in (True, False):
        out = torch.empty(T, d, dtype=dtype, device=DEV)
        tc = torch.empty(T, n, device=DEV)
        p = torch.empty(T, n, device=DEV)
        npr = torch.empty(n, device=DEV)
        dots = torch.full((n, T), float("nan"), device=DEV)
        tail = (base.data_ptr(), h0.data_ptr() if boundary else None, 0.75, cbar.data_ptr(), cols, c0.data_ptr(),
                cols, lam, d ** -0.5, out.data_ptr(), tc.data_ptr(), p.data_ptr(), npr.data_ptr(), T, d, dt, st)
        if one_pass:
            L.check(L.LIB.ldr_read_fwd_online(vp, rp, n, q.data_ptr(), dots.data_ptr(), T, *tail), "read_fwd_online")
        else:
            L.check(L.LIB.ldr_dots_online(vp, n, q.data_ptr(), dots.data_ptr(), T, T, d, dt, st), "dots_online")
            L.check(L.LIB.ldr_read_fwd(vp, rp, n, dots.data_ptr(), T, *tail), "read_fwd")
        torch.cuda.synchronize()
        res.append((out, tc, p, npr, dots))
    (o1, tc1, p1, np1, d1), (o2, tc2, p2, np2, d2) = res
    assert torch.equal(d1, d2) and torch.equal(np1, np2)
    assert torch.isfinite(o1.float()).all() and torch.isfinite(tc1).all()
    assert (p1 - p2).abs().max().item() <= 1e-6
    if q_std == 0.0:
        assert torch.equal(o1, o2) and torch.equal(tc1, tc2)
        return
    assert (tc1 - tc2).abs().max().item() <= 1e-6 * tc2.abs().max().item()
    if dtype == torch.float32:
        assert err_rms(o1, o2) <= 1e-5
    else:
        a, b = o1.float(), o2.float()
        scale = b.pow(2).mean().sqrt().item()
        assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * ulp_rel(dtype) + 2e-5 * scale).all()


@pytest.mark.parametrize("order", ["rising", "falling", "alternating"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_online_read_rescale_paths(order, dtype):
    """The one-pass online read against the two-pass read (C ABI) when every source moves the running maximum:
    sources v_i = cos(t_i) u + sin(t_i) w with u along the query and w orthogonal to it give logits |q| cos(t_i)
    (the RMS scale removes the magnitude), here spread over [-120, 120] rising, falling or alternating across 31
    sources, so the reference maximum moves (and the sums are rescaled) at most sources, or never after the first."""
    from loopback_amd import _lib as L
    T, d, n = 64, 1024, 31
    gen = torch.Generator().manual_seed(5)
    qdir = torch.randn(d, generator=gen)
    qdir /= qdir.norm()
    w = torch.randn(T, d, generator=gen)
    w -= (w @ qdir)[:, None] * qdir[None, :]
    w /= w.norm(dim=1, keepdim=True)
    zs = torch.linspace(-0.99, 0.99, n)
    if order == "falling":
        zs = zs.flip(0)
    elif order == "alternating":
        zs = torch.stack([zs[: (n + 1) // 2], torch.cat([zs[(n + 1) // 2:], zs[:1]])], 1).flatten()[:n]
    vs = [((c * qdir[None, :] + (1 - c * c) ** 0.5 * w) * (1.0 + 0.1 * i)).to(dtype).to(DEV)
          for i, c in enumerate(zs.tolist())]
    rs = [torch.rsqrt(v.float().pow(2).mean(-1) + 1e-6).contiguous() for v in vs]
    q = (qdir * 120.0).to(DEV)   # r (q . v) / sqrt(d) = |q| cos t_i r |v| / sqrt(d) = 120 cos t_i (r |v| = sqrt(d))
    base = torch.randn(T, d, generator=gen).to(dtype).to(DEV)
    cbar = (torch.rand(T, n, generator=gen) + 0.1).to(DEV)
    c0 = (torch.rand(n, generator=gen) + 0.1).to(DEV)
    dt = lib_dtype(dtype)
    vp = L.u64_array(v.data_ptr() for v in vs)
    rp = L.u64_array(r.data_ptr() for r in rs)
    st = torch.cuda.current_stream().cuda_stream
    res = []
    for one_pass in (True, False):
        out = torch.empty(T, d, dtype=dtype, device=DEV)
        tc = torch.empty(T, n, device=DEV)
        p = torch.empty(T, n, device=DEV)
        dots = torch.empty(n, T, device=DEV)
        tail = (base.data_ptr(), None, 0.0, cbar.data_ptr(), n, c0.data_ptr(), n, 1.0, d ** -0.5, out.data_ptr(),
                tc.data_ptr(), p.data_ptr(), None, T, d, dt, st)
        if one_pass:
            L.check(L.LIB.ldr_read_fwd_online(vp, rp, n, q.data_ptr(), dots.data_ptr(), T, *tail), "read_fwd_online")
        else:
            L.check(L.LIB.ldr_dots_online(vp, n, q.data_ptr(), dots.data_ptr(), T, T, d, dt, st), "dots_online")
            L.check(L.LIB.ldr_read_fwd(vp, rp, n, dots.data_ptr(), T, *tail), "read_fwd")
        torch.cuda.synchronize()
        res.append((out, tc, p, dots))
    (o1, tc1, p1, d1), (o2, tc2, p2, d2) = res
    z = d1 * torch.stack(rs) * d ** -0.5
    assert z.max().item() > 100 and z.min().item() < -100   # the logits do span the range
    assert torch.equal(d1, d2)
    assert torch.isfinite(o1.float()).all() and (p1 - p2).abs().max().item() <= 1e-6
    if dtype == torch.float32:
        assert err_rms(o1, o2) <= 1e-5
    else:
        a, b = o1.float(), o2.float()
        scale = b.pow(2).mean().sqrt().item()
        assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * ulp_rel(dtype) + 2e-5 * scale).all()
