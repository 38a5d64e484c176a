"""The any-shape kernels (the *_any entry points) against the oracle: the shapes the row-layout kernels do not
take -- widths that are not a multiple of 8 or exceed LDR_MAX_WIDTH, reads of more than LDR_MAX_SOURCES sources (a
stack of more than 64 steps, as an evaluation with more iterations than trained builds), rows that are not 16-byte
aligned. The reference's kernels mask any width and source count (fused_dattn.py:60-63, 191-194) and its DattnStack
takes any shape (fused_dattn.py:647-661); these tests hold the same paths to the same bars as the row-layout ones:

  1. single list reads (FusedDattnRead through cell.combine), fp32: out, tc and every gradient within max-abs
     1e-5 x RMS of the reference read evaluated exactly (fp64 oracle), d in {1, 12, 100, 8200}, in-iteration and
     iteration-end reads; sources that start 2 bytes past a 16-byte boundary (views into a larger buffer);
  2. K x R chains, fwd+bwd, every mode and both glue paths, fp32, bf16 and fp16 (the chain bars of test_gpu_stack:
     check_chain), at d = 100 and d = 8200;
  3. a 70-step stacked chain (reads of up to 70 sources; the write stores no scores for more than 64 queries, so the
     reads form them) against the exact chain, fwd+bwd and no-grad;
  4. the zero-query identity out == base, tc == c0 bitwise;
  5. entry-point level, at a shape both kernel families take: the update gradient and the blend sum of the
     any-shape kernels are bitwise those of the row-layout kernels on the same tables; the read and backward pass 1
     agree with them to fp32 round-off.
"""
import itertools

import pytest
import torch

from gpu_helpers import DEV, err_rms, lib_dtype, lowp, make, within_ulps
from test_gpu_read import compare, run_hip, run_oracle
from test_gpu_stack import check_chain, grad_list, hip_chain, ref_chain

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,t,d,n", [(1, 5, 1, 3), (2, 9, 12, 4), (1, 33, 100, 7), (1, 6, 8200, 3)])
@pytest.mark.parametrize("boundary", [False, True])
def test_list_read_any_width(b, t, d, n, boundary):
    args = make(b, t, d, n, torch.float32, seed=53 * n + d + int(boundary))
    print(f"case any-width read b{b} t{t} d{d} n{n} boundary={boundary}", flush=True)
    hip = run_hip(d, n, args, boundary)
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    assert max(e64.values()) <= 1e-5, e64


def test_list_read_any_width_many_tokens():
    """A ragged 40001 tokens at d = 100: every any-shape kernel takes several rows per wave (grid-stride loops) and
    backward pass 1 spreads the tokens over its 512 partial rows; fp32 against the exact read, 1e-5 x RMS."""
    b, t, d, n = 1, 40001, 100, 5
    args = make(b, t, d, n, torch.float32, seed=401)
    print(f"case any-width read t{t} d{d} n{n}", flush=True)
    hip = run_hip(d, n, args, True)
    ref64 = run_oracle(d, n, args, True, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    assert max(e64.values()) <= 1e-5, e64


def test_list_read_many_sources():
    """A read of 80 sources (more than the row-layout kernels' 64)."""
    b, t, d, n = 1, 7, 64, 80
    args = make(b, t, d, n, torch.float32, seed=80)
    print(f"case any read n{n}", flush=True)
    hip = run_hip(d, n, args, True)
    ref64 = run_oracle(d, n, args, True, dtype=torch.float64)
    e64 = compare(hip, ref64, err_rms)
    assert max(e64.values()) <= 1e-5, e64


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_list_read_unaligned_rows(dtype):
    """Sources, proposal and h0 as contiguous views starting one element past a 16-byte boundary: the row-layout
    kernels' vector loads cannot take them; the same values through the aligned path give the same result."""
    from loopback_amd.cell import LoopDeltaAttnRes
    b, t, d, n = 1, 24, 256, 5
    deltas, proposal, h0, q, prior, coeffs, up, up2 = make(b, t, d, n, dtype, seed=91)
    print(f"case unaligned read {dtype}", flush=True)

    def shifted(x):
        buf = torch.empty(x.numel() + 8, dtype=x.dtype, device=DEV)
        v = buf[1:1 + x.numel()].view(x.shape)
        v.copy_(x.to(DEV))
        assert v.data_ptr() % 16 != 0 and v.is_contiguous()
        return v

    def run(conv):
        dl = [conv(x).requires_grad_() for x in deltas]
        p, h = conv(proposal).requires_grad_(), conv(h0).requires_grad_()
        cell = LoopDeltaAttnRes(d, num_loops=2, num_blocks=n, beta=0.75, eps=1e-6).to(DEV)
        with torch.no_grad():
            cell.query[n - 2].copy_(q)
        cf = coeffs.to(DEV).requires_grad_()
        out, tc, _ = cell.combine(p, h, dl, cf, prior.to(DEV), 0, n - 1)
        ((out.float() * up.to(DEV)).sum() + (tc * up2.to(DEV)).sum()).backward()
        torch.cuda.synchronize()
        return [out, tc, cell.query.grad, p.grad, h.grad, cf.grad] + [x.grad for x in dl]

    got = run(lambda x: shifted(x).detach())
    ref = run(lambda x: x.to(DEV).clone())
    tol = 1e-5 if dtype == torch.float32 else lowp(1e-2, dtype)
    for a, r in zip(got, ref):
        if a.dtype == torch.float32:
            assert err_rms(a, r) <= tol
        else:   # 16-bit: up to two roundings (a source's gradient: its read's share, then the scale's term added)
            assert within_ulps(a, r, k=2)


@pytest.mark.parametrize("d", [100, 8200])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode,glue", [("list", "1"), ("stack", "1"), ("scores", "1"), ("stack", "0"),
                                       ("scores", "0")])
def test_chain_any_width_matches_oracle(monkeypatch, d, dtype, mode, glue):
    from loopback_amd.chain import ChainConfig
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    t = 40 if d > 4096 else 96
    cfg = ChainConfig(f"any-d{d}", d, 2, 3, 1, t, dtype, True, q_std=0.5)
    print(f"case any-width chain d{d} {dtype} {mode} glue={glue}", flush=True)
    h, g = hip_chain(cfg, mode)
    check_chain(h, g, cfg)


@pytest.mark.parametrize("mode,glue", [("scores", "1"), ("stack", "0"), ("list", "1")])
def test_chain_of_70_steps(monkeypatch, mode, glue):
    """K = 2, R = 35: the last reads take 70 sources; with stored scores the stack keeps none (69 queries), the reads
    form them. fp32 against the exact chain, final state and every gradient: max-abs / RMS <= 1e-5, or where the
    chain's depth puts the reference read itself in fp32 above that (the updates' gradients, up to 2.5e-5 x RMS from
    the exact chain here), no more than twice the fp32 reference read's own error. The no-grad pass is bitwise the
    training forward."""
    from loopback_amd.chain import ChainConfig
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = ChainConfig("any-70", 64, 2, 35, 1, 24, torch.float32, True, q_std=0.5)
    print(f"case 70-step chain {mode} glue={glue}", flush=True)
    h, g = hip_chain(cfg, mode)
    hr, gr = ref_chain(cfg, torch.float64)
    h32, g32 = ref_chain(cfg, None)
    e = [err_rms(h, hr)] + [err_rms(a, b) for a, b in zip(grad_list(g), grad_list(gr))]
    er = [err_rms(h32, hr)] + [err_rms(a, b) for a, b in zip(grad_list(g32), grad_list(gr))]
    assert all(x <= max(1e-5, 2 * y) for x, y in zip(e, er)), (e, er)
    h_eval, _ = hip_chain(cfg, mode, grad=False)
    assert torch.equal(h_eval, h)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("boundary", [False, True])
def test_zero_query_identity_any_width(dtype, boundary):
    """Zero query and cbar == c0: out == base and tc == c0 bitwise at a width only the any-shape kernels take."""
    from loopback_amd.cell import LoopDeltaAttnRes
    b, t, d, n = 2, 11, 36, 5
    deltas, proposal, h0, _, prior, _, _, _ = make(b, t, d, n, dtype, seed=n, zero_query=True)
    nb = n if boundary else n + 1
    cell = LoopDeltaAttnRes(d, num_loops=2, num_blocks=nb, beta=0.75, eps=1e-6).to(DEV)
    coeffs = prior.view(1, 1, -1).expand(b, t, -1).contiguous().to(DEV)
    print(f"case any zero query {dtype} boundary={boundary}", flush=True)
    with torch.no_grad():
        out, tc, nxt = cell.combine(proposal.to(DEV), h0.to(DEV), [x.to(DEV) for x in deltas], coeffs,
                                    prior.to(DEV), 0, n - 1)
        p, h = proposal.to(DEV), h0.to(DEV)
        base = p + 0.75 * (h - p) if boundary else p
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    assert torch.equal(tc, nxt.view(1, 1, -1).expand(b, t, -1))


def _u64(lib, vals):
    return lib.u64_array(list(vals))


def _dev(vals):
    return torch.tensor(list(vals), dtype=torch.int64, device=DEV)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_entry_points_agree_with_row_layout(dtype):
    """At d = 256, n = 6 (both families take it): ldr_dv_assemble_any (rounding once and per read) and
    ldr_blend_sum_any give the row-layout kernels' bits; ldr_read_fwd_any (stored and online scores) and ldr_read_bwd1_any agree with ldr_read_fwd /
    ldr_read_fwd_online / ldr_read_bwd1 within fp32 round-off (max-abs <= 1e-5 x RMS; 16-bit outputs within one unit
    in the last place: one rounding each), their scalars too, and the blend gradients bitwise."""
    from loopback_amd import _lib as L
    from loopback_amd import fused_dattn as FD
    lib = L.LIB
    T, d, n = 300, 256, 6
    dt = lib_dtype(dtype)
    g_ = torch.Generator().manual_seed(12)
    V = [(torch.randn(T, d, generator=g_) * (0.5 + 0.2 * i)).to(dtype).to(DEV) for i in range(n)]
    R = [FD.rstd(v, 1e-6).reshape(T) for v in V]
    q = (torch.randn(d, generator=g_) * 0.4).to(DEV)
    base = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    h0 = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    cbar = (torch.rand(T, n, generator=g_) + 0.2).to(DEV)
    c0 = (torch.rand(n, generator=g_) + 0.2).to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    inv = 1.0 / d ** 0.5
    print(f"case any entry points {dtype}", flush=True)

    def check(code):
        assert code == 0, lib.ldr_strerror(code)

    vh, rh = _u64(L, (v.data_ptr() for v in V)), _u64(L, (r.data_ptr() for r in R))
    vd, rd = _dev(v.data_ptr() for v in V), _dev(r.data_ptr() for r in R)
    outs = {}
    for name in ("fast_online", "any_online", "fast_stored", "any_stored"):
        out = torch.empty_like(base)
        tc = torch.empty(T, n, device=DEV)
        p = torch.empty(T, n, device=DEV)
        nxt = torch.empty(n, device=DEV)
        dots = torch.empty(n, T, device=DEV) if "online" in name else outs["fast_online"][4]
        tail = (base.data_ptr(), h0.data_ptr(), 0.75, cbar.data_ptr(), n, c0.data_ptr(), n, 1.0, inv, out.data_ptr(),
                tc.data_ptr(), p.data_ptr(), nxt.data_ptr(), T, d, dt, st)
        if name == "fast_online":
            check(lib.ldr_read_fwd_online(vh, rh, n, q.data_ptr(), dots.data_ptr(), T, *tail))
        elif name == "any_online":
            check(lib.ldr_read_fwd_any(vd.data_ptr(), rd.data_ptr(), n, q.data_ptr(), dots.data_ptr(), T, *tail))
        elif name == "fast_stored":
            check(lib.ldr_read_fwd(vh, rh, n, dots.data_ptr(), T, *tail))
        else:
            check(lib.ldr_read_fwd_any(vd.data_ptr(), rd.data_ptr(), n, None, dots.data_ptr(), T, *tail))
        torch.cuda.synchronize()
        outs[name] = (out, tc, p, nxt, dots)
    ref = outs["fast_stored"]
    for name in ("fast_online", "any_online", "any_stored"):
        for a, b in zip(outs[name], ref):   # 16-bit outputs: one rounding of fp32 sums that differ in their last bits
            assert err_rms(a, b) <= 1e-5 if a.dtype == torch.float32 else within_ulps(a, b), name
    assert torch.equal(outs["any_stored"][3], ref[3])

    # backward pass 1 on the stored read's outputs
    _, tc, p, _, dots = ref
    g = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    gt = torch.randn(T, n, generator=g_).to(DEV)
    res = {}
    for name in ("fast", "any"):
        dcbar = torch.empty(T, n, device=DEV)
        dr = torch.zeros(n, T, device=DEV)
        wz = torch.empty(n, T, 2, device=DEV)
        parts = max(1, L.bwd1_parts(T, d))
        dq_part = torch.empty(parts, d, device=DEV)
        gp, gh = torch.empty_like(g), torch.empty_like(g)
        head = (n, g.data_ptr(), gt.data_ptr(), p.data_ptr(), dots.data_ptr(), T, tc.data_ptr(), cbar.data_ptr(), n,
                c0.data_ptr(), n, 1.0, inv, dcbar.data_ptr(), n)
        if name == "fast":
            check(lib.ldr_read_bwd1(vh, rh, *head, _u64(L, (dr[i].data_ptr() for i in range(n))), 0, wz.data_ptr(),
                                    T, dq_part.data_ptr(), d, gp.data_ptr(), gh.data_ptr(), 0.75, T, d, dt, st))
        else:
            drd = _dev(dr[i].data_ptr() for i in range(n))
            check(lib.ldr_read_bwd1_any(vd.data_ptr(), rd.data_ptr(), *head, drd.data_ptr(), 0, wz.data_ptr(), T,
                                        dq_part.data_ptr(), parts, d, gp.data_ptr(), gh.data_ptr(), 0.75, T, d, dt,
                                        st))
        dq = torch.empty(d, device=DEV)
        check(lib.ldr_reduce_rows(dq_part.data_ptr(), parts, d, dq.data_ptr(), st))
        torch.cuda.synchronize()
        res[name] = (dcbar, dr, wz, dq, gp, gh)
    for a, b in zip(res["any"], res["fast"]):
        assert err_rms(a, b) <= 1e-5
    assert torch.equal(res["any"][4], res["fast"][4]) and torch.equal(res["any"][5], res["fast"][5])

    # the update gradient over m = 3 reads (the added gradient the last read's own) and the blend sum: bitwise
    wz = res["fast"][2]
    gs = [torch.randn(T, d, generator=g_).to(dtype).to(DEV) for _ in range(3)]
    qs = [(torch.randn(d, generator=g_) * 0.3).to(DEV) for _ in range(3)]
    wzp = [wz[i].data_ptr() for i in range(3)]
    gr = torch.randn(T, generator=g_).to(DEV)
    for (add, beta), per_read in itertools.product(((None, 0.0), (gs[2], 0.0), (gs[2], 0.75), (gs[0], 0.0)), (0, 1)):
        dvs = {}
        for name in ("fast", "any"):
            dv, dvn = torch.empty_like(V[0]), torch.empty_like(V[0])
            tail = (3, V[1].data_ptr(), R[1].data_ptr(), gr.data_ptr(), None if add is None else add.data_ptr(), beta,
                    per_read, dv.data_ptr(), dvn.data_ptr(), T, d, dt, st)
            if name == "fast":
                check(lib.ldr_dv_assemble(_u64(L, (x.data_ptr() for x in gs)), _u64(L, wzp),
                                          _u64(L, (x.data_ptr() for x in qs)), *tail))
            else:
                tabs = (_dev(x.data_ptr() for x in gs), _dev(wzp), _dev(x.data_ptr() for x in qs))
                check(lib.ldr_dv_assemble_any(*(x.data_ptr() for x in tabs), *tail))
            torch.cuda.synchronize()
            dvs[name] = (dv, dvn)
        assert torch.equal(dvs["any"][0], dvs["fast"][0]) and torch.equal(dvs["any"][1], dvs["fast"][1])
    for pr in (0, 1):
        sums = []
        for name in ("fast", "any"):
            out = torch.empty_like(V[0])
            if name == "fast":
                check(lib.ldr_blend_sum(_u64(L, (x.data_ptr() for x in gs)), 3, 0.75, pr, out.data_ptr(), T, d, dt,
                                        st))
            else:
                tab = _dev(x.data_ptr() for x in gs)
                check(lib.ldr_blend_sum_any(tab.data_ptr(), 3, 0.75, pr, out.data_ptr(), T, d, dt, st))
            torch.cuda.synchronize()
            sums.append(out)
        assert torch.equal(sums[0], sums[1])
        if pr:   # rounded after every addition, in table order, as torch adds the rounded shares
            ref = (gs[0] * 0.75).to(gs[0].dtype)
            for x in gs[1:]:
                ref = ref + (x * 0.75).to(x.dtype)
            assert torch.equal(sums[0], ref)


def test_any_shape_refuses_graph_capture():
    """The any-shape path copies its address tables from host memory on the launch stream; under HIP graph capture
    it raises instead (a replay would read a host buffer torch may have reused), and nothing is launched."""
    from loopback_amd.cell import LoopDeltaAttnRes
    d, n = 36, 3
    cell = LoopDeltaAttnRes(d, num_loops=2, num_blocks=n + 1, beta=0.75, eps=1e-6).to(DEV)
    xs = [torch.randn(1, 8, d, device=DEV) for _ in range(n)]
    prop, h0 = torch.randn(1, 8, d, device=DEV), torch.randn(1, 8, d, device=DEV)
    coeffs, prior = torch.ones(1, 8, n - 1, device=DEV), torch.ones(n - 1, device=DEV)
    print("case any-shape under capture", flush=True)
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="HIP graph"):
            with torch.cuda.graph(graph, stream=side):
                cell.combine(prop, h0, xs, coeffs, prior, 0, n - 1)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [256, 8192])
def test_one_source_without_coefficient_columns(dtype, d):
    """A read of one source with no stored cbar or prior column (cbar_cols = c0_cols = 0: the newest column implied,
    lam) against the same read given those columns explicitly as ones (lam x 1 = lam), through the C ABI: the read
    forward (both scores paths; d = 8192 takes the 512-lane launch), backward pass 1 and every scalar bitwise equal.
    The kernels load cbar at a clamped address before its column is tested; with no column they load another
    operand's first element instead and use lam."""
    from loopback_amd import _lib as L
    from loopback_amd import fused_dattn as FD
    lib = L.LIB
    T, n = 300, 1
    dt = lib_dtype(dtype)
    g_ = torch.Generator().manual_seed(d + 5)
    V = [torch.randn(T, d, generator=g_).to(dtype).to(DEV)]
    R = [FD.rstd(V[0], 1e-6).reshape(T)]
    q = (torch.randn(d, generator=g_) * 0.4).to(DEV)
    base = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    h0 = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    g = torch.randn(T, d, generator=g_).to(dtype).to(DEV)
    gt = torch.randn(T, n, generator=g_).to(DEV)
    ones_t, ones_1 = torch.ones(T, 1, device=DEV), torch.ones(1, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    inv, lam = 1.0 / d ** 0.5, 0.75
    vh, rh = _u64(L, (v.data_ptr() for v in V)), _u64(L, (r.data_ptr() for r in R))
    print(f"case one source, no coefficient columns {dtype} d{d}", flush=True)

    def check(code):
        assert code == 0, lib.ldr_strerror(code)

    res = {}
    for cols in (0, 1):
        # with no column the pointers are another tensor's (any readable address): nothing may be read from them
        cbar = ones_t if cols else gt
        c0 = ones_1 if cols else gt
        outs = []
        dots = torch.empty(n, T, device=DEV)
        for online in (True, False):
            out, tc, p, nxt = (torch.empty_like(base), torch.empty(T, n, device=DEV), torch.empty(T, n, device=DEV),
                               torch.empty(n, device=DEV))
            tail = (base.data_ptr(), h0.data_ptr(), 0.75, cbar.data_ptr(), cols, c0.data_ptr(), cols, lam, inv,
                    out.data_ptr(), tc.data_ptr(), p.data_ptr(), nxt.data_ptr(), T, d, dt, st)
            if online:
                check(lib.ldr_read_fwd_online(vh, rh, n, q.data_ptr(), dots.data_ptr(), T, *tail))
            else:
                check(lib.ldr_read_fwd(vh, rh, n, dots.data_ptr(), T, *tail))
            outs += [out, tc, p, nxt]
        _, tc, p, _ = outs[4:]
        dcbar = torch.empty(T, n, device=DEV)
        dr = torch.zeros(n, T, device=DEV)
        wz = torch.empty(n, T, 2, device=DEV)
        parts = max(1, L.bwd1_parts(T, d))
        dq_part = torch.empty(parts, d, device=DEV)
        gp, gh = torch.empty_like(g), torch.empty_like(g)
        check(lib.ldr_read_bwd1(vh, rh, n, g.data_ptr(), gt.data_ptr(), p.data_ptr(), dots.data_ptr(), T,
                                tc.data_ptr(), cbar.data_ptr(), cols, c0.data_ptr(), cols, lam, inv, dcbar.data_ptr(),
                                0, _u64(L, (dr[i].data_ptr() for i in range(n))), 0, wz.data_ptr(), T,
                                dq_part.data_ptr(), d, gp.data_ptr(), gh.data_ptr(), 0.75, T, d, dt, st))
        dq = torch.empty(d, device=DEV)
        check(lib.ldr_reduce_rows(dq_part.data_ptr(), parts, d, dq.data_ptr(), st))
        torch.cuda.synchronize()
        res[cols] = outs + [dots, dr, wz, dq, gp, gh]
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)
    assert torch.isfinite(res[0][0].float()).all() and res[0][2].eq(1.0).all() and res[0][6].eq(1.0).all()   # p = 1
