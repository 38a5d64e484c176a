"""The stacked write (DattnStack.write, fused_dattn.py:679-695): V[s] = h - x rounded to the stack dtype (bitwise
what torch's subtraction gives), R[s] the RMS scale of the rounded update, and the scores of the update against
the queries of the reads still to come, DOTS[j, s, tok] = q_j . V[s, tok] for j >= s - 1 -- against an fp64 matmul
of the rounded update (matrix cores from the queries' three bf16 parts; an fp16 update as the exact sum of two bf16
values, an fp32 one as the sum of three -- for 16-bit updates k_write_rows at widths that are multiples of 256, here
768 and 2048, k_write_mfma for the others; k_write_mfma32 for fp32). Ragged token
counts, widths below one 64-column chunk and a width with a partial chunk included; every slice is checked
again after the last write."""
import pytest
import torch

from gpu_helpers import DEV, err_rms, lib_dtype

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("T,d", [(37, 64), (100, 768), (257, 1096), (64, 2048), (19, 40), (5, 8)])
@pytest.mark.parametrize("N", [2, 9, 33, 64])   # 64: up to 63 queries, the 4-block score kernels
def test_write_scores(dtype, T, d, N):
    from loopback_amd import fused_dattn as FD
    from oracle.reference_read import rstd_ref
    gen = torch.Generator().manual_seed(T + d + N)
    Q = (torch.randn(N - 1, d, generator=gen) * 0.3).to(DEV)
    stack = FD.DattnStack(N, (1, T, d), dtype, DEV, query=Q, eps=1e-6)
    hs = [torch.randn(1, T, d, generator=gen).to(dtype).to(DEV) for _ in range(N)]
    xs = [torch.randn(1, T, d, generator=gen).to(dtype).to(DEV) for _ in range(N)]
    with torch.no_grad():
        for s in range(N):
            v = stack.write(s, hs[s], xs[s])
            assert torch.equal(v, hs[s] - xs[s]), s
            assert stack.r_done[s]
    torch.cuda.synchronize()
    for s in range(N):   # no later write touched an earlier slice
        assert torch.equal(stack.V[s].reshape(1, T, d), hs[s] - xs[s]), s
    V = stack.V.double().cpu().reshape(N, T, d)
    rr = rstd_ref(V, 1e-6).squeeze(-1)
    assert err_rms(stack.R.reshape(N, T).cpu(), rr) <= 2e-6
    ref = torch.einsum("jd,std->jst", Q.double().cpu(), V)           # [query, source, token]
    got = stack.DOTS.cpu()
    for s in range(N):
        j_lo = max(0, s - 1)
        if j_lo < N - 1:
            assert err_rms(got[j_lo:, s], ref[j_lo:, s]) <= 1e-5, s


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("m,T,d", [(1, 5, 64), (8, 77, 768), (3, 16, 8192)])
@pytest.mark.parametrize("per_read", [0, 1])
def test_blend_sum_bitwise(dtype, m, T, d, per_read):
    """ldr_blend_sum: round(sum_j round(beta g_j)) in fp32, j in order -- or with per_read each addition in the
    update dtype, as torch adds the rounded shares -- bitwise the same sequence in torch."""
    from loopback_amd import _lib as L
    gen = torch.Generator().manual_seed(m * 1000 + d)
    gs = [torch.randn(T, d, generator=gen).to(dtype).to(DEV) for _ in range(m)]
    out = torch.empty(T, d, dtype=dtype, device=DEV)
    code = L.LIB.ldr_blend_sum(L.u64_array(g.data_ptr() for g in gs), m, 0.75, per_read, out.data_ptr(), T, d,
                               lib_dtype(dtype), torch.cuda.current_stream().cuda_stream)
    L.check(code, "blend_sum")
    torch.cuda.synchronize()
    if per_read:
        ref = (gs[0] * 0.75).to(dtype)
        for g in gs[1:]:
            ref = ref + (g * 0.75).to(dtype)
        assert torch.equal(out, ref)
        return
    acc = torch.zeros(T, d, dtype=torch.float32, device=DEV)
    for g in gs:
        acc = acc + (g * 0.75).to(dtype).float()
    assert torch.equal(out, acc.to(dtype))


@pytest.mark.parametrize("d", [256, 2048, 8192])
@pytest.mark.parametrize("nq", [0, 1, 16, 17, 32, 40, 63])
@pytest.mark.parametrize("T", [1, 77, 333])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_whole_row_write_is_the_matrix_core_write_bitwise(d, nq, T, dtype):
    """k_write_rows (rows streamed whole, the write for widths that are multiples of 256) against k_write_mfma (the
    matrix cores' layout), bf16 and fp16 updates, and k_write_rows32 against k_write_mfma32 for fp32 updates
    (three bf16 parts per value), on the same inputs through the C ABI, scoring the last nq of 64
    queries (so the first 16-query block scored starts inside the table at every nq not a multiple of 16): V, R and
    the scores bitwise
    equal (the same chunks per wave, operands and order of every sum), the scores within 1e-5 x RMS of an fp64
    product. k_write_mfma and k_write_mfma32 come from the test fixture library built with the alternative kernel
    shapes (LDR_WM_ROWS=0, LDR_W32_ROWS=0; loopback_amd.build builds it beside the product library)."""
    import ctypes
    from loopback_amd import _lib as L
    from loopback_amd import build as B
    other = ctypes.CDLL(B.TEST_LIB_ALT)
    res, args = L.SIGNATURES["ldr_write_dots"]
    fns = [L.LIB.ldr_write_dots, other.ldr_write_dots]
    fns[1].restype, fns[1].argtypes = res, args
    gen = torch.Generator().manual_seed(d + 7 * nq + T)
    h = torch.randn(T, d, generator=gen).to(dtype).to(DEV)
    x = torch.randn(T, d, generator=gen).to(dtype).to(DEV)
    NQ = 64                                       # the pass's queries; this write scores the last nq of them
    q = (torch.randn(NQ, d, generator=gen) * 0.3).to(DEV)
    qb = torch.empty(int(L.LIB.ldr_query_parts_elems(NQ, d)), dtype=torch.bfloat16, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    L.check(L.LIB.ldr_split_queries(q.data_ptr(), NQ, d, qb.data_ptr(), st), "split_queries")
    outs = []
    print(f"case write layouts d{d} nq{nq} T{T} {dtype}", flush=True)
    for fn in fns:
        v = torch.empty(T, d, dtype=dtype, device=DEV)
        r = torch.empty(T, device=DEV)
        dots = torch.full((max(nq, 1), T), float("nan"), device=DEV)
        L.check(fn(h.data_ptr(), x.data_ptr(), v.data_ptr(), r.data_ptr(), q.data_ptr(), qb.data_ptr(), NQ,
                   NQ - nq, dots.data_ptr(), T, d, T, 1e-6, lib_dtype(dtype), st), "write_dots")
        torch.cuda.synchronize()
        outs.append((v.cpu(), r.cpu(), dots.cpu()))
    (v1, r1, s1), (v2, r2, s2) = outs
    assert torch.equal(v1, v2) and torch.equal(r1, r2)
    assert torch.equal(v1, h.cpu() - x.cpu())
    if nq > 0:
        assert torch.equal(s1[:nq], s2[:nq])
        ref = q[NQ - nq:].double().cpu() @ v1.double().T              # the scores against an fp64 product
        assert ((s1[:nq].double() - ref).abs().max() / ref.pow(2).mean().sqrt()).item() <= 1e-5


@pytest.mark.parametrize("dtype,d,n", [("bf16", 2048, 5), ("bf16", 2048, 32), ("bf16", 1024, 12), ("bf16", 1024, 20),
                                       ("bf16", 768, 17), ("bf16", 768, 40), ("bf16", 1536, 8), ("fp32", 2048, 5),
                                       ("fp32", 2048, 31), ("bf16", 3072, 9)])
@pytest.mark.parametrize("T", [1, 77, 1000, 4099])
@pytest.mark.parametrize("blend", [False, True])
def test_read_forward_launch_shapes_agree_bitwise(dtype, d, n, T, blend):
    """ldr_read_fwd in its two launch shapes -- 512-lane workgroups (the product library, for reads of at least
    28 KiB of rows per token) with 32-token tiles, or 16-token tiles for rows of 4-8 KiB (fp32 rows of 2048, bf16 rows
    of 3072), and 256-lane workgroups with 16-token tiles, 8-token ones for rows of 4-8 KiB (the fixture library built
    with the alternative kernel shapes) -- on the same inputs: out, tc, p and next_prior bitwise equal (each row sums
    its sources in the same order, and the softmax spreads a token over the same lanes in both: 16, or 32 for rows of
    4-8 KiB), with and without the iteration-end blend, over ragged token counts."""
    import ctypes
    from loopback_amd import _lib as L
    from loopback_amd import build as B
    other = ctypes.CDLL(B.TEST_LIB_ALT)
    res, args = L.SIGNATURES["ldr_read_fwd"]
    fns = [L.LIB.ldr_read_fwd, other.ldr_read_fwd]
    fns[1].restype, fns[1].argtypes = res, args
    dt, code = (torch.float32, L.F32) if dtype == "fp32" else (torch.bfloat16, L.BF16)
    gen = torch.Generator().manual_seed(d + 13 * n + T + int(blend))
    V = [(torch.randn(T, d, generator=gen) * (0.5 + 0.05 * i)).to(dt).to(DEV) for i in range(n)]
    R = [(torch.rand(T, generator=gen) + 0.5).to(DEV) for _ in range(n)]
    dots = (torch.randn(n, T, generator=gen) * 3.0).to(DEV)
    base = torch.randn(T, d, generator=gen).to(dt).to(DEV)
    h0 = torch.randn(T, d, generator=gen).to(dt).to(DEV)
    cbar = (torch.rand(T, n, generator=gen) + 0.1).to(DEV)
    c0 = (torch.rand(n, generator=gen) + 0.1).to(DEV)
    vp = L.u64_array([v.data_ptr() for v in V])
    rp = L.u64_array([r.data_ptr() for r in R])
    st = torch.cuda.current_stream().cuda_stream
    print(f"case read shapes {dtype} d{d} n{n} T{T} blend={blend}", flush=True)
    outs = []
    for fn in fns:
        out = torch.empty(T, d, dtype=dt, device=DEV)
        tc, p = torch.empty(T, n, device=DEV), torch.empty(T, n, device=DEV)
        nxt = torch.empty(n, device=DEV)
        L.check(fn(vp, rp, n, dots.data_ptr(), T, base.data_ptr(), h0.data_ptr() if blend else None, 0.75,
                   cbar.data_ptr(), n, c0.data_ptr(), n, 0.25 if blend else 1.0, d ** -0.5, out.data_ptr(),
                   tc.data_ptr(), p.data_ptr(), nxt.data_ptr(), T, d, code, st), "read_fwd")
        torch.cuda.synchronize()
        outs.append((out.cpu(), tc.cpu(), p.cpu(), nxt.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
