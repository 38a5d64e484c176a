"""ldr_read_bwd1_noalloc -- backward pass 1 and its query gradient with no workspace argument and no allocation --
against the entry points it varies (ldr_read_bwd1 with a caller workspace, then ldr_reduce_rows over the partials),
through the C ABI on the same inputs: every output bitwise equal (dq, dcbar, the accumulated dr, the wz pairs, the
blend gradients), on two calls in a row, the second with fewer tokens and a narrower row (the library's array then
still holds the first call's partials), bf16, fp16 and fp32; an empty batch gives a zero query gradient; a repeated call
leaves the device's free memory unchanged (torch.cuda.mem_get_info: device-wide, so it also sees an allocation the
library would make outside torch's allocator; another process on the same GPU could move it, none runs beside these
tests); captured in a HIP graph after a warm-up call outside capture (which looks the array's address up), every
replay -- with eager calls and synchronizations between them -- is bitwise the workspace path."""
import pytest
import torch

from gpu_helpers import DEV, lib_dtype

pytestmark = pytest.mark.gpu


def _inputs(n, T, d, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    vals = [torch.randn(T, d, generator=gen).to(dtype).to(DEV) for _ in range(n)]
    rs = [(torch.rand(T, generator=gen) + 0.5).to(DEV) for _ in range(n)]
    g = torch.randn(T, d, generator=gen).to(dtype).to(DEV)
    gt = torch.randn(T, n, generator=gen).to(DEV)
    p = torch.softmax(torch.randn(T, n, generator=gen), -1).to(DEV)
    dots = torch.randn(n, T, generator=gen).to(DEV)
    tc = torch.randn(T, n, generator=gen).to(DEV)
    cbar = torch.randn(T, n, generator=gen).to(DEV)
    c0 = (torch.rand(n, generator=gen) + 0.1).to(DEV)
    dr0 = torch.randn(n, T, generator=gen).to(DEV)
    return vals, rs, g, gt, p, dots, tc, cbar, c0, dr0


def _run(noalloc, n, T, d, dtype, args):
    """One call of either path on fresh output buffers; returns the outputs (on the CPU)."""
    from loopback_amd import _lib as L
    vals, rs, g, gt, p, dots, tc, cbar, c0, dr0 = args
    dt = lib_dtype(dtype)
    st = torch.cuda.current_stream().cuda_stream
    vp = L.u64_array([v.data_ptr() for v in vals])
    rp = L.u64_array([r.data_ptr() for r in rs])
    dr = dr0.clone()
    drp = L.u64_array([dr[i].data_ptr() for i in range(n)])
    dcbar = torch.full((T, n), float("nan"), device=DEV)
    wz = torch.full((n, T, 2), float("nan"), device=DEV)
    g_prop = torch.empty_like(g)
    g_h0 = torch.empty_like(g)
    dq = torch.full((d,), float("nan"), device=DEV)
    common = (vp, rp, n, g.data_ptr(), gt.data_ptr(), p.data_ptr(), dots.data_ptr(), T, tc.data_ptr(),
              cbar.data_ptr(), n, c0.data_ptr(), n, 1.0, 1.0 / d ** 0.5, dcbar.data_ptr(), n, drp, 1, wz.data_ptr(), T)
    tail = (g_prop.data_ptr(), g_h0.data_ptr(), 0.75, T, d, dt, st)
    if noalloc:
        free0 = torch.cuda.mem_get_info()[0]
        L.check(L.LIB.ldr_read_bwd1_noalloc(*common, dq.data_ptr(), *tail), "read_bwd1_noalloc")
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0 or free0 is None
    else:
        parts = L.bwd1_parts(T, d)
        ws = torch.empty((max(1, parts), d), device=DEV)
        L.check(L.LIB.ldr_read_bwd1(*common, ws.data_ptr(), d, *tail), "read_bwd1")
        L.check(L.LIB.ldr_reduce_rows(ws.data_ptr(), parts, d, dq.data_ptr(), st), "reduce_rows")
        torch.cuda.synchronize()
    return [x.cpu() for x in (dq, dcbar, dr, wz, g_prop, g_h0)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_noalloc_backward_pass1_is_the_workspace_one(dtype):
    for call, (n, T, d) in enumerate([(9, 3000, 2048), (5, 333, 1024)]):
        print(f"case noalloc {dtype} call {call}: n{n} T{T} d{d}", flush=True)
        args = _inputs(n, T, d, dtype, seed=100 * call + (dtype == torch.float32))
        want = _run(False, n, T, d, dtype, args)
        got = _run(True, n, T, d, dtype, args)
        for name, a, b in zip(("dq", "dcbar", "dr", "wz", "g_prop", "g_h0"), got, want):
            assert torch.equal(a, b), (call, name)
        assert torch.isfinite(got[0]).all()


def test_noalloc_empty_batch_gives_zero_query_gradient():
    from loopback_amd import _lib as L
    n, d = 3, 768
    dq = torch.full((d,), float("nan"), device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    null = L.u64_array([0] * n)
    c0 = torch.ones(n, device=DEV)
    print("case noalloc empty batch", flush=True)
    L.check(L.LIB.ldr_read_bwd1_noalloc(null, null, n, None, None, None, None, 0, None, None, n, c0.data_ptr(), n,
                                        1.0, 1.0 / d ** 0.5, None, n, null, 1, None, 0, dq.data_ptr(), None, None,
                                        0.0, 0, d, L.BF16, st), "read_bwd1_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(dq.cpu(), torch.zeros(d))


def test_noalloc_rejects_bad_arguments_before_any_launch():
    from loopback_amd import _lib as L
    st = torch.cuda.current_stream().cuda_stream
    null = L.u64_array([0])
    c0 = torch.ones(1, device=DEV)
    # no dq; then a width the kernels do not take
    assert L.LIB.ldr_read_bwd1_noalloc(null, null, 1, None, None, None, None, 0, None, None, 1, c0.data_ptr(), 1, 1.0,
                                       1.0, None, 1, null, 0, None, 0, None, None, None, 0.0, 0, 64, L.BF16, st) == -1
    dq = torch.empty(8200, device=DEV)
    assert L.LIB.ldr_read_bwd1_noalloc(null, null, 1, None, None, None, None, 0, None, None, 1, c0.data_ptr(), 1, 1.0,
                                       1.0, None, 1, null, 0, None, 0, dq.data_ptr(), None, None, 0.0, 0, 8200,
                                       L.BF16, st) == -2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_replays_in_a_graph(dtype):
    """The entry point's callers include code under HIP graph capture. After one call outside capture on this device
    (it looks the array's address up; an empty batch suffices), a capture of the call on torch's capture stream
    replays, three times with eager work between, to the workspace path's outputs bitwise. dr_accum = 0 so a replay
    does not add to the previous replay's scale gradients."""
    from loopback_amd import _lib as L
    n, T, d = 7, 1500, 2048
    print(f"case noalloc graph {dtype}", flush=True)
    vals, rs, g, gt, p, dots, tc, cbar, c0, dr0 = _inputs(n, T, d, dtype, seed=7)
    dt = lib_dtype(dtype)
    vp = L.u64_array([v.data_ptr() for v in vals])
    rp = L.u64_array([r.data_ptr() for r in rs])

    def outputs():
        dr = torch.full((n, T), float("nan"), device=DEV)
        return dict(dr=dr, drp=L.u64_array([dr[i].data_ptr() for i in range(n)]),
                    dcbar=torch.full((T, n), float("nan"), device=DEV),
                    wz=torch.full((n, T, 2), float("nan"), device=DEV), g_prop=torch.empty_like(g),
                    g_h0=torch.empty_like(g), dq=torch.full((d,), float("nan"), device=DEV))

    def call(o, noalloc, st):
        common = (vp, rp, n, g.data_ptr(), gt.data_ptr(), p.data_ptr(), dots.data_ptr(), T, tc.data_ptr(),
                  cbar.data_ptr(), n, c0.data_ptr(), n, 1.0, 1.0 / d ** 0.5, o["dcbar"].data_ptr(), n, o["drp"], 0,
                  o["wz"].data_ptr(), T)
        tail = (o["g_prop"].data_ptr(), o["g_h0"].data_ptr(), 0.75, T, d, dt, st)
        if noalloc:
            L.check(L.LIB.ldr_read_bwd1_noalloc(*common, o["dq"].data_ptr(), *tail), "read_bwd1_noalloc")
        else:
            parts = L.bwd1_parts(T, d)
            ws = torch.empty((parts, d), device=DEV)
            L.check(L.LIB.ldr_read_bwd1(*common, ws.data_ptr(), d, *tail), "read_bwd1")
            L.check(L.LIB.ldr_reduce_rows(ws.data_ptr(), parts, d, o["dq"].data_ptr(), st), "reduce_rows")

    names = ("dq", "dcbar", "dr", "wz", "g_prop", "g_h0")
    ref = outputs()
    call(ref, False, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = [ref[k].clone() for k in names]
    # the warm-up outside capture: an empty batch (it launches only the zero fill of its own dq)
    dq0 = torch.empty(d, device=DEV)
    null = L.u64_array([0] * n)
    L.check(L.LIB.ldr_read_bwd1_noalloc(null, null, n, None, None, None, None, 0, None, None, n, c0.data_ptr(), n,
                                        1.0, 1.0 / d ** 0.5, None, n, null, 0, None, 0, dq0.data_ptr(), None, None,
                                        0.0, 0, d, dt, torch.cuda.current_stream().cuda_stream), "warm-up")
    torch.cuda.synchronize()
    o = outputs()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(o, True, torch.cuda.current_stream().cuda_stream)
    for k in range(3):
        for key in names:
            o[key].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for key, w in zip(names, want):
            assert torch.equal(o[key], w), (k, key)
        other = outputs()                          # eager work between replays: the workspace path again
        call(other, False, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(other["dq"], want[0])
