"""Shared helpers of the GPU parity tests: seeded inputs (generated on the CPU, copied to the GPU, so the oracle and
the HIP path see the same numbers) and the error measures the tolerances are stated in."""
import torch

DEV = torch.device("cuda", 0)


def make(b, t, d, n, dtype, seed, zero_query=False):
    """The reference test's inputs (tests/test_fused_dattn.py:35-45): deltas N(0,1)(0.5 + 0.1 i), proposal and h0
    N(0,1), q 0.3 N(0,1) (or 0), prior U(0.1, 1) of n - 1 entries, coeffs = prior + 0.2 N(0,1), upstream gradients
    N(0,1) on out and on tc. CPU tensors; `to_dev` moves them."""
    g = torch.Generator().manual_seed(seed)
    deltas = [(torch.randn(b, t, d, generator=g) * (0.5 + 0.1 * i)).to(dtype) for i in range(n)]
    proposal = torch.randn(b, t, d, generator=g).to(dtype)
    h0 = torch.randn(b, t, d, generator=g).to(dtype)
    q = torch.zeros(d) if zero_query else torch.randn(d, generator=g) * 0.3
    prior = torch.rand(n - 1, generator=g) * 0.9 + 0.1
    coeffs = prior.view(1, 1, -1) + 0.2 * torch.randn(b, t, n - 1, generator=g)
    up = torch.randn(b, t, d, generator=g)
    up2 = torch.randn(b, t, n, generator=g)
    return deltas, proposal, h0, q, prior, coeffs, up, up2


def rms(x):
    return x.double().pow(2).mean().sqrt().clamp_min(1e-30).item()


def err_rms(a, ref):
    """max |a - ref| / RMS(ref): the fp32 tolerance of the target (<= 1e-5)."""
    return ((a.double().cpu() - ref.double().cpu()).abs().max().item()) / rms(ref)


def err_max(a, ref):
    """max |a - ref| / max |ref|: the reference test's relative error (tests/test_fused_dattn.py:76-77)."""
    ref = ref.double().cpu()
    return ((a.double().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def err_norm(a, ref):
    """||a - ref|| / ||ref||: the stacked-layout test's relative error (tests/test_dattn_stack.py:64-65)."""
    ref = ref.double().cpu()
    return ((a.double().cpu() - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def lib_dtype(dtype):
    """The C ABI's code of an update dtype."""
    from loopback_amd import _lib as L
    return {torch.float32: L.F32, torch.bfloat16: L.BF16, torch.float16: L.F16}[dtype]


def lowp(bf16_bar, dtype):
    """A bar stated for bf16 carried to fp16: fp16 rounds to 2^-11 relative where bf16 rounds to 2^-8, so the bar
    is 8 times tighter."""
    return bf16_bar if dtype == torch.bfloat16 else bf16_bar / 8


def ulp_rel(dtype):
    """The spacing of the dtype's values in [1, 2), relative: 2^-7 (bf16), 2^-10 (fp16) -- one rounding of an exact
    value moves it by at most half of that."""
    return {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]


def within_ulps(a, ref, k=1, floor=2e-5):
    """Elementwise |a - ref| <= k units in the last place of their 16-bit dtype at max(|a|, |ref|), plus floor x
    RMS(ref): what k roundings of fp32 values that differ only in their last bits can leave between two results."""
    u = ulp_rel(ref.dtype)
    a, ref = a.double().cpu(), ref.double().cpu()
    bound = torch.maximum(a.abs(), ref.abs()) * (k * u) + floor * rms(ref)
    return bool(((a - ref).abs() <= bound).all())
