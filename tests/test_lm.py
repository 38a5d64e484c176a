"""The minimal Loopback LM (loopback_amd/lm.py) with the HIP read integrated (the benchmark's config 5 model).

CPU (no GPU): the model's wiring with the oracle read in fp64 -- topology and sharing, the Plain-Loop identity of
Loopback at beta = 0 with zero queries (the reference audit's C6: every coefficient is then 1, so the read is the
plain residual sum), and a loss near log(vocab) at init.
GPU: the model with the HIP read against the same weights on the CPU with the oracle read in fp64 -- loss and every
parameter gradient (fp32: norm-relative 1e-4; bf16: loss within 1e-2 relative) -- the model through every read
path (stored / online scores, list layout, torch glue) agreeing, the model at init bitwise the same with the
reference read run on the GPU, and a few training steps that lower the loss on a fixed batch; the reference's
whole-model layout test (stacked == list bit for bit with per-read rounding: loss, logits, every gradient) with a
deterministic attention. CPU also: the meta-device init path leaves the queries at zero.
"""
import copy
import math

import pytest
import torch
import torch.nn as nn

from loopback_amd.lm import LMConfig, LoopbackLM, make_optimizer, train_step
from oracle.reference_read import OracleCell

TINY = dict(hidden_size=64, num_heads=4, vocab_size=97, prelude=1, loop_blocks=2, loops=3, coda=1,
            hidden_ratio=4, rope_theta=1e4)


class OracleRead(nn.Module):
    """The reference read cell as the LM's read (list layout, any dtype, on its inputs' device)."""

    def __init__(self, read):
        super().__init__()
        self.query = read.query
        self.cfg = (read.dim, read.num_loops, read.num_blocks, read.beta, read.eps)

    def combine(self, proposal, h0, deltas, coeffs, prior, loop_idx, block_idx, keys=None):
        dim, loops, blocks, beta, eps = self.cfg
        cell = OracleCell(dim, loops, blocks, beta, eps, self.query)
        return cell.combine(proposal, h0, deltas, coeffs, prior, loop_idx, block_idx, keys=keys)


def oracle_model(model: LoopbackLM, dtype=torch.float64) -> LoopbackLM:
    """A CPU copy of `model` in `dtype` whose read is the oracle's."""
    ref = copy.deepcopy(model).to(device="cpu", dtype=dtype)
    if ref.read is not None:
        ref.read = OracleRead(ref.read)
    return ref


def ids_for(cfg, b=2, t=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.vocab_size, (b, t), generator=g)


def test_topology_and_sharing():
    cfg = LMConfig(**TINY)
    m = LoopbackLM(cfg)
    assert cfg.topology() == "[1->2x3->1]" and cfg.intermediate == 256
    assert len(m.middle) == 2 and m.read.query.shape == (2 * 3 - 1, 64) and not m.read.query.any()
    assert LMConfig().intermediate == 2048 and LMConfig().topology() == "[2->4x4->2]"
    with pytest.raises(ValueError):
        LMConfig(hidden_size=64, num_heads=5)


def test_loopback_at_beta0_zero_query_is_plain_loop():
    torch.manual_seed(0)
    cfg = LMConfig(**TINY, beta=0.0)
    lb = oracle_model(LoopbackLM(cfg))
    plain = LoopbackLM(LMConfig(**TINY, residual=None)).to(torch.float64)
    plain.load_state_dict({k: v for k, v in lb.state_dict().items() if not k.startswith("read.")})
    ids = ids_for(cfg)
    a, b = lb(ids), plain(ids)
    assert abs(a.item() - b.item()) < 1e-12
    assert abs(a.item() - math.log(cfg.vocab_size)) < 0.1      # near-uniform logits at init


def _grads(model):
    return {k: p.grad.detach().double().cpu() for k, p in model.named_parameters() if p.grad is not None}


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hip_lm_matches_oracle_lm(dtype):
    torch.manual_seed(1)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg)
    with torch.no_grad():
        model.read.query.normal_(0, 0.5)                      # a non-trivial read
    ref = oracle_model(model)
    gpu = copy.deepcopy(model).to(device="cuda", dtype=dtype)
    ids = ids_for(cfg, b=2, t=48)
    print(f"case lm {dtype}", flush=True)
    loss = gpu(ids.cuda())
    loss.backward()
    torch.cuda.synchronize()
    lref = ref(ids)
    lref.backward()
    rel = abs(loss.item() - lref.item()) / abs(lref.item())
    if dtype == torch.float32:
        assert rel < 1e-5, rel
        g, gr = _grads(gpu), _grads(ref)
        assert set(g) == set(gr)
        for k in gr:
            err = ((g[k] - gr[k]).norm() / gr[k].norm().clamp_min(1e-30)).item()
            assert err < 1e-4, (k, err)
    else:
        assert rel < 1e-2, rel
        g, gr = _grads(gpu), _grads(ref)
        assert set(g) == set(gr)
        for k in gr:
            assert torch.isfinite(g[k]).all(), k


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lm_at_init_is_the_reference_read_bitwise(dtype):
    """The reference's whole-model check (tests/test_fused_dattn.py:128-154, 210-215): at init (zero queries) the
    model with the HIP read and the same model with the reference read -- the oracle cell, on the same GPU, so every
    other op is the same kernel -- give the same loss bitwise: at zero query the read is exactly its base in both.
    The gradients (summed in other orders by the two backwards) agree to 1e-5 (fp32) / 1e-2 (bf16) norm-relative."""
    torch.manual_seed(4)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg)
    assert not model.read.query.any()                         # the reference's zero init
    hip = copy.deepcopy(model).to(device="cuda", dtype=dtype)
    ref = copy.deepcopy(model).to(device="cuda", dtype=dtype)
    ref.read = OracleRead(ref.read)
    ids = ids_for(cfg, b=2, t=40).cuda()
    print(f"case lm at init {dtype}", flush=True)
    la, lb = hip(ids), ref(ids)
    assert torch.equal(la, lb), (la.item(), lb.item())
    la.backward()
    lb.backward()
    torch.cuda.synchronize()
    ga, gb = _grads(hip), _grads(ref)
    assert set(ga) == set(gb)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    for k in gb:
        err = ((ga[k] - gb[k]).norm() / gb[k].norm().clamp_min(1e-30)).item()
        assert err <= tol, (k, err)


@pytest.mark.gpu
def test_lm_training_lowers_loss():
    torch.manual_seed(2)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg).to(device="cuda", dtype=torch.bfloat16)
    opt = make_optimizer(model)
    ids = ids_for(cfg, b=4, t=64).cuda()
    first = train_step(model, opt, ids).item()
    for _ in range(20):
        last = train_step(model, opt, ids).item()
    torch.cuda.synchronize()
    assert last < first - 0.5, (first, last)
    assert model.read.query.abs().sum().item() > 0            # the read's query is trained


def test_meta_device_init_gives_zero_queries():
    """The reference's init guard (check_equivalence_init.py:109-156): a model built on the meta device and
    materialized with reset_parameters has the read's query (K R - 1, d) at zero and the decay-only read."""
    cfg = LMConfig(**TINY)
    with torch.device("meta"):
        m = LoopbackLM(cfg)
    assert m.read.query.is_meta
    m = m.to_empty(device="cpu")
    m.reset_parameters()
    assert m.read.query.shape == (cfg.loop_blocks * cfg.loops - 1, cfg.hidden_size)
    assert not m.read.query.any()
    assert all(torch.isfinite(p).all() for p in m.parameters())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lm_read_modes_agree(monkeypatch, dtype):
    """The whole model through every path of the read (tests/test_dattn_stack.py:120-159): stacked with stored
    scores, stacked with online scores, the list layout, and the stacked layout with the caller's glue as torch ops.
    Loss and every parameter gradient agree (fp32: norm-relative 1e-6; bf16: 1e-2)."""
    torch.manual_seed(3)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg)
    with torch.no_grad():
        model.read.query.normal_(0, 0.5)
    ids = ids_for(cfg, b=2, t=40).cuda()
    runs = {}
    for name, env in {"scores": ("1", "1", "1"), "stack": ("1", "0", "1"), "list": ("0", "1", "1"),
                      "torch-glue": ("1", "1", "0")}.items():
        monkeypatch.setenv("LOOP_DATTN_STACK", env[0])
        monkeypatch.setenv("LOOP_DATTN_DOTS", env[1])
        monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", env[2])
        m = copy.deepcopy(model).to(device="cuda", dtype=dtype)
        loss = m(ids)
        loss.backward()
        torch.cuda.synchronize()
        runs[name] = (loss.item(), _grads(m))
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    l0, g0 = runs["scores"]
    for name, (l, g) in runs.items():
        assert abs(l - l0) <= tol * abs(l0), (name, l, l0)
        for k in g0:
            err = ((g[k] - g0[k]).norm() / g0[k].norm().clamp_min(1e-30)).item()
            assert err <= tol, (name, k, err)


@pytest.mark.gpu
def test_config5_lm_at_full_shape():
    """Benchmark config 5 at its own shape: d=768, 12 heads, SwiGLU intermediate 2048, [2 -> 4x4 -> 2], vocab 32000,
    batch 8 x seq 2048, bf16 weights, uniform random ids, the HIP read on the stacked layout with stored scores.
      * at init (zero queries) the loss equals bitwise that of the same model with the reference read (the oracle
        cell on the same GPU: every other op is the same kernel), as the reference's whole-model check;
      * with a learned query (N(0, 0.02^2), as the benchmark's), one training step: every read of the pass, on a
        subset of tokens (the read is per token), against the oracle on the recorded inputs -- out and the installed
        coefficients within 1e-2 x max |ref| of the exact (fp64) read of the same base (at an iteration end the
        caller's blend proposal + beta (h0 - proposal), rounded to bf16 op by op as the caller's torch ops round it:
        the oracle cell in fp64 would blend exactly, a difference of the caller's glue, not of the read), and no
        further from it than the bf16 reference read (<= 2 err_ref + 2e-3); the loss within 1e-2 of the
        reference-read model's; every parameter gradient finite, the query's nonzero; an optimizer step keeps the
        loss finite."""
    from gpu_helpers import err_max
    torch.manual_seed(5)
    cfg = LMConfig()
    assert (cfg.hidden_size, cfg.num_heads, cfg.intermediate, cfg.topology(), cfg.vocab_size) == \
        (768, 12, 2048, "[2->4x4->2]", 32000)
    model = LoopbackLM(cfg)
    ids = torch.randint(0, cfg.vocab_size, (8, 2048), generator=torch.Generator().manual_seed(5)).cuda()
    hip = copy.deepcopy(model).to(device="cuda", dtype=torch.bfloat16)
    ref = copy.deepcopy(model).to(device="cuda", dtype=torch.bfloat16)
    ref.read = OracleRead(ref.read)
    print("case config5 at init", flush=True)
    with torch.no_grad():
        la, lb = hip(ids), ref(ids)
    assert torch.equal(la, lb), (la.item(), lb.item())

    with torch.no_grad():
        hip.read.query.normal_(0, 0.02)
        ref.read.query.copy_(hip.read.query)
    g = torch.Generator().manual_seed(6)
    sub = torch.randperm(8 * 2048, generator=g)[:64].sort().values.cuda()
    pick = lambda t: t.detach().reshape(-1, t.shape[-1])[sub].unsqueeze(0).cpu()
    records = []
    combine = hip.read.combine

    def recording(proposal, h0, deltas, coeffs, prior, loop_idx, block_idx, keys=None, stack=None):
        out = combine(proposal, h0, deltas, coeffs, prior, loop_idx, block_idx, keys=keys, stack=stack)
        records.append((pick(proposal), pick(h0), [pick(x) for x in deltas],
                        None if coeffs is None else pick(coeffs), None if prior is None else prior.detach().cpu(),
                        loop_idx, block_idx, pick(out[0]), pick(out[1])))
        return out

    hip.read.combine = recording
    print("case config5 training step", flush=True)
    opt = make_optimizer(hip)
    loss = hip(ids)
    loss.backward()
    torch.cuda.synchronize()
    hip.read.combine = combine
    with torch.no_grad():
        lref = ref(ids)
    assert abs(loss.item() - lref.item()) <= 1e-2 * abs(lref.item()), (loss.item(), lref.item())
    grads = _grads(hip)
    assert all(torch.isfinite(v).all() for v in grads.values())
    assert grads["read.query"].abs().sum().item() > 0
    K, R = cfg.loop_blocks, cfg.loops
    q = hip.read.query.detach().cpu()
    assert len(records) == K * R
    from oracle.reference_read import read_core
    for proposal, h0, deltas, coeffs, prior, l, blk, out, tc in records:
        n = len(deltas)
        if n < 2:
            continue
        step = l * K + blk
        at_end = blk == K - 1
        base = proposal + cfg.beta * (h0 - proposal) if at_end else proposal    # bf16, the caller's roundings
        lam = 1.0 - cfg.beta if at_end else 1.0
        cbar = torch.cat((coeffs.double(), torch.ones(*coeffs.shape[:-1], 1, dtype=torch.float64)), -1) * lam
        c0 = torch.cat((prior.double(), torch.ones(1, dtype=torch.float64)), -1) * lam
        o64, t64 = read_core(q[step - 1].double(), base.double(), cbar, c0, [x.double() for x in deltas],
                             cfg.norm_eps)
        o16, t16 = read_core(q[step - 1].float(), base, cbar.float(), c0.float(), deltas, cfg.norm_eps)
        for hip_v, v64, v16 in ((out, o64, o16), (tc, t64, t16)):
            e, e_ref = err_max(hip_v, v64), err_max(v16, v64)
            assert e <= 1e-2 and e <= 2 * e_ref + 2e-3, (l, blk, e, e_ref)
    opt.step()
    opt.zero_grad(set_to_none=True)
    with torch.no_grad():
        assert torch.isfinite(hip(ids)).all()


def _fp32_attention(q, k, v, is_causal=True):
    """Causal attention by explicit fp32 products of contiguous operands, rounded back to the input dtype: the same
    bits on every run (the library kernels may split their sums differently), as the reference's layout test runs
    its model with a reference attention (tests/test_dattn_stack.py:34-47)."""
    qf, kf, vf = q.float().contiguous(), k.float().contiguous(), v.float().contiguous()
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * qf.shape[-1] ** -0.5
    T = s.shape[-1]
    s = s.masked_fill(torch.ones(T, T, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s, -1), vf).to(q.dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("glue", ["0", "1"])
def test_lm_layout_contract(monkeypatch, dtype, glue):
    """The reference's whole-model layout test (tests/test_dattn_stack.py:129-160) on this LM with a deterministic
    attention: with LOOP_DATTN_GRAD_ROUNDING=per_read the stacked layout with online scores is the list layout bit
    for bit -- loss, logits and every parameter gradient -- in bf16 (the reference's training dtype), fp16 and fp32;
    with the default rounding, the stacked layout with stored scores within the reference's bar of the list layout
    (norm-relative 1e-5 in fp32, 3e-2 in bf16, fp16 3.75e-3), logits and every gradient. The list run twice gives the
    same bits first, so the comparisons are of the read's layouts alone."""
    import torch.nn.functional as F
    monkeypatch.setattr(F, "scaled_dot_product_attention", _fp32_attention)
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    torch.manual_seed(4)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg)
    with torch.no_grad():
        model.read.query.normal_(0, 0.3)
    ids = ids_for(cfg, b=2, t=48, seed=1).cuda()
    print(f"case LM layout contract {dtype} glue={glue}", flush=True)

    def run(stack, dots, rounding):
        monkeypatch.setenv("LOOP_DATTN_STACK", stack)
        monkeypatch.setenv("LOOP_DATTN_DOTS", dots)
        monkeypatch.setenv("LOOP_DATTN_GRAD_ROUNDING", rounding)
        m = copy.deepcopy(model).to(device="cuda", dtype=dtype)
        logits = m.head(m.hidden(ids))
        labels = torch.cat((ids[:, 1:], torch.full_like(ids[:, :1], -100)), dim=1)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), labels.reshape(-1), ignore_index=-100)
        loss.backward()
        torch.cuda.synchronize()
        return loss.item(), logits.detach().cpu(), {k: p.grad.detach().cpu() for k, p in m.named_parameters()
                                                   if p.grad is not None}

    ll, Ll, gl = run("0", "1", "once")
    ll2, Ll2, gl2 = run("0", "1", "once")
    assert ll == ll2 and torch.equal(Ll, Ll2) and all(torch.equal(gl[k], gl2[k]) for k in gl)
    ls, Ls, gs = run("1", "0", "per_read")
    assert ls == ll and torch.equal(Ls, Ll)
    assert set(gs) == set(gl) and all(torch.equal(gs[k], gl[k]) for k in gl), \
        [k for k in gl if not torch.equal(gs[k], gl[k])]
    lw, Lw, gw = run("1", "1", "once")
    tol = {torch.float32: 1e-5, torch.bfloat16: 3e-2, torch.float16: 3e-2 / 8}[dtype]
    rel = lambda a, b: ((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30)).item()
    assert rel(Lw, Ll) <= tol
    assert max(rel(gw[k], gl[k]) for k in gl) <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("stack,dots", [("1", "1"), ("1", "0"), ("0", "1")])
def test_lm_training_memory_is_steady(monkeypatch, stack, dots):
    """A training loop (loss, backward, optimizer step) through every read layout: once the optimizer's state exists
    (after the first step), the allocated device memory between steps is the same after every step -- nothing of a
    pass (its stack, the reads' kept output gradients, address tables, scale gradients) outlives it."""
    monkeypatch.setenv("LOOP_DATTN_STACK", stack)
    monkeypatch.setenv("LOOP_DATTN_DOTS", dots)
    torch.manual_seed(5)
    cfg = LMConfig(**TINY)
    model = LoopbackLM(cfg).to(device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        model.read.query.normal_(0, 0.3)
    opt = make_optimizer(model)
    ids = ids_for(cfg, b=2, t=256).cuda()
    print(f"case LM memory stack={stack} dots={dots}", flush=True)
    seen = []
    for _ in range(6):
        loss = train_step(model, opt, ids)
        del loss
        torch.cuda.synchronize()
        seen.append(torch.cuda.memory_allocated())
    assert len(set(seen[1:])) == 1, seen
