"""A minimal Loopback language model with the HIP read integrated, and its training step (the model of
looped_transformer.py:5-33, 431-615, restated for this build; trainer checkpoints are out of scope).

Architecture (`LMConfig`): token embedding; pre-RMSNorm blocks of causal multi-head attention with RoPE and a
SwiGLU MLP (intermediate = the multiple of 256 at or above 2/3 * hidden * hidden_ratio); topology
[P -> K x R -> C]: P unique prelude blocks, R iterations over K shared blocks, C unique coda blocks; final RMSNorm,
LM head (optionally tied to the embedding), next-token cross entropy. The residual rule between the middle block
applications is Loopback's read (`residual="delta_attnres"`, `loopback_amd.cell.LoopDeltaAttnRes` on the stacked
layout: each block update is written into the stack, the read combines them) or plain addition (`residual=None`,
Plain Loop). Init: every Linear and the embedding N(0, initializer_range), RMSNorm gains 1, the read query zero.

MI355X choices (not the reference's parameterization): q, k, v come from one fused projection and the MLP's gate and
up from another (one GEMM each instead of three / two); attention is torch's SDPA restricted to its flash and
memory-efficient kernels in 16-bit (never the math path's batched products in bf16).

    python -m loopback_amd.lm --steps 10 --warmup 3            # config 5: the Loopback LM step, tokens/s
    python -m loopback_amd.lm --residual none                  # the same model as Plain Loop
    python -m loopback_amd.lm --prefill --batch 8 --seq 4096 [--graph]   # no-grad forward, tokens/s
"""
from __future__ import annotations

import argparse
import gc
import json
import sys
import time
from dataclasses import asdict, dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .cell import LoopDeltaAttnRes


@dataclass
class LMConfig:
    hidden_size: int = 768
    num_heads: int = 12
    vocab_size: int = 32000
    prelude: int = 2            # P
    loop_blocks: int = 4        # K
    loops: int = 4              # R
    coda: int = 2               # C
    hidden_ratio: int = 4
    intermediate_size: int | None = None
    rope_theta: float = 1e6
    norm_eps: float = 1e-6
    initializer_range: float = 0.02
    tie_word_embeddings: bool = False
    residual: str | None = "delta_attnres"
    beta: float = 0.75

    def __post_init__(self):
        if self.hidden_size % self.num_heads:
            raise ValueError(f"hidden_size {self.hidden_size} not divisible by num_heads {self.num_heads}")
        if (self.hidden_size // self.num_heads) % 2:
            raise ValueError("RoPE needs an even head dimension")
        if self.residual not in (None, "delta_attnres"):
            raise ValueError(f"residual must be None or 'delta_attnres', got {self.residual!r}")
        if min(self.prelude, self.coda) < 0 or min(self.loop_blocks, self.loops) < 1:
            raise ValueError("prelude, coda >= 0 and loop_blocks, loops >= 1")
        if not 0.0 <= float(self.beta) < 1.0:
            raise ValueError(f"beta must be in [0, 1), got {self.beta}")

    @property
    def intermediate(self) -> int:
        if self.intermediate_size is not None:
            return self.intermediate_size
        size = int(self.hidden_size * self.hidden_ratio * 2 / 3)
        return 256 * ((size + 255) // 256)

    def topology(self) -> str:
        return f"[{self.prelude}->{self.loop_blocks}x{self.loops}->{self.coda}]"


CONFIG5 = LMConfig()   # the benchmark's config 5: d=768, 12 heads, SwiGLU 8/3 (2048), [2 -> 4x4 -> 2], vocab 32000


class Rotary(nn.Module):
    """Non-interleaved RoPE: the two halves of each head rotate as pairs; cos / sin from fp32 positions and inverse
    frequencies, rounded to the activation dtype (as the reference caches them), the rotation computed in fp32 and
    rounded back. q and k rotate in one pass."""

    def __init__(self, head_dim: int, theta: float):
        super().__init__()
        self.head_dim, self.theta = head_dim, float(theta)
        self._cache = None

    def tables(self, seq: int, device, dtype):
        """Full-width fp32 (seq, head_dim) cos and sin (each half-table repeated), through `dtype`."""
        c = self._cache
        if c is None or c[0] < seq or c[1].device != device or c[3] != dtype:
            inv = 1.0 / (self.theta ** (torch.arange(0, self.head_dim, 2, device=device, dtype=torch.float32)
                                        / self.head_dim))
            f = torch.outer(torch.arange(seq, device=device, dtype=torch.float32), inv)
            cos = torch.cos(f).to(dtype).float()
            sin = torch.sin(f).to(dtype).float()
            self._cache = c = (seq, torch.cat((cos, cos), -1), torch.cat((sin, sin), -1), dtype)
        return c[1][:seq], c[2][:seq]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: (B, T, ..., head_dim) -> rotated, same dtype."""
        T, hd = x.shape[1], self.head_dim
        cos, sin = self.tables(T, x.device, x.dtype)
        shape = (1, T) + (1,) * (x.dim() - 3) + (hd,)
        xf = x.float()
        rot = torch.cat((-xf[..., hd // 2:], xf[..., :hd // 2]), -1)
        return (xf * cos.view(shape) + rot * sin.view(shape)).to(x.dtype)


def attention_kernels(dtype):
    """SDPA backends: flash / memory-efficient only in 16-bit; fp32 may also take the math path."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    kinds = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
    if dtype == torch.float32 or dtype == torch.float64:
        kinds.append(SDPBackend.MATH)
    return sdpa_kernel(kinds)


class Attention(nn.Module):
    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.h, self.dh = cfg.num_heads, cfg.hidden_size // cfg.num_heads
        self.qkv = nn.Linear(cfg.hidden_size, 3 * cfg.hidden_size, bias=False)
        self.o = nn.Linear(cfg.hidden_size, cfg.hidden_size, bias=False)
        self.rotary = Rotary(self.dh, cfg.rope_theta)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, D = x.shape
        qkv = self.qkv(x).view(B, T, 3, self.h, self.dh)
        q, k = self.rotary(qkv[:, :, :2]).permute(2, 0, 3, 1, 4).unbind(0)   # (B, H, T, dh) views
        v = qkv[:, :, 2].transpose(1, 2)
        if x.is_cuda:
            with attention_kernels(x.dtype):
                a = F.scaled_dot_product_attention(q, k, v.contiguous(), is_causal=True)
        else:
            a = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.o(a.transpose(1, 2).reshape(B, T, D))


class SwiGLU(nn.Module):
    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.gate_up = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate, bias=False)
        self.down = nn.Linear(cfg.intermediate, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g, u = self.gate_up(x).chunk(2, dim=-1)
        return self.down(F.silu(g) * u)


class Block(nn.Module):
    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.attn_norm = nn.RMSNorm(cfg.hidden_size, eps=cfg.norm_eps)
        self.attn = Attention(cfg)
        self.mlp_norm = nn.RMSNorm(cfg.hidden_size, eps=cfg.norm_eps)
        self.mlp = SwiGLU(cfg)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.attn_norm(x))
        return x + self.mlp(self.mlp_norm(x))


class LoopbackLM(nn.Module):
    """The causal LM. `forward(ids)` returns the mean next-token loss (labels = ids shifted, the last position
    ignored), as the reference LM's forward with labels=input_ids."""

    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.prelude = nn.ModuleList(Block(cfg) for _ in range(cfg.prelude))
        self.middle = nn.ModuleList(Block(cfg) for _ in range(cfg.loop_blocks))   # shared over the R iterations
        self.coda = nn.ModuleList(Block(cfg) for _ in range(cfg.coda))
        self.norm = nn.RMSNorm(cfg.hidden_size, eps=cfg.norm_eps)
        self.head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        self.read = (LoopDeltaAttnRes(cfg.hidden_size, cfg.loops, cfg.loop_blocks, beta=cfg.beta, eps=cfg.norm_eps)
                     if cfg.residual == "delta_attnres" else None)
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        std = self.cfg.initializer_range
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, mean=0.0, std=std)
            elif isinstance(m, nn.RMSNorm):
                nn.init.ones_(m.weight)
        if self.read is not None:
            self.read.reset_parameters()
        if self.cfg.tie_word_embeddings:
            self.head.weight = self.embed.weight

    def hidden(self, ids: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        h = self.embed(ids)
        for blk in self.prelude:
            h = blk(h)
        K = cfg.loop_blocks
        if self.read is None:                                   # Plain Loop
            for k in range(K * cfg.loops):
                h = self.middle[k % K](h)
        else:                                                   # Loopback (modeling_looped_transformer.py:437-481)
            h0 = h
            stack = None
            if h.is_cuda and hasattr(self.read, "new_stack"):
                stack = self.read.new_stack(h.shape, h.dtype, h.device)
            deltas, keys, coeffs, prior = [], [], None, None
            for k in range(K * cfg.loops):
                l, blk = divmod(k, K)
                x = h
                hs = self.middle[blk](x)
                if stack is not None:
                    deltas.append(stack.write(k, hs, x))
                    h, coeffs, prior = self.read.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys,
                                                         stack=stack)
                else:
                    deltas.append(hs - x)
                    h, coeffs, prior = self.read.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys)
        for blk in self.coda:
            h = blk(h)
        return self.norm(h)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        logits = self.head(self.hidden(ids))
        labels = torch.cat((ids[:, 1:], torch.full_like(ids[:, :1], -100)), dim=1)
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), labels.reshape(-1), ignore_index=-100)

    def num_params(self) -> int:
        seen = {id(p): p.numel() for p in self.parameters()}
        return sum(seen.values())


def train_step(model: LoopbackLM, opt: torch.optim.Optimizer, ids: torch.Tensor) -> torch.Tensor:
    """One training step: loss, backward, optimizer step, gradients released. Returns the loss (not synchronized)."""
    loss = model(ids)
    loss.backward()
    opt.step()
    opt.zero_grad(set_to_none=True)
    return loss.detach()


def make_optimizer(model: nn.Module) -> torch.optim.Optimizer:
    return torch.optim.AdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                             foreach=True)


def bench(argv=None):
    ap = argparse.ArgumentParser(description="config 5: the Loopback LM training step on one GPU")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--residual", default="delta_attnres", choices=["delta_attnres", "none"])
    ap.add_argument("--prefill", action="store_true",
                    help="time the no-grad forward (logits) instead of the training step; with --graph replayed as "
                         "one HIP graph")
    ap.add_argument("--graph", action="store_true")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("lm: no GPU visible", file=sys.stderr)
        sys.exit(3)
    if a.prefill:
        dev = torch.device("cuda", 0)
        cfg = LMConfig(residual=None if a.residual == "none" else "delta_attnres")
        torch.manual_seed(0)
        model = LoopbackLM(cfg).to(device=dev, dtype=torch.bfloat16)
        gen = torch.Generator(device=dev).manual_seed(1)
        ids = torch.randint(0, cfg.vocab_size, (a.batch, a.seq), device=dev, generator=gen)
        return _prefill(model, cfg, ids, a)
    print(json.dumps(time_training(a.steps, a.warmup, a.batch, a.seq, a.residual)), flush=True)


def time_training(steps: int = 10, warmup: int = 3, batch: int = 8, seq: int = 2048,
                  residual: str = "delta_attnres") -> dict:
    """Config 5's training step on cuda:0 -- the random-init LM in bf16, uniform random ids (batch, seq), AdamW --
    timed over `steps` steps after `warmup`; residual "none" is the same model as Plain Loop. Returns the record."""
    dev = torch.device("cuda", 0)
    cfg = LMConfig(residual=None if residual == "none" else "delta_attnres")
    torch.manual_seed(0)
    model = LoopbackLM(cfg).to(device=dev, dtype=torch.bfloat16)
    gen = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq), device=dev, generator=gen)
    opt = make_optimizer(model)
    for _ in range(warmup):
        train_step(model, opt, ids)
    torch.cuda.synchronize()
    gc.collect()
    gc.freeze()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = train_step(model, opt, ids)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gc.unfreeze()
    tokens = batch * seq
    rec = {"metric": "LM training step tokens/sec (config 5)", "value": tokens * steps / dt, "unit": "tokens/s",
           "ms_per_step": 1e3 * dt / steps, "steps": steps, "warmup": warmup, "loss": float(loss),
           "params": model.num_params(), "dtype": "bf16", "data": "uniform random token ids",
           "optimizer": "AdamW (foreach)",
           "config": {"topology": cfg.topology(), **asdict(cfg), "batch": batch, "seq": seq}}
    del model, opt, ids
    torch.cuda.empty_cache()
    return rec


def _prefill(model: LoopbackLM, cfg: LMConfig, ids: torch.Tensor, a) -> None:
    """No-grad forward to the logits (the reference's prefill measurement, results/README.md:163-177), eagerly or
    replayed from one HIP graph (the read records nothing for a backward and allocates nothing itself)."""
    model.eval()

    def fwd():
        return model.head(model.hidden(ids))

    with torch.no_grad():
        for _ in range(a.warmup):
            fwd()
        torch.cuda.synchronize()
        if a.graph:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                fwd()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                fwd()
            run = graph.replay
        else:
            run = fwd
        run()
        torch.cuda.synchronize()
        gc.collect()
        gc.freeze()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            run()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    tokens = a.batch * a.seq
    print(json.dumps({"metric": "LM prefill tokens/sec (no-grad forward to logits)", "value": tokens * a.steps / dt,
                      "unit": "tokens/s", "ms_per_pass": 1e3 * dt / a.steps, "steps": a.steps, "graph": a.graph,
                      "dtype": "bf16", "data": "uniform random token ids",
                      "config": {"topology": cfg.topology(), "residual": cfg.residual, "batch": a.batch,
                                 "seq": a.seq}}), flush=True)


if __name__ == "__main__":
    bench()
