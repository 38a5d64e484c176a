"""The caller of the read: Loopback's read cell `LoopDeltaAttnRes`, wired to the HIP read only.

This mirrors the cell of the reference's trainer model (modeling_looped_transformer.py:93-201; the plain-PyTorch
port's copy is looped_transformer.py:334-424) and its mode switches (`_fused_dattn`, looped_transformer.py:312-331;
stack creation, modeling_looped_transformer.py:437-444):
  * LOOP_DATTN_STACK=1 (default): the updates live in a DattnStack and the stacked kernels read it;
    LOOP_DATTN_DOTS=1 (default): the stack also stores each update's scores at its write;
  * LOOP_DATTN_STACK=0: the list layout (FusedDattnRead), one tensor per update;
  * LOOP_DATTN_FUSE_GLUE=1 (default, this build's own switch): in the stacked layout the glue below runs inside the
    read's kernels (FusedCombineStk); 0 keeps it as torch ops;
  * LOOP_DATTN_GRAD_ROUNDING=once (default, this build's own switch) or per_read: how the stacked layout rounds the
    updates' gradients (fused_dattn.grad_rounding).
The glue around the kernels -- the iteration-end blend base = proposal + beta (h0 - proposal), the coefficient
bookkeeping (cat, lambda scaling) -- is the reference's, op for op. Unlike the reference, the cell has no PyTorch
read of its own: an unsupported layout raises instead of falling back (that read lives in oracle/ as the checker).
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn

from . import fused_dattn as FD


def fuse_glue() -> bool:
    """LOOP_DATTN_FUSE_GLUE=0 keeps the caller's glue (blend, coefficient bookkeeping) as torch ops around the
    stacked read, as the reference cell has it; the default runs it inside the read's kernels."""
    return os.environ.get("LOOP_DATTN_FUSE_GLUE", "1") == "1"


def stack_mode() -> str:
    """'scores' (stacked, scores stored at write), 'stack' (stacked, online scores) or 'list', from the env flags
    read at every forward (modeling_looped_transformer.py:438-440)."""
    if os.environ.get("LOOP_DATTN_STACK", "1") != "1":
        return "list"
    return "scores" if os.environ.get("LOOP_DATTN_DOTS", "1") == "1" else "stack"


class LoopDeltaAttnRes(nn.Module):
    """Loopback's read (`delta_attnres`): after application s of shared block k the update d_s joins the history and
    h_{s+1} = h_0 + sum_{i<=s} c_{s,i} d_i with c_{s,i} = B_s softmax_i(q_s . RMSNorm(d_i) / sqrt(d) + log c0_{s,i}),
    c0_{s,i} = lambda^(floor((s+1)/K) - floor(i/K)), lambda = 1 - beta. One learned query per read (KR - 1 rows of
    width d), zero at init. Same constructor, parameter and `combine` contract as the reference cell."""

    def __init__(self, hidden_size: int, num_loops: int, num_blocks: int, beta: float = 0.75, eps: float = 1e-6):
        super().__init__()
        if num_loops < 1 or num_blocks < 1:
            raise ValueError(f"delta_attnres needs positive num_loops/num_blocks, got {num_loops}/{num_blocks}")
        if not 0.0 <= float(beta) < 1.0:
            raise ValueError(f"delta_attnres needs 0 <= beta < 1, got {beta}")
        self.dim = int(hidden_size)
        self.num_loops = int(num_loops)
        self.num_blocks = int(num_blocks)
        self.num_steps = self.num_loops * self.num_blocks
        self.beta = float(beta)
        self.eps = float(eps)
        self.query = nn.Parameter(torch.zeros(self.num_steps - 1, self.dim))
        self.reset_parameters()

    def reset_parameters(self):
        with torch.no_grad():
            self.query.zero_()

    def new_stack(self, shape, dtype, device, mode: str | None = None):
        """The pass's DattnStack for the current mode (None for the list layout)."""
        mode = stack_mode() if mode is None else mode
        if mode == "list":
            return None
        return FD.DattnStack(self.num_steps, tuple(shape), dtype, device,
                             query=self.query if mode == "scores" else None, eps=self.eps)

    def combine(self, proposal, h0, deltas, coeffs, prior_coeffs, loop_idx, block_idx, keys=None, stack=None):
        if not 0 <= block_idx < self.num_blocks:
            raise ValueError(f"delta_attnres block_idx={block_idx}, need [0,{self.num_blocks})")
        step = loop_idx * self.num_blocks + block_idx
        if step >= self.num_steps:
            raise ValueError(f"delta_attnres step {step} exceeds constructed depth {self.num_steps}")
        if len(deltas) != step + 1:
            raise ValueError(f"delta_attnres step {step} received {len(deltas)} deltas, expected {step + 1}")

        at_boundary = block_idx == self.num_blocks - 1
        if stack is not None and step >= 1 and fuse_glue():
            # the stacked read with the glue below inside its kernels (same results; no glue kernels)
            if keys is not None and len(keys) < len(deltas):
                keys.append(stack.rstd(step, deltas[-1], self.eps))
            R_list = keys if keys is not None else [FD._alias(stack.R, i) for i in range(len(deltas))]
            return FD.FusedCombineStk.apply(stack, step, self.query, proposal, h0 if at_boundary else None,
                                            coeffs, prior_coeffs, self.beta, at_boundary, *R_list)
        base = proposal + self.beta * (h0 - proposal) if at_boundary else proposal

        b, t, _ = proposal.shape
        one_tok = torch.ones(b, t, 1, device=proposal.device, dtype=torch.float32)
        one_prior = torch.ones(1, device=proposal.device, dtype=torch.float32)
        base_coeffs = one_tok if coeffs is None else torch.cat((coeffs, one_tok), dim=-1)
        next_prior = one_prior if prior_coeffs is None else torch.cat((prior_coeffs, one_prior), dim=-1)
        if at_boundary:
            r = 1.0 - self.beta
            base_coeffs = r * base_coeffs
            next_prior = r * next_prior

        if stack is not None:             # the stacked layout: the deltas are the stack's slices
            if keys is not None and len(keys) < len(deltas):
                keys.append(stack.rstd(step, deltas[-1], self.eps))
            if len(deltas) == 1:
                return base, base_coeffs, next_prior
            R_list = keys if keys is not None else [FD._alias(stack.R, i) for i in range(len(deltas))]
            out, target = FD.FusedDattnReadStk.apply(stack, step, self.query[step - 1], base, base_coeffs,
                                                     next_prior, *deltas, *R_list)
            return out, target, next_prior

        if keys is not None and len(keys) < len(deltas):
            keys.append(FD.rstd(deltas[-1], self.eps))
        if len(deltas) == 1:
            return base, base_coeffs, next_prior
        R_list = keys if keys is not None else [FD.rstd(d, self.eps) for d in deltas]
        if not FD.fused_read_supported(base, deltas, R_list, base_coeffs):
            raise RuntimeError("delta_attnres: the HIP read does not take this layout (fused_read_supported is False)")
        out, target = FD.FusedDattnRead.apply(self.query[step - 1], base, base_coeffs, next_prior, *deltas, *R_list)
        return out, target, next_prior


def remap_query(query: torch.Tensor, num_blocks: int, trained_loops: int, num_loops: int,
                policy: str = "last") -> torch.Tensor:
    """The read queries of a cell run for `num_loops` iterations, from one trained with `trained_loops`
    (scripts/eval_extra_visits.py:43-63, the `loop_dattn.query` entry): read s uses row s - 1; reads the trained
    cell had keep their row; a read past them takes, with policy "last", the row of the read at the same block
    position in the last trained iteration ((trained_loops - 1) K + s mod K - 1, when that is a read), with "zero"
    a zero row (its prior alone). Returns a new (num_blocks * num_loops - 1, d) tensor."""
    K, R0, R = int(num_blocks), int(trained_loops), int(num_loops)
    if policy not in ("last", "zero"):
        raise ValueError(f"remap_query: policy must be 'last' or 'zero', got {policy!r}")
    if query.dim() != 2 or query.shape[0] != K * R0 - 1:
        raise ValueError(f"remap_query: query must be ({K * R0 - 1}, d), got {tuple(query.shape)}")
    out = query.new_zeros((K * R - 1, query.shape[1]))
    for s in range(1, K * R):
        if s < K * R0:
            out[s - 1] = query[s - 1]
        elif policy == "last":
            row = (R0 - 1) * K + s % K - 1
            if row >= 0:
                out[s - 1] = query[row]
    return out
