"""Optimizer-step semantics of the ZeRO engines at world_size=1, and the
single-process trainer loop, restated on the CPU.

At world_size=1 every collective of zero/stage{0,1,2,3} is the identity
(collectives/interface.py:59-78), so each stage performs: gradient (in the
parameter dtype) -> fp32 -> global L2 norm -> clip when norm > max ->
AdamW on the fp32 master (zero/stage0_ddp.py:66-88, stage1:73-146,
stage2:145-215, stage3:438-479) -> parameters = master cast to the parameter
dtype.  `EngineRef` keeps the fp32 (or fp64) master, moments and step count.

`train_reference` is the train.py loop (train.py:229-300): gradient
accumulation over micro-batches, clip_grad_norm_(max 1.0), torch.optim.AdamW.
"""
from __future__ import annotations

import math
import time
from typing import Callable, Dict, Iterator, List, Optional, Sequence

import torch

from . import model as M
from . import ops


class EngineRef:
    def __init__(self, master: torch.Tensor, *, lr: float, betas=(0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.1) -> None:
        self.master = master.clone()
        self.exp_avg = torch.zeros_like(self.master)
        self.exp_avg_sq = torch.zeros_like(self.master)
        self.lr, self.betas, self.eps, self.weight_decay = lr, tuple(betas), eps, weight_decay
        self.step_count = 0

    def step(self, flat_grad: torch.Tensor, max_grad_norm: float = 0.0) -> float:
        g = flat_grad.to(self.master.dtype).clone()
        grad_norm = float(g.norm(2).item())
        scale = ops.clip_scale(grad_norm, max_grad_norm)
        if scale != 1.0:
            g.mul_(scale)
        self.step_count += 1
        ops.adamw_update(self.master, self.exp_avg, self.exp_avg_sq, g, lr=self.lr, beta1=self.betas[0],
                         beta2=self.betas[1], eps=self.eps, weight_decay=self.weight_decay, step=self.step_count)
        return grad_norm


def train_reference(
    cfg: M.Cfg,
    P: Dict[str, torch.Tensor],
    chunks: Iterator[torch.Tensor],
    *,
    steps: int,
    grad_accum_steps: int,
    lr: float = 3e-4,
    betas=(0.9, 0.95),
    weight_decay: float = 0.1,
    max_grad_norm: float = 1.0,
    loss_chunk_size: int = 128,
    on_step: Optional[Callable[[int, float, float, Dict[str, torch.Tensor]], None]] = None,
    param_dtype: torch.dtype = torch.float32,
    low_precision_state: bool = False,
) -> Dict[str, List[float]]:
    """Runs the train.py loop on CPU tensors (P is updated in place).  Returns
    per-step mean micro-batch loss, pre-clip grad norm and step seconds.
    `on_step(step, loss, grad_norm, grads[, params])` sees the (clipped)
    gradients and, when it takes five arguments, the parameters of that step,
    before the optimizer update.

    param_dtype=torch.bfloat16 gives the reference's bf16-parameter semantics
    (train_zero.py:150-153 with an fp32 master, zero/stage0_ddp.py:44-47): the
    forward and backward see the fp32 master rounded to bf16, the update is
    applied to the fp32 master.  The arithmetic itself stays fp32.

    low_precision_state=True (with param_dtype bf16 or fp16) gives the
    reference train.py's own semantics at --dtype bfloat16 (train.py:157-160
    builds the model in that dtype, :206-211 hands its parameters to
    torch.optim.AdamW, :259-271 clips): no fp32 master; the parameters, their
    gradients and AdamW's exp_avg / exp_avg_sq are all in param_dtype, so
    clip_grad_norm_ and every op of the update round to it.  The forward and
    backward still run in fp32 arithmetic on the parameters' values, and each
    gradient is rounded to param_dtype once."""
    if low_precision_state and param_dtype == torch.float32:
        raise ValueError("low_precision_state needs a 16-bit param_dtype")
    store = param_dtype if low_precision_state else torch.float32
    params = {k: v.detach().to(store).clone().requires_grad_(True) for k, v in P.items()}
    opt = torch.optim.AdamW(list(params.values()), lr=lr, betas=betas, weight_decay=weight_decay)
    out = {"loss": [], "grad_norm": [], "seconds": []}
    for step in range(1, steps + 1):
        t0 = time.perf_counter()
        opt.zero_grad(set_to_none=True)
        if param_dtype == torch.float32:
            work = params
        else:
            work = {k: v.detach().to(param_dtype).to(torch.float32).requires_grad_(True) for k, v in params.items()}
        losses = []
        for _ in range(grad_accum_steps):
            chunk = next(chunks)
            ids = chunk[:, :-1].contiguous()
            loss = M.loss(work, cfg, ids, ids.clone(), chunk_size=loss_chunk_size)
            losses.append(float(loss.detach().item()))
            (loss / grad_accum_steps).backward()
        if work is not params:
            for k, v in params.items():
                v.grad = work[k].grad.to(store)
        if max_grad_norm > 0:
            gn = float(torch.nn.utils.clip_grad_norm_(list(params.values()), max_norm=max_grad_norm).item())
        else:
            gn = math.nan
        if on_step is not None:
            grads = {k: v.grad.detach().to(torch.float32, copy=True) for k, v in params.items()}
            if on_step.__code__.co_argcount >= 5:
                on_step(step, sum(losses) / len(losses), gn, grads, {k: v.detach().float() for k, v in params.items()})
            else:
                on_step(step, sum(losses) / len(losses), gn, grads)
        opt.step()
        out["loss"].append(sum(losses) / len(losses))
        out["grad_norm"].append(gn)
        out["seconds"].append(time.perf_counter() - t0)
    with torch.no_grad():
        for k in P:
            P[k].copy_(params[k].to(P[k].dtype))
    return out
