"""One training step (zero_grad, forward and backward over the gradient
accumulation micro-batches, gradient clipping, AdamW) recorded once in a HIP
graph and replayed, for models small enough that host-side launch overhead
sets the step time (the reference's train.py loop, train.py:236-282, launches
every kernel from the host on every step).

The step must be free of host synchronisation and keep its buffers at fixed
addresses: the micro-batch ids live in static device tensors that each call
overwrites, gradients and temporaries come from the graph's private memory
pool, and the optimizer must be FusedAdamW(capturable=True), whose step count
and bias-correction factors are advanced by a kernel inside the graph.  The
learning rate is the one in effect at capture.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import ops


class GraphedTrainStep:
    def __init__(self, model, opt, batch_shape, grad_accum: int, max_grad_norm: float, device, grads=None) -> None:
        """grads: an optional functional.GradSink over the model's parameters
        (the backward kernels then write the gradients; no autograd
        accumulation kernels are recorded)."""
        if not getattr(opt, "capturable", False):
            raise ValueError("GraphedTrainStep needs an optimizer built with capturable=True")
        if grad_accum < 1:
            raise ValueError("grad_accum must be >= 1")
        self.model, self.opt, self.grads = model, opt, grads
        self.grad_accum, self.max_grad_norm = int(grad_accum), float(max_grad_norm)
        self.ids = [ops.zeros(tuple(batch_shape), torch.int64, device) for _ in range(grad_accum)]
        self.seed = ops.fill_(torch.empty((), dtype=torch.float32, device=device), 1.0 / self.grad_accum)
        self.graph = None
        self.loss = None

    def _body(self) -> torch.Tensor:
        if self.grads is not None:
            self.grads.begin_step()
        else:
            self.opt.zero_grad(set_to_none=True)
        loss = None
        for ids in self.ids:
            loss = self.model(input_ids=ids, labels=ids, return_logits=False).loss
            loss.backward(gradient=self.seed)  # = (loss / grad_accum).backward()
        if self.grads is not None:
            self.grads.finish()
        if self.max_grad_norm > 0:
            self.opt.clip_grad_norm_(self.max_grad_norm)
        self.opt.step()
        return loss

    def _load(self, micro_batches: Sequence[torch.Tensor]) -> None:
        if len(micro_batches) != self.grad_accum:
            raise ValueError(f"expected {self.grad_accum} micro-batches, got {len(micro_batches)}")
        for dst, src in zip(self.ids, micro_batches):
            if src.shape != dst.shape:
                raise ValueError(f"micro-batch shape {tuple(src.shape)} != {tuple(dst.shape)}")
            dst.copy_(src, non_blocking=True)

    def warmup(self, micro_batches: Sequence[torch.Tensor]) -> torch.Tensor:
        """One eager step on a side stream (a real optimizer step on these
        micro-batches); at least one must precede capture() so that optimizer
        state and workspaces exist before recording."""
        self._load(micro_batches)
        side = torch.cuda.Stream(device=self.ids[0].device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            loss = self._body()
        torch.cuda.current_stream().wait_stream(side)
        return loss

    def capture(self) -> None:
        """Records one step; recording runs nothing, so the model and
        optimizer state are unchanged until the first replay."""
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.loss = self._body()

    def __call__(self, micro_batches: Sequence[torch.Tensor]) -> torch.Tensor:
        """One optimizer step on these micro-batches by graph replay; returns
        the last micro-batch's loss (a device tensor the next call overwrites)."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self._load(micro_batches)
        self.graph.replay()
        return self.loss
