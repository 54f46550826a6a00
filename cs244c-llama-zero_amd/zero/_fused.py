"""The optimizer arithmetic every ZeRO stage shares, as HIP kernels.

Reference semantics (zero/stage0_ddp.py:66-88; identical update in stage1/2/3):
global L2 norm of the fp32 gradients, clip by max/(norm+1e-6) when
0 < max < norm, then AdamW on the fp32 master with the step counter
incremented first.  Here the norm is accumulated on the device (sum of squares
in float64), the clip factor is computed on the device and read by the AdamW
kernel, and the host reads the norm once at the end of the step — the only
synchronisation the reference's API (a float grad_norm) requires.

With clipping off (the reference's default max_grad_norm = 0.0) the norm is
only reported: when it is taken over exactly the gradient buffer AdamW reads,
the AdamW pass accumulates it (lz_adamw_norm) instead of a pass of its own.
"""
from __future__ import annotations

from typing import Iterable, Optional, Tuple

import torch

from lzhip import ops


class FusedStep:
    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.sumsq = ops.zeros((1,), torch.float64, device)
        self.norm = torch.empty((1,), dtype=torch.float32, device=device)
        self.scale = torch.empty((1,), dtype=torch.float32, device=device)
        self._deferred: Optional[torch.Tensor] = None  # gradient whose norm the next adamw() sums
        self._workspace: Optional[torch.Tensor] = None

    def grad_norm_and_scale(self, grads: Iterable[torch.Tensor], max_grad_norm: float) -> None:
        """norm = ||concat(grads)||_2 and the clip factor, both on the device.

        Without clipping and with a single gradient buffer, the sum of squares
        is left to the AdamW pass over that buffer (adamw below); read_norm()
        computes it separately if no such pass comes."""
        ops.fill_(self.sumsq, 0.0)
        live = [g for g in grads if g is not None and g.numel()]
        if max_grad_norm <= 0 and len(live) == 1:
            self._deferred = live[0]
            return
        self._deferred = None
        for g in live:
            ops.sumsq_(g, self.sumsq)
        ops.clip_finalize(self.sumsq, float(max_grad_norm), self.norm, self.scale)

    def _finish_deferred(self) -> None:
        g, self._deferred = self._deferred, None
        if g is not None:
            ops.sumsq_(g, self.sumsq)
        ops.clip_finalize(self.sumsq, 0.0, self.norm, self.scale)

    def adamw(self, master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor, grads: torch.Tensor,
              *, lr: float, betas: Tuple[float, float], eps: float, weight_decay: float, step: int,
              max_grad_norm: float, p_out: Optional[torch.Tensor] = None) -> None:
        g = self._deferred
        fuse = (g is not None and max_grad_norm <= 0 and master.numel() > 0 and g.dtype == grads.dtype
                and g.numel() == grads.numel() and g.data_ptr() == grads.data_ptr())
        if g is not None and not fuse:
            self._finish_deferred()
        if master.numel() == 0:
            return
        if fuse:
            self._deferred = None
            words = ops.adamw_norm_workspace_words(master.numel())
            if self._workspace is None or self._workspace.numel() < words:
                self._workspace = torch.empty((words,), dtype=torch.float64, device=self.device)
            ops.adamw_norm_(master, exp_avg, exp_avg_sq, grads, self.sumsq, self._workspace, lr=lr, beta1=betas[0],
                            beta2=betas[1], eps=eps, weight_decay=weight_decay, step=step, p_out=p_out)
            ops.clip_finalize(self.sumsq, float(max_grad_norm), self.norm, self.scale)
            return
        ops.adamw_(master, exp_avg, exp_avg_sq, grads, lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
                   weight_decay=weight_decay, step=step, grad_scale=self.scale if max_grad_norm > 0 else None,
                   p_out=p_out)

    def read_norm(self) -> float:
        if self._deferred is not None:
            self._finish_deferred()
        return float(self.norm.item())
