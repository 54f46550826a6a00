"""torch.optim-compatible AdamW on the fused HIP kernel, for the single-process
trainer (reference train.py:206-211,259-271: torch.optim.AdamW with
clip_grad_norm_).

FusedAdamW implements torch.optim.AdamW's update (decoupled weight decay,
bias-corrected moments) with one multi-tensor kernel launch per 24
parameters.  Parameters in a
low-precision dtype get an fp32 master copy and fp32 moments; the kernel writes
the rounded parameter back.  clip_grad_norm_() computes the global gradient
norm and the clip factor on the device; the factor is folded into the next
step() instead of rescaling every gradient in a separate pass.

LossScaler is torch.cuda.amp.GradScaler's dynamic loss scaling for fp16
training (reference train.py:213-214,254-269) over FusedAdamW: the backward
is seeded with the scale instead of multiplying the loss, unscaling rides on
clip_grad_norm_'s factor, and a step whose gradients hold an inf or NaN is
skipped and halves the scale.
"""
from __future__ import annotations

import math
from typing import Iterable, Optional

import torch

from . import ops


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params: Iterable, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, capturable: bool = False) -> None:
        """capturable=True keeps each group's step count on the device
        (advanced by a kernel each step), so that a step recorded in a HIP
        graph (torch.cuda.graph) is correct on every replay; the learning rate
        is then fixed at capture time."""
        if lr < 0.0 or eps < 0.0 or weight_decay < 0.0:
            raise ValueError("lr, eps and weight_decay must be non-negative")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))
        self.capturable = bool(capturable)
        self._grad_scale: Optional[torch.Tensor] = None
        self._norm_buf: Optional[torch.Tensor] = None

    def _params_with_grad(self):
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    yield group, p

    @torch.no_grad()
    def clip_grad_norm_(self, max_norm: float, inv_grad_scale: float = 1.0) -> torch.Tensor:
        """Returns the global L2 norm of all gradients (a device scalar) and
        arms the clip factor max/(norm+1e-6) (when norm > max) for step().
        With inv_grad_scale (1 / a loss scale the gradients carry) the norm
        returned is the unscaled one, and the armed factor also unscales."""
        dev = None
        for _, p in self._params_with_grad():
            dev = p.grad.device
            break
        if dev is None:
            return torch.zeros((), dtype=torch.float32)
        acc = ops.zeros((1,), torch.float64, dev)
        by_dtype = {}
        for _, p in self._params_with_grad():
            g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            by_dtype.setdefault(g.dtype, []).append(g)
        for grads in by_dtype.values():
            ops.sumsq_multi_(grads, acc)
        norm = torch.empty((1,), dtype=torch.float32, device=dev)
        scale = torch.empty((1,), dtype=torch.float32, device=dev)
        ops.clip_finalize(acc, float(max_norm), norm, scale, inv_grad_scale)
        self._grad_scale = scale if (max_norm > 0 or inv_grad_scale != 1.0) else None
        return norm.view(())

    def discard_step(self) -> None:
        """Drops the factor armed by clip_grad_norm_ when step() is skipped."""
        self._grad_scale = None

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        hypers = {}
        if self.capturable:
            for group in self.param_groups:
                if not any(p.grad is not None for p in group["params"]):
                    continue
                dev = next(p.device for p in group["params"] if p.grad is not None)
                if "step_dev" not in group:
                    group["step_dev"] = ops.zeros((1,), torch.int64, dev)
                    group["hyper_dev"] = ops.zeros((3,), torch.float32, dev)
                beta1, beta2 = group["betas"]
                ops.adamw_step_(group["step_dev"], group["lr"], beta1, beta2, group["weight_decay"],
                                group["hyper_dev"])
                hypers[id(group)] = group["hyper_dev"]
        batches = {}
        for group, p in self._params_with_grad():
            ops.require_gpu(p)
            st = self.state[p]
            if not st:
                if self.capturable and group.get("_steps_taken", 0) > 0:
                    # the group's one device step count would bias-correct this
                    # parameter as if it had been stepped from the start
                    raise RuntimeError(
                        "FusedAdamW(capturable=True) keeps one device step count per parameter group: every "
                        "parameter of a group must receive a gradient from the group's first step on "
                        f"(a parameter of shape {tuple(p.shape)} got its first gradient at step "
                        f"{group['_steps_taken'] + 1})")
                st["step"] = 0
                st["exp_avg"] = ops.zeros(p.shape, torch.float32, p.device)
                st["exp_avg_sq"] = ops.zeros(p.shape, torch.float32, p.device)
                if p.dtype != torch.float32:
                    st["master"] = ops.cast(p.detach().contiguous(), torch.float32)
            st["step"] += 1
            master = st.get("master")
            g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            if master is None:
                if not p.is_contiguous():
                    raise ValueError("FusedAdamW needs contiguous parameters")
                target, out = p.data, None
            else:
                target, out = master, p.data
            key = (id(group), g.dtype, None if out is None else out.dtype, st["step"])
            batch = batches.setdefault(key, (group, [], [], [], [], []))
            for lst, t in zip(batch[1:], (target, st["exp_avg"], st["exp_avg_sq"], g, out)):
                lst.append(t)
        if self.capturable:
            for group in self.param_groups:
                if any(p.grad is not None for p in group["params"]):
                    group["_steps_taken"] = group.get("_steps_taken", 0) + 1
        # one multi-tensor launch per (group, dtypes, step) batch
        for key, (group, ps, ms, vs, gs, outs) in batches.items():
            beta1, beta2 = group["betas"]
            ops.adamw_multi_(ps, ms, vs, gs, outs, lr=group["lr"], beta1=beta1, beta2=beta2, eps=group["eps"],
                             weight_decay=group["weight_decay"], step=key[3], grad_scale=self._grad_scale,
                             hyper=hypers.get(id(group)))
        self._grad_scale = None
        return loss


class LossScaler:
    """Dynamic loss scaling with torch.cuda.amp.GradScaler's schedule and
    defaults (reference train.py:213-214,254-269): gradients are computed for
    loss * scale; a step whose gradients hold an inf or NaN is skipped and
    the scale multiplied by backoff_factor; after growth_interval finite steps
    in a row it is multiplied by growth_factor.  Disabled, it is the
    identity.  Use with FusedAdamW:

        seed = scaler.scale_value() / accum_steps     # backward's seed
        ...backward of every micro-batch...
        norm = scaler.unscale_(optimizer, max_norm)  # true norm, clip armed
        scaler.step(optimizer, float(norm))          # skipped if not finite
        scaler.update()
    """

    def __init__(self, init_scale: float = 2.0 ** 16, growth_factor: float = 2.0, backoff_factor: float = 0.5,
                 growth_interval: int = 2000, enabled: bool = True) -> None:
        if not (growth_factor > 1.0 and 0.0 < backoff_factor < 1.0 and growth_interval > 0 and init_scale > 0):
            raise ValueError("invalid loss scaler settings")
        self._enabled = bool(enabled)
        self._scale = float(init_scale)
        self.growth_factor = float(growth_factor)
        self.backoff_factor = float(backoff_factor)
        self.growth_interval = int(growth_interval)
        self._growth_tracker = 0
        self._found_inf: Optional[bool] = None

    def is_enabled(self) -> bool:
        return self._enabled

    def scale_value(self) -> float:
        """The current scale (1.0 when disabled)."""
        return self._scale if self._enabled else 1.0

    def get_scale(self) -> float:
        return self.scale_value()

    def unscale_(self, optimizer: FusedAdamW, max_norm: float = 0.0) -> torch.Tensor:
        """The global norm of the unscaled gradients (device scalar; inf or
        NaN when they overflowed), with optimizer's next step armed to unscale
        and, when max_norm > 0, clip them."""
        return optimizer.clip_grad_norm_(max_norm, 1.0 / self.scale_value())

    def step(self, optimizer: FusedAdamW, grad_norm: float) -> bool:
        """optimizer.step() unless grad_norm is inf or NaN; returns whether
        the step ran."""
        finite = math.isfinite(grad_norm)
        self._found_inf = not finite
        if finite or not self._enabled:
            optimizer.step()
            return True
        optimizer.discard_step()
        return False

    def update(self) -> None:
        if not self._enabled or self._found_inf is None:
            return
        if self._found_inf:
            self._scale *= self.backoff_factor
            self._growth_tracker = 0
        else:
            self._growth_tracker += 1
            if self._growth_tracker == self.growth_interval:
                self._scale *= self.growth_factor
                self._growth_tracker = 0
        self._found_inf = None

    def state_dict(self) -> dict:
        if not self._enabled:
            return {}
        return {"scale": self._scale, "growth_factor": self.growth_factor, "backoff_factor": self.backoff_factor,
                "growth_interval": self.growth_interval, "_growth_tracker": self._growth_tracker}

    def load_state_dict(self, state: dict) -> None:
        if not state:
            return
        self._scale = float(state["scale"])
        self.growth_factor = float(state["growth_factor"])
        self.backoff_factor = float(state["backoff_factor"])
        self.growth_interval = int(state["growth_interval"])
        self._growth_tracker = int(state["_growth_tracker"])
