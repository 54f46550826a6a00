"""ZeRO stage 0 — replicated fp32 master + gradient all-reduce + AdamW
(reference: zero/stage0_ddp.py:28-169), single GPU.

Step data path on the GPU (all HIP kernels, one host sync for grad_norm):
  gradients -> flat param-dtype buffer in 25M-element buckets (multi-tensor
  gather) -> all-reduce each bucket (identity at world_size 1) -> sum of
  squares + clip factor -> fused AdamW reading the param-dtype gradient,
  updating the fp32 master/moments and writing the new parameters straight
  into the flat parameter buffer the model's parameters are views of (which
  is what assign_flat_params achieves in the reference).
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from collectives import CollectiveOps, LocalCollectives
from lzhip import ops
from profiler import MemoryTracker

from ._fused import FusedStep
from .common import (
    backward_from_loss,
    GRAD_BUCKET_NUMEL,
    assign_flat_params,
    bucket_ranges,
    build_flat_param_metadata,
    bytes_to_mb,
    flatten_grads_dtype,
    flatten_params_dtype,
    flatten_params_fp32,
    get_rank_world_size,
    grads_num_bytes,
    model_param_dtype,
    params_num_bytes,
    tensors_num_bytes,
    views_into,
)


def _require_single_rank(world_size: int) -> None:
    if world_size != 1:
        raise RuntimeError("this build runs the ZeRO engines on one GPU (world_size=1)")


@dataclass
class ZeROStage0DDP:
    """Stage 0 baseline: full replication + gradient allreduce + local AdamW update."""

    model: nn.Module
    lr: float = 3e-4
    betas: Tuple[float, float] = (0.9, 0.95)
    eps: float = 1e-8
    weight_decay: float = 0.1
    collectives: Optional[CollectiveOps] = None
    memory_tracker: Optional[MemoryTracker] = None
    memory_trace_active: bool = False
    memory_state_timeline: Optional[List[Dict[str, object]]] = None
    grad_bucket_numel: int = GRAD_BUCKET_NUMEL

    _stage_label = "stage0"

    def __post_init__(self) -> None:
        self.rank, self.world_size = get_rank_world_size()
        _require_single_rank(self.world_size)
        if self.collectives is None:
            self.collectives = LocalCollectives()
        self.meta = build_flat_param_metadata(self.model)
        self.param_dtype = model_param_dtype(self.meta)
        self._init_state()
        self.step_count = 0
        # parameters become views of one flat buffer: AdamW writes them in place
        self._flat_params = flatten_params_dtype(self.meta, self.param_dtype)
        views_into(self.meta, self._flat_params)
        self._flat_grads: Optional[torch.Tensor] = None
        self._fused = FusedStep(self.meta.device)

    # stage-specific optimizer state --------------------------------------
    def _init_state(self) -> None:
        self.master_params = flatten_params_fp32(self.meta)
        self.exp_avg = ops.zeros(self.master_params.shape, torch.float32, self.meta.device)
        self.exp_avg_sq = ops.zeros(self.master_params.shape, torch.float32, self.meta.device)

    def _master(self) -> torch.Tensor:
        return self.master_params

    def _shard_range(self) -> Tuple[int, int]:
        return 0, self.meta.total_numel

    # engine API -------------------------------------------------------------
    def backward(self, loss: torch.Tensor) -> None:
        backward_from_loss(loss)

    def prepare_forward(self) -> Dict[str, float]:
        return {"prepare_comm_ms": 0.0}

    def zero_grad(self) -> None:
        for param in self.meta.params:
            param.grad = None

    def _record_memory_event(self, label: str) -> None:
        if self.memory_tracker is None or not self.memory_trace_active:
            return
        self.memory_tracker.record(label)
        if self.memory_state_timeline is not None:
            self.memory_state_timeline.append({"label": label, **self.live_model_state_breakdown_mb()})

    def _params_are_flat_views(self) -> bool:
        base = self._flat_params.data_ptr()
        esz = self._flat_params.element_size()
        return all(p.data.data_ptr() == base + off * esz for p, off in zip(self.meta.params, self.meta.offsets))

    def _flatten_and_allreduce(self) -> Tuple[torch.Tensor, float]:
        """Gradients -> flat buffer, bucket by bucket, each bucket all-reduced."""
        if self._flat_grads is None:
            self._flat_grads = torch.empty(self.meta.total_numel, dtype=self.param_dtype, device=self.meta.device)
        flat = self._flat_grads
        comm_ms = 0.0
        for b0, b1 in bucket_ranges(0, self.meta.total_numel, self.grad_bucket_numel):
            bucket = flat[b0:b1]
            flatten_grads_dtype(self.meta, self.param_dtype, out=bucket, begin=b0, end=b1)
            t0 = time.perf_counter()
            with self.collectives.label_scope(f"{self._stage_label}.step.allreduce.grad_bucket"):
                self.collectives.allreduce_inplace(bucket, average=False)
            comm_ms += (time.perf_counter() - t0) * 1000.0
        return flat, comm_ms

    def step_with_stats(self, max_grad_norm: float = 0.0) -> Dict[str, float]:
        t0 = time.perf_counter()
        label = self._stage_label
        self._record_memory_event(f"measured_step_{label}_pre_allreduce")
        flat_grads, comm_ms = self._flatten_and_allreduce()
        self._record_memory_event(f"measured_step_{label}_post_allreduce")

        s0, s1 = self._shard_range()
        local = flat_grads[s0:s1]
        self._fused.grad_norm_and_scale([flat_grads], max_grad_norm)

        t_opt0 = time.perf_counter()
        self.step_count += 1
        in_place = self._params_are_flat_views()
        self._fused.adamw(self._master(), self.exp_avg, self.exp_avg_sq, local, lr=self.lr, betas=self.betas,
                          eps=self.eps, weight_decay=self.weight_decay, step=self.step_count,
                          max_grad_norm=max_grad_norm, p_out=self._flat_params[s0:s1] if in_place else None)
        optim_ms = (time.perf_counter() - t_opt0) * 1000.0
        comm_ms += self._publish_params(in_place)
        self._record_memory_event(f"measured_step_{label}_post_optimizer")
        grad_norm = self._fused.read_norm()
        return {
            "grad_norm": grad_norm,
            "comm_ms": comm_ms,
            "optim_ms": optim_ms,
            "total_ms": (time.perf_counter() - t0) * 1000.0,
        }

    def _publish_params(self, written_in_place: bool) -> float:
        """Makes the updated master visible in the model's parameters."""
        if not written_in_place:
            assign_flat_params(self.meta, self.master_params)
            self._flat_params = flatten_params_dtype(self.meta, self.param_dtype)
            views_into(self.meta, self._flat_params)
        return 0.0

    def step(self, max_grad_norm: float = 0.0) -> float:
        return float(self.step_with_stats(max_grad_norm=max_grad_norm)["grad_norm"])

    def _optimizer_tensors(self) -> List[torch.Tensor]:
        return [self._master(), self.exp_avg, self.exp_avg_sq]

    def memory_state_breakdown_mb(self) -> Dict[str, float]:
        params_mb = bytes_to_mb(params_num_bytes(self.meta.params))
        grads_mb = bytes_to_mb(grads_num_bytes(self.meta.params))
        optimizer_mb = bytes_to_mb(tensors_num_bytes(self._optimizer_tensors()))
        return {"params_mb": params_mb, "grads_mb": grads_mb, "optimizer_mb": optimizer_mb,
                "total_mb": params_mb + grads_mb + optimizer_mb}

    def live_model_state_breakdown_mb(self) -> Dict[str, float]:
        return self.memory_state_breakdown_mb()

    def _hparams(self) -> Dict[str, object]:
        return {"lr": self.lr, "betas": self.betas, "eps": self.eps, "weight_decay": self.weight_decay}

    def state_dict(self) -> Dict[str, object]:
        return {
            "rank": self.rank,
            "world_size": self.world_size,
            "step_count": self.step_count,
            "master_params": self.master_params.detach().cpu(),
            "exp_avg": self.exp_avg.detach().cpu(),
            "exp_avg_sq": self.exp_avg_sq.detach().cpu(),
            "hparams": self._hparams(),
        }

    def load_state_dict(self, state: Dict[str, object]) -> None:
        dev = self.meta.device
        self.step_count = int(state["step_count"])
        self.master_params = state["master_params"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg = state["exp_avg"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg_sq = state["exp_avg_sq"].to(device=dev, dtype=torch.float32).contiguous()
        self._write_params_from_master()

    def _write_params_from_master(self) -> None:
        s0, s1 = self._shard_range()
        ops.cast(self._master(), self.param_dtype, out=self._flat_params[s0:s1])
        views_into(self.meta, self._flat_params)
