"""ZeRO stage 2 — sharded optimizer state and gradients, replicated parameters
(reference: zero/stage2_optimizer.py:30-311), single GPU.

Post-accumulate-grad hooks add each parameter's gradient into one flat
param-dtype buffer (in-place HIP add) and release p.grad; at the end of
backward the buffer is reduce-scattered (identity at world_size 1) and
accumulated into the fp32 gradient shard; step() clips on the global norm and
runs the fused AdamW, writing the updated parameters into the flat parameter
buffer the model's parameters are views of.  Buffer lifetimes (allocated in
zero_grad, released after step) follow the reference, since its memory
accounting is part of the API.
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
    ShardSpec,
    assign_flat_params,
    build_flat_param_metadata,
    bytes_to_mb,
    compute_shard_spec,
    flatten_param_shard_fp32,
    flatten_params_dtype,
    get_rank_world_size,
    grads_num_bytes,
    model_param_dtype,
    params_num_bytes,
    tensor_num_bytes,
    tensors_num_bytes,
    views_into,
)
from .stage0_ddp import _require_single_rank


@dataclass
class ZeROStage2Optimizer:
    """Stage 2: shard optimizer state and gradients, keep params replicated."""

    model: nn.Module
    lr: float = 3e-4
    betas: Tuple[float, float] = (0.9, 0.95)
    eps: float = 1e-8
    weight_decay: float = 0.1
    grad_bucket_numel: int = 16 * 1024 * 1024
    collectives: Optional[CollectiveOps] = None
    memory_tracker: Optional[MemoryTracker] = None
    memory_trace_active: bool = False
    memory_state_timeline: Optional[List[Dict[str, object]]] = None

    def __post_init__(self) -> None:
        self.rank, self.world_size = get_rank_world_size()
        _require_single_rank(self.world_size)
        if self.collectives is None:
            self.collectives = LocalCollectives()
        self.meta = build_flat_param_metadata(self.model)
        self.param_dtype = model_param_dtype(self.meta)
        self.shard: ShardSpec = compute_shard_spec(self.meta.total_numel, rank=self.rank, world_size=self.world_size)
        self.local_master_param_shard = flatten_param_shard_fp32(self.meta, self.shard.shard_start, self.shard.shard_end)
        dev = self.meta.device
        self.exp_avg = ops.zeros(self.local_master_param_shard.shape, torch.float32, dev)
        self.exp_avg_sq = ops.zeros(self.local_master_param_shard.shape, torch.float32, dev)
        self.grad_shard: Optional[torch.Tensor] = None
        self.flat_grad_buffer: Optional[torch.Tensor] = None
        self._flat_grad_buffer_dirty = False
        self.step_count = 0
        self._reset_comm_stats()
        self._flat_params = flatten_params_dtype(self.meta, self.param_dtype)
        views_into(self.meta, self._flat_params)
        self._fused = FusedStep(dev)
        self._register_grad_hooks()

    def _reset_comm_stats(self) -> None:
        self._backward_comm_ms = 0.0
        self._post_step_allgather_ms = 0.0
        self._backward_reduce_scatter_calls = 0
        self._post_step_allgather_calls = 0
        self._backward_reduce_scatter_bytes = 0
        self._post_step_allgather_bytes = 0

    def backward(self, loss: torch.Tensor) -> None:
        backward_from_loss(loss)
        self._flush_flat_grad_buffer()

    def prepare_forward(self) -> Dict[str, float]:
        return {"prepare_comm_ms": 0.0}

    def zero_grad(self) -> None:
        self._reset_comm_stats()
        dev = self.meta.device
        self.grad_shard = ops.zeros((self.shard.shard_numel,), torch.float32, dev)
        self.flat_grad_buffer = ops.zeros((self.meta.total_numel,), self.param_dtype, dev)
        self._flat_grad_buffer_dirty = False
        for p in self.meta.params:
            p.grad = None

    def _register_grad_hooks(self) -> None:
        for idx, param in enumerate(self.meta.params):

            def _hook(grad_param: torch.Tensor, *, _idx: int = idx) -> None:
                del grad_param
                p = self.meta.params[_idx]
                if p.grad is None:
                    return
                if self.flat_grad_buffer is None:
                    raise RuntimeError("stage2 flat_grad_buffer must be initialized in zero_grad before backward")
                start = self.meta.offsets[_idx]
                g = p.grad.detach()
                if not g.is_contiguous():
                    g = g.contiguous()
                dst = self.flat_grad_buffer[start : start + p.numel()]
                if g.dtype != self.param_dtype:
                    g = ops.cast(g.view(-1), self.param_dtype)
                ops.add_(dst, g.view(-1))
                self._flat_grad_buffer_dirty = True
                p.grad = None

            param.register_post_accumulate_grad_hook(_hook)

    def _flush_flat_grad_buffer(self) -> None:
        if self.flat_grad_buffer is None or not self._flat_grad_buffer_dirty:
            return
        self._record_memory_event("measured_step_stage2_pre_reduce_scatter")
        t0 = time.perf_counter()
        if self.collectives.is_identity:
            reduced = self.flat_grad_buffer
        else:
            with self.collectives.label_scope("stage2.backward.reduce_scatter.flat_grad_buffer"):
                reduced = self.collectives.reduce_scatter(self.flat_grad_buffer)
        self._backward_comm_ms += (time.perf_counter() - t0) * 1000.0
        self._backward_reduce_scatter_calls += 1
        self._backward_reduce_scatter_bytes += tensor_num_bytes(self.flat_grad_buffer)
        self._record_memory_event("measured_step_stage2_post_reduce_scatter")
        if self.grad_shard is None:
            self.grad_shard = ops.zeros((self.shard.shard_numel,), torch.float32, self.meta.device)
        n = self.shard.shard_numel
        ops.axpy_f32_(self.grad_shard, reduced[:n], 1.0 / self.world_size)
        ops.fill_(self.flat_grad_buffer, 0.0)
        self._flat_grad_buffer_dirty = False

    def _record_memory_event(self, label: str) -> None:
        if self.memory_tracker is None or not self.memory_trace_active:
            return
        self.memory_tracker.record(label)
        if self.memory_state_timeline is not None:
            self.memory_state_timeline.append(
                {"label": label, **self.live_model_state_breakdown_mb(), **self._debug_memory_components_mb()}
            )

    def _debug_memory_components_mb(self) -> Dict[str, float]:
        esz = torch.tensor([], dtype=self.param_dtype).element_size()
        return {
            "logical_params_mb": bytes_to_mb(params_num_bytes(self.meta.params)),
            "logical_grads_mb": bytes_to_mb(self.shard.shard_numel * esz),
            "logical_optimizer_mb": bytes_to_mb(
                tensors_num_bytes([self.local_master_param_shard, self.exp_avg, self.exp_avg_sq])
            ),
            "live_full_grads_mb": bytes_to_mb(grads_num_bytes(self.meta.params)),
            "live_flat_grad_buffer_mb": bytes_to_mb(tensor_num_bytes(self.flat_grad_buffer)),
            "live_grad_shard_mb": bytes_to_mb(tensor_num_bytes(self.grad_shard)),
            "comm_temp_mb": 0.0,
        }

    def debug_memory_components_mb(self) -> Dict[str, float]:
        return self._debug_memory_components_mb()

    def step_with_stats(self, max_grad_norm: float = 0.0) -> Dict[str, float]:
        t0 = time.perf_counter()
        if any(p.grad is not None for p in self.meta.params):
            raise RuntimeError("Stage 2 should drain param.grad into the contiguous flat buffer during backward")
        self._flush_flat_grad_buffer()
        if self.grad_shard is None:
            raise RuntimeError("Stage 2 grad_shard must be initialized before optimizer step")

        self._fused.grad_norm_and_scale([self.grad_shard], max_grad_norm)
        t_opt0 = time.perf_counter()
        self.step_count += 1
        s0, s1 = self.shard.shard_start, self.shard.shard_end
        base = self._flat_params.data_ptr()
        esz = self._flat_params.element_size()
        in_place = all(p.data.data_ptr() == base + o * esz for p, o in zip(self.meta.params, self.meta.offsets))
        self._fused.adamw(self.local_master_param_shard, self.exp_avg, self.exp_avg_sq, self.grad_shard, lr=self.lr,
                          betas=self.betas, eps=self.eps, weight_decay=self.weight_decay, step=self.step_count,
                          max_grad_norm=max_grad_norm, p_out=self._flat_params[s0:s1] if in_place else None)
        optim_ms = (time.perf_counter() - t_opt0) * 1000.0

        self._record_memory_event("measured_step_stage2_pre_allgather")
        t1 = time.perf_counter()
        local = self._flat_params[s0:s1] if in_place else ops.cast(self.local_master_param_shard, self.param_dtype)
        if not (in_place and self.collectives.is_identity):
            with self.collectives.label_scope("stage2.step.allgather.updated_param_shard"):
                full = self.collectives.allgather(local)
            assign_flat_params(self.meta, full[: self.meta.total_numel])
            if not in_place:
                self._flat_params = flatten_params_dtype(self.meta, self.param_dtype)
                views_into(self.meta, self._flat_params)
        self._post_step_allgather_ms += (time.perf_counter() - t1) * 1000.0
        self._post_step_allgather_calls += 1
        self._post_step_allgather_bytes += tensor_num_bytes(local)
        self._record_memory_event("measured_step_stage2_post_allgather")

        self.grad_shard = None
        self.flat_grad_buffer = None
        self._flat_grad_buffer_dirty = False
        self._record_memory_event("measured_step_stage2_post_step_free_grad_shard")
        grad_norm = self._fused.read_norm()
        return {
            "grad_norm": grad_norm,
            "comm_ms": self._backward_comm_ms + self._post_step_allgather_ms,
            "communication_backward_reduce_scatter_ms": self._backward_comm_ms,
            "communication_backward_reduce_scatter_calls": float(self._backward_reduce_scatter_calls),
            "communication_backward_reduce_scatter_bytes": float(self._backward_reduce_scatter_bytes),
            "communication_post_allgather_ms": self._post_step_allgather_ms,
            "communication_post_allgather_calls": float(self._post_step_allgather_calls),
            "communication_post_allgather_bytes": float(self._post_step_allgather_bytes),
            "optim_ms": optim_ms,
            "total_ms": (time.perf_counter() - t0) * 1000.0,
        }

    def step(self, max_grad_norm: float = 0.0) -> float:
        return float(self.step_with_stats(max_grad_norm=max_grad_norm)["grad_norm"])

    def memory_state_breakdown_mb(self) -> Dict[str, float]:
        esz = torch.tensor([], dtype=self.param_dtype).element_size()
        params_mb = bytes_to_mb(params_num_bytes(self.meta.params))
        grads_mb = bytes_to_mb(self.shard.shard_numel * esz)
        optimizer_mb = bytes_to_mb(tensors_num_bytes([self.local_master_param_shard, self.exp_avg, self.exp_avg_sq]))
        return {"params_mb": params_mb, "grads_mb": grads_mb, "optimizer_mb": optimizer_mb,
                "total_mb": params_mb + grads_mb + optimizer_mb}

    def live_model_state_breakdown_mb(self) -> Dict[str, float]:
        params_mb = bytes_to_mb(params_num_bytes(self.meta.params))
        grads_mb = bytes_to_mb(
            grads_num_bytes(self.meta.params) + tensor_num_bytes(self.flat_grad_buffer) + tensor_num_bytes(self.grad_shard)
        )
        optimizer_mb = bytes_to_mb(tensors_num_bytes([self.local_master_param_shard, self.exp_avg, self.exp_avg_sq]))
        return {"params_mb": params_mb, "grads_mb": grads_mb, "optimizer_mb": optimizer_mb,
                "total_mb": params_mb + grads_mb + optimizer_mb}

    def state_dict(self) -> Dict[str, object]:
        return {
            "step_count": self.step_count,
            "rank": self.rank,
            "world_size": self.world_size,
            "shard_start": self.shard.shard_start,
            "shard_end": self.shard.shard_end,
            "local_master_param_shard": self.local_master_param_shard.detach().cpu(),
            "exp_avg": self.exp_avg.detach().cpu(),
            "exp_avg_sq": self.exp_avg_sq.detach().cpu(),
            "grad_shard": None if self.grad_shard is None else self.grad_shard.detach().cpu(),
            "hparams": {"lr": self.lr, "betas": self.betas, "eps": self.eps, "weight_decay": self.weight_decay},
        }

    def load_state_dict(self, state: Dict[str, object]) -> None:
        dev = self.meta.device
        self.step_count = int(state["step_count"])
        self.local_master_param_shard = state["local_master_param_shard"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg = state["exp_avg"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg_sq = state["exp_avg_sq"].to(device=dev, dtype=torch.float32).contiguous()
        gs = state.get("grad_shard")
        self.grad_shard = None if gs is None else gs.to(device=dev, dtype=torch.float32).contiguous()
        s0, s1 = self.shard.shard_start, self.shard.shard_end
        ops.cast(self.local_master_param_shard, self.param_dtype, out=self._flat_params[s0:s1])
        views_into(self.meta, self._flat_params)
