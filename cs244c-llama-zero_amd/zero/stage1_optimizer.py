"""ZeRO stage 1 — sharded fp32 master/moments, gradient all-reduce, updated
parameter all-gather (reference: zero/stage1_optimizer.py:30-189), single GPU.

Same fused data path as stage 0 on this rank's shard [r*ceil(P/ws), ...) (the
whole flat buffer at world_size 1); AdamW writes the updated shard in the
parameter dtype straight into the flat parameter buffer, which is what the
all-gather + assign_flat_params produce in the reference.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, Tuple

import torch

from lzhip import ops

from .common import (
    ShardSpec,
    assign_flat_params,
    compute_shard_spec,
    flatten_param_shard_fp32,
    flatten_params_dtype,
    views_into,
)
from .stage0_ddp import ZeROStage0DDP


@dataclass
class ZeROStage1Optimizer(ZeROStage0DDP):
    """Stage 1: shard optimizer state, allreduce full gradients, allgather updated params."""

    _stage_label = "stage1"

    def _init_state(self) -> None:
        self.shard: ShardSpec = compute_shard_spec(self.meta.total_numel, rank=self.rank, world_size=self.world_size)
        self.local_master_param_shard = flatten_param_shard_fp32(self.meta, self.shard.shard_start,
                                                                 self.shard.shard_end)
        n = self.local_master_param_shard.shape
        self.exp_avg = ops.zeros(n, torch.float32, self.meta.device)
        self.exp_avg_sq = ops.zeros(n, torch.float32, self.meta.device)

    def _master(self) -> torch.Tensor:
        return self.local_master_param_shard

    def _shard_range(self) -> Tuple[int, int]:
        return self.shard.shard_start, self.shard.shard_end

    def _publish_params(self, written_in_place: bool) -> float:
        if written_in_place and self.collectives.is_identity:
            return 0.0  # the updated shard already is the whole parameter buffer
        s0, s1 = self._shard_range()
        local = self._flat_params[s0:s1] if written_in_place else ops.cast(self._master(), self.param_dtype)
        t0 = time.perf_counter()
        with self.collectives.label_scope("stage1.step.allgather.updated_param_shard"):
            full = self.collectives.allgather(local)
        comm_ms = (time.perf_counter() - t0) * 1000.0
        assign_flat_params(self.meta, full[: self.meta.total_numel])
        if not written_in_place:
            self._flat_params = flatten_params_dtype(self.meta, self.param_dtype)
            views_into(self.meta, self._flat_params)
        return comm_ms

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
            "hparams": self._hparams(),
        }

    def load_state_dict(self, state: Dict[str, object]) -> None:
        dev = self.meta.device
        self.step_count = int(state["step_count"])
        self.local_master_param_shard = state["local_master_param_shard"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg = state["exp_avg"].to(device=dev, dtype=torch.float32).contiguous()
        self.exp_avg_sq = state["exp_avg_sq"].to(device=dev, dtype=torch.float32).contiguous()
        self._write_params_from_master()
