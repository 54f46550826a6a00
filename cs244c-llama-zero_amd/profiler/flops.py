"""Closed-form training FLOPs (reference: profiler/flops.py:30-63) and the
torch.profiler-based FlopTracker (profiler/flops.py:67-100)."""
from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import TYPE_CHECKING, Callable, Dict, List, Optional, TypeVar

import torch

if TYPE_CHECKING:
    from model.config import ModelConfig

T = TypeVar("T")


@dataclass
class FlopSnapshot:
    label: str
    total_flops: float

    def to_dict(self) -> Dict[str, float | str]:
        return asdict(self)


def flops_to_tflops_per_second(total_flops: float, step_time_s: float) -> float:
    if total_flops < 0.0 or step_time_s <= 0.0:
        raise ValueError("total_flops must be >= 0 and step_time_s must be > 0")
    return float(total_flops) / 1e12 / float(step_time_s)


def forward_flops_breakdown(cfg: "ModelConfig", batch_size: int, seq_len: int) -> Dict[str, float]:
    """Per-forward FLOPs by component, as the reference estimator counts them
    (attention scores/apply over the full S x S square)."""
    tokens = float(batch_size * seq_len)
    d, L, f = float(cfg.dim), float(cfg.n_layers), float(cfg.ffn_dim)
    heads, hd = float(cfg.n_heads), float(cfg.head_dim)
    kv = float(cfg.n_kv_heads * cfg.head_dim)
    V = float(cfg.vocab_size)
    proj = 2.0 * tokens * (2.0 * d * d + 2.0 * d * kv)
    score = 2.0 * float(batch_size) * heads * float(seq_len) * float(seq_len) * hd
    mlp = 2.0 * tokens * d * f * 3.0
    pointwise = tokens * (8.0 * d + 4.0 * f)
    lm_head = 2.0 * tokens * d * V
    return {
        "attn_proj": L * proj,
        "attn_score": L * score,
        "attn_apply": L * score,
        "mlp": L * mlp,
        "norm_pointwise": L * pointwise,
        "lm_head": lm_head,
    }


def estimate_transformer_train_flops(
    cfg: "ModelConfig",
    batch_size: int,
    seq_len: int,
    grad_accum_steps: int = 1,
    world_size: int = 1,
    stage: int = 0,
) -> float:
    """Forward FLOPs x 3 (x 4 for ZeRO-3's recomputed forward) x micro-batches x ranks."""
    if batch_size <= 0 or seq_len <= 0 or grad_accum_steps <= 0 or world_size <= 0:
        raise ValueError("batch_size, seq_len, grad_accum_steps, and world_size must be positive")
    fwd = sum(forward_flops_breakdown(cfg, batch_size, seq_len).values())
    mult = 4.0 if stage == 3 else 3.0
    return fwd * mult * float(grad_accum_steps * world_size)


@dataclass
class FlopTracker:
    device: Optional[torch.device] = None
    snapshots: List[FlopSnapshot] = None

    def __post_init__(self) -> None:
        if self.snapshots is None:
            self.snapshots = []

    def measure(self, label: str, fn: Callable[[], T]) -> tuple[T, float | None]:
        acts = [torch.profiler.ProfilerActivity.CPU]
        gpu = self.device is not None and self.device.type == "cuda" and torch.cuda.is_available()
        if gpu:
            acts.append(torch.profiler.ProfilerActivity.CUDA)
        with torch.profiler.profile(activities=acts, with_flops=True, acc_events=True) as prof:
            result = fn()
            if gpu:
                torch.cuda.synchronize(self.device)
        total = float(sum(float(getattr(e, "flops", 0.0) or 0.0) for e in prof.key_averages()))
        if total <= 0.0:
            return result, None
        self.snapshots.append(FlopSnapshot(label=label, total_flops=total))
        return result, total

    def as_dicts(self) -> List[Dict[str, float | str]]:
        return [s.to_dict() for s in self.snapshots]
