"""Memory snapshots with the reference's API (profiler/memory.py:13-99:
MemorySnapshot, take_memory_snapshot, MemoryTracker.record / reset_peak_stats
/ peak_stats_mb / as_dicts), whose snapshot fields are part of the profile
JSON that train_zero.py writes.

Design: the device figures come from one read of the caching allocator's
statistics (torch.cuda.memory_stats) per snapshot.  Those counters change
when the host allocates or frees, not when the GPU runs, so a snapshot waits
only for the current stream (the work enqueued so far) rather than the
whole device.  Host memory is the process's peak resident set.
"""
from __future__ import annotations

import resource
import sys
import time
from dataclasses import asdict, dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

_MIB = float(1 << 20)


def _on_gpu(device: Optional[torch.device]) -> bool:
    return device is not None and device.type == "cuda" and torch.cuda.is_available()


def _host_peak_rss_mb() -> float:
    peak = float(resource.getrusage(resource.RUSAGE_SELF).ru_maxrss)
    # ru_maxrss is in bytes on macOS and in KiB on Linux
    return peak / _MIB if sys.platform == "darwin" else peak / 1024.0


def _device_counters_mb(device: Optional[torch.device]) -> Tuple[float, float, float, float]:
    """(allocated, reserved, peak allocated, peak reserved) in MiB."""
    if not _on_gpu(device):
        return 0.0, 0.0, 0.0, 0.0
    st = torch.cuda.memory_stats(device)
    keys = ("allocated_bytes.all.current", "reserved_bytes.all.current", "allocated_bytes.all.peak",
            "reserved_bytes.all.peak")
    return tuple(float(st.get(k, 0)) / _MIB for k in keys)  # type: ignore[return-value]


@dataclass
class MemorySnapshot:
    label: str
    timestamp_s: float
    host_maxrss_mb: float
    cuda_allocated_mb: float
    cuda_reserved_mb: float
    cuda_max_allocated_mb: float
    cuda_max_reserved_mb: float

    @classmethod
    def capture(cls, label: str, device: Optional[torch.device] = None) -> "MemorySnapshot":
        return cls(label, time.time(), _host_peak_rss_mb(), *_device_counters_mb(device))

    def to_dict(self) -> Dict[str, float | str]:
        return asdict(self)


def take_memory_snapshot(label: str, device: Optional[torch.device] = None) -> MemorySnapshot:
    return MemorySnapshot.capture(label, device)


@dataclass
class MemoryTracker:
    device: Optional[torch.device] = None
    snapshots: List[MemorySnapshot] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.snapshots is None:
            self.snapshots = []

    def synchronize(self) -> None:
        """Waits for the work enqueued so far on the current stream."""
        if _on_gpu(self.device):
            torch.cuda.current_stream(self.device).synchronize()

    def record(self, label: str) -> MemorySnapshot:
        self.synchronize()
        snap = MemorySnapshot.capture(label, self.device)
        self.snapshots.append(snap)
        return snap

    def reset_peak_stats(self) -> None:
        if _on_gpu(self.device):
            self.synchronize()
            torch.cuda.reset_peak_memory_stats(self.device)

    def peak_stats_mb(self) -> Dict[str, float]:
        self.synchronize()
        _, _, peak_alloc, peak_res = _device_counters_mb(self.device)
        return {"peak_allocated_mb": peak_alloc, "peak_reserved_mb": peak_res}

    def as_dicts(self) -> List[Dict[str, float | str]]:
        return [s.to_dict() for s in self.snapshots]
