"""Named step timers with the reference's API (profiler/timer.py:24-99:
NamedTimer.start/stop/summary, TimerRegistry.timer/summarize, TimerSummary).

Design: on a GPU a timer records HIP events on the current stream and keeps
them as pending intervals.  stop() waits only for its own end event (not for
the whole device) and returns the interval; stop(wait=False) returns
immediately and leaves the interval to be resolved when a summary is taken,
so a caller that only needs the aggregate never stalls the stream.  Events
are pooled per timer.  On the host the timer reads time.perf_counter().
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch


@dataclass
class TimerSummary:
    name: str
    count: int
    total_ms: float
    mean_ms: float
    p50_ms: float
    p95_ms: float
    min_ms: float
    max_ms: float


def _quantile(sorted_ms: List[float], q: float) -> float:
    """Nearest-rank quantile, as the reference's summary takes it
    (profiler/timer.py:62-64): the sample at index round(q*(n-1)) of the
    sorted samples, with Python's round() (ties to even)."""
    return float(sorted_ms[int(round((len(sorted_ms) - 1) * q))])


def _on_gpu(device: Optional[torch.device]) -> bool:
    return device is not None and device.type == "cuda" and torch.cuda.is_available()


@dataclass
class NamedTimer:
    name: str
    device: Optional[torch.device] = None
    _done_ms: List[float] = field(default_factory=list)
    _pending: List[Tuple[object, object]] = field(default_factory=list)
    _pool: List[object] = field(default_factory=list)
    _open: Optional[object] = None  # start event (GPU) or start time (host)

    def _event(self):
        return self._pool.pop() if self._pool else torch.cuda.Event(enable_timing=True)

    def start(self) -> None:
        if _on_gpu(self.device):
            ev = self._event()
            ev.record()
            self._open = ev
        else:
            self._open = time.perf_counter()

    def stop(self, wait: bool = True) -> float:
        """Ends the interval opened by start().  Returns its length in ms;
        with wait=False on a GPU it returns NaN and the interval is resolved
        by the next summary()."""
        if self._open is None:
            raise RuntimeError("Timer.stop() called before Timer.start()")
        begin, self._open = self._open, None
        if not isinstance(begin, torch.cuda.Event):
            ms = (time.perf_counter() - begin) * 1000.0
            self._done_ms.append(ms)
            return ms
        end = self._event()
        end.record()
        if not wait:
            self._pending.append((begin, end))
            return math.nan
        end.synchronize()
        ms = float(begin.elapsed_time(end))
        self._done_ms.append(ms)
        self._pool.extend((begin, end))
        return ms

    def _resolve(self) -> None:
        for begin, end in self._pending:
            end.synchronize()
            self._done_ms.append(float(begin.elapsed_time(end)))
            self._pool.extend((begin, end))
        self._pending.clear()

    @property
    def _samples_ms(self) -> List[float]:
        self._resolve()
        return self._done_ms

    def summary(self) -> TimerSummary:
        samples = sorted(self._samples_ms)
        if not samples:
            raise RuntimeError(f"Timer '{self.name}' has no samples")
        total = math.fsum(samples)
        return TimerSummary(name=self.name, count=len(samples), total_ms=total, mean_ms=total / len(samples),
                            p50_ms=_quantile(samples, 0.50), p95_ms=_quantile(samples, 0.95), min_ms=samples[0],
                            max_ms=samples[-1])


@dataclass
class TimerRegistry:
    device: Optional[torch.device] = None
    _timers: Dict[str, NamedTimer] = field(default_factory=dict)

    def timer(self, name: str) -> NamedTimer:
        t = self._timers.get(name)
        if t is None:
            t = self._timers[name] = NamedTimer(name=name, device=self.device)
        return t

    def summarize(self) -> Dict[str, TimerSummary]:
        return {name: t.summary() for name, t in self._timers.items() if t._samples_ms}
