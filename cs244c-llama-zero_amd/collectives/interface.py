"""Collective-communication interface consumed by the ZeRO engines
(reference: collectives/interface.py:30-78, 246-338).

This build runs on one GPU, where every collective is the identity:
LocalCollectives keeps the reference's return semantics (allreduce/allgather/
reduce_scatter return a flattened copy, allreduce_inplace returns its input),
TracingCollectives records per-call labels, byte counts and timings.  The
multi-process implementations (ring send/recv, torch.distributed) are not part
of this single-GPU build: constructing them raises.
"""
from __future__ import annotations

import time
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Dict, Iterator, List

import torch
import torch.distributed as dist


def _copy(t: torch.Tensor) -> torch.Tensor:
    flat = t.contiguous().view(-1)
    if flat.device.type == "cuda":
        from lzhip import ops

        return ops.cast(flat, flat.dtype)
    return flat.clone()


@dataclass
class CollectiveOps:
    """Black-box communication interface consumed by ZeRO wrappers."""

    def allreduce(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        raise NotImplementedError

    def allreduce_inplace(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        reduced = self.allreduce(tensor, average=average)
        if reduced.data_ptr() != tensor.data_ptr():
            tensor.copy_(reduced)
        return tensor

    def reduce_scatter(self, tensor: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def allgather(self, local_shard: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    @contextmanager
    def label_scope(self, label: str) -> Iterator[None]:
        del label
        yield

    def consume_trace(self) -> List[Dict[str, object]]:
        return []

    # True when every operation is the identity on this process's data (one
    # rank): engines may then use the input buffer instead of a returned copy.
    @property
    def is_identity(self) -> bool:
        return False


@dataclass
class LocalCollectives(CollectiveOps):
    """Single-process collectives (world_size 1)."""

    def allreduce(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        return _copy(tensor).view_as(tensor)  # dividing by world size 1 is the identity

    def allreduce_inplace(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        return tensor

    def reduce_scatter(self, tensor: torch.Tensor) -> torch.Tensor:
        return _copy(tensor)

    def allgather(self, local_shard: torch.Tensor) -> torch.Tensor:
        return _copy(local_shard)

    @property
    def is_identity(self) -> bool:
        return True


class _MultiProcessUnavailable(CollectiveOps):
    def __init__(self, *args, **kwargs) -> None:
        raise RuntimeError(
            f"{type(self).__name__} exchanges data between processes; this build runs the ZeRO engines on one GPU "
            "(world_size=1), where LocalCollectives is the collective implementation."
        )


class SendRecvCollectives(_MultiProcessUnavailable):
    """Ring collectives over point-to-point send/recv (multi-process only)."""


class TorchCollectives(_MultiProcessUnavailable):
    """torch.distributed collectives (multi-process only)."""


@dataclass
class TracingCollectives(CollectiveOps):
    """Collective wrapper that records per-call timing and tensor sizes."""

    inner: CollectiveOps

    def __post_init__(self) -> None:
        self._label_stack: List[str] = []
        self._trace: List[Dict[str, object]] = []

    @property
    def is_identity(self) -> bool:
        return False  # calls must go through so they are recorded

    @staticmethod
    def _world_size() -> int:
        if dist.is_available() and dist.is_initialized():
            return int(dist.get_world_size())
        return 1

    def _record(self, *, op: str, input_tensor: torch.Tensor, output_tensor: torch.Tensor, elapsed_ms: float) -> None:
        self._trace.append(
            {
                "op": op,
                "label": "/".join(self._label_stack),
                "input_bytes": int(input_tensor.numel() * input_tensor.element_size()),
                "output_bytes": int(output_tensor.numel() * output_tensor.element_size()),
                "elapsed_ms": float(elapsed_ms),
                "world_size": self._world_size(),
                "device": str(input_tensor.device),
                "dtype": str(input_tensor.dtype).replace("torch.", ""),
            }
        )

    @contextmanager
    def label_scope(self, label: str) -> Iterator[None]:
        self._label_stack.append(label)
        try:
            yield
        finally:
            self._label_stack.pop()

    def consume_trace(self) -> List[Dict[str, object]]:
        trace = list(self._trace)
        self._trace.clear()
        return trace

    def _timed(self, op: str, fn, tensor: torch.Tensor, *args):
        t0 = time.perf_counter()
        out = fn(tensor, *args)
        self._record(op=op, input_tensor=tensor, output_tensor=out, elapsed_ms=(time.perf_counter() - t0) * 1000.0)
        return out

    def allreduce(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        return self._timed("allreduce", self.inner.allreduce, tensor, average)

    def allreduce_inplace(self, tensor: torch.Tensor, average: bool = False) -> torch.Tensor:
        return self._timed("allreduce_inplace", self.inner.allreduce_inplace, tensor, average)

    def reduce_scatter(self, tensor: torch.Tensor) -> torch.Tensor:
        return self._timed("reduce_scatter", self.inner.reduce_scatter, tensor)

    def allgather(self, local_shard: torch.Tensor) -> torch.Tensor:
        return self._timed("allgather", self.inner.allgather, local_shard)
