"""Flat-buffer metadata and flatten/assign helpers shared by the ZeRO engines
(reference: zero/common.py).

The index maps are the reference's, bit for bit: parameters deduplicated by
identity in model.parameters() order (the tied LM head drops out), offsets are
prefix sums of numel, shard = [r*ceil(P/ws), min(+chunk, P)).  Data movement
between parameter storages and flat buffers runs as multi-tensor HIP kernels
(one launch per <=48 segments) instead of per-parameter torch copies.

Additions: bucket_ranges() (25M-element gradient buckets whose concatenation
is the flat layout) and FlatParamMetadata.segment_table() for the kernels.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Iterable, List, Optional, Sequence, Tuple

import torch
import torch.distributed as dist
import torch.nn as nn

from lzhip import ops

GRAD_BUCKET_NUMEL = 25_000_000


@dataclass
class FlatParamMetadata:
    params: List[nn.Parameter]
    offsets: List[int]
    shapes: List[torch.Size]
    total_numel: int
    device: torch.device

    @property
    def numels(self) -> List[int]:
        return [math.prod(s) for s in self.shapes]

    def segment_table(self, tensors: Sequence[Optional[torch.Tensor]]) -> ops.HostTable:
        """Records {ptr, numel, offset} of per-parameter tensors laid out like
        the flat buffer (None reads as zeros)."""
        return ops.HostTable.from_tensors(tensors, self.offsets, self.numels)


@dataclass
class ShardSpec:
    rank: int
    world_size: int
    shard_start: int
    shard_end: int
    shard_numel: int
    chunk_size: int


_UNIT_SEEDS: dict = {}


def backward_from_loss(loss: torch.Tensor) -> None:
    """loss.backward() with the seed gradient 1 taken from a cached
    device scalar (written once by this library's fill kernel) rather than
    created by autograd's ones_like on every step."""
    if loss.device.type != "cuda" or loss.numel() != 1:
        loss.backward()
        return
    key = (loss.device, loss.dtype, tuple(loss.shape))
    seed = _UNIT_SEEDS.get(key)
    if seed is None:
        seed = _UNIT_SEEDS[key] = ops.fill_(torch.empty(loss.shape, dtype=loss.dtype, device=loss.device), 1.0)
    loss.backward(gradient=seed)


def tensor_num_bytes(tensor: torch.Tensor | None) -> int:
    if tensor is None:
        return 0
    return int(tensor.numel() * tensor.element_size())


def bytes_to_mb(num_bytes: int) -> float:
    return float(num_bytes) / (1024.0 * 1024.0)


def params_num_bytes(params: Iterable[nn.Parameter]) -> int:
    return sum(tensor_num_bytes(p.data) for p in unique_trainable_params(list(params)))


def grads_num_bytes(params: Iterable[nn.Parameter]) -> int:
    return sum(tensor_num_bytes(p.grad) for p in unique_trainable_params(list(params)))


def tensors_num_bytes(tensors: Iterable[torch.Tensor | None]) -> int:
    return sum(tensor_num_bytes(t) for t in tensors)


def get_rank_world_size() -> Tuple[int, int]:
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(), dist.get_world_size()
    return 0, 1


def unique_trainable_params(params: List[nn.Parameter]) -> List[nn.Parameter]:
    """Trainable parameters, first occurrence by identity (zero/common.py:59-70)."""
    out: List[nn.Parameter] = []
    seen = set()
    for p in params:
        if not p.requires_grad or id(p) in seen:
            continue
        seen.add(id(p))
        out.append(p)
    return out


def build_flat_param_metadata_from_params(params: List[nn.Parameter]) -> FlatParamMetadata:
    params = unique_trainable_params(params)
    if not params:
        raise ValueError("Model has no trainable parameters")
    offsets: List[int] = []
    shapes: List[torch.Size] = []
    cursor = 0
    for p in params:
        offsets.append(cursor)
        shapes.append(torch.Size(p.shape))
        cursor += p.numel()
    return FlatParamMetadata(params=params, offsets=offsets, shapes=shapes, total_numel=cursor,
                             device=params[0].device)


def build_flat_param_metadata(model: nn.Module) -> FlatParamMetadata:
    return build_flat_param_metadata_from_params(list(model.parameters()))


def compute_shard_spec(total_numel: int, rank: int, world_size: int) -> ShardSpec:
    chunk = max(1, math.ceil(total_numel / world_size))
    start = rank * chunk
    end = min(start + chunk, total_numel)
    return ShardSpec(rank=rank, world_size=world_size, shard_start=start, shard_end=end,
                     shard_numel=max(0, end - start), chunk_size=chunk)


def bucket_ranges(begin: int, end: int, bucket_numel: int = GRAD_BUCKET_NUMEL) -> List[Tuple[int, int]]:
    """[begin, end) cut into consecutive buckets of at most bucket_numel."""
    if bucket_numel <= 0:
        raise ValueError("bucket_numel must be positive")
    return [(s, min(s + bucket_numel, end)) for s in range(begin, end, bucket_numel)]


def model_param_dtype(meta: FlatParamMetadata) -> torch.dtype:
    return meta.params[0].dtype


# ---------------------------------------------------------------------------
# flatten / assign (HIP multi-tensor kernels)
# ---------------------------------------------------------------------------

def _gather(meta: FlatParamMetadata, tensors: Sequence[Optional[torch.Tensor]], src_dtype: torch.dtype,
            out: torch.Tensor, begin: int, end: int, accumulate: bool = False) -> torch.Tensor:
    if end > begin:
        ops.mt_gather_host(meta.segment_table(tensors), src_dtype, out, begin, end, accumulate=accumulate)
    return out


def flatten_params_fp32(meta: FlatParamMetadata) -> torch.Tensor:
    return flatten_params_dtype(meta, torch.float32)


def flatten_params_dtype(meta: FlatParamMetadata, dtype: torch.dtype) -> torch.Tensor:
    out = torch.empty(meta.total_numel, dtype=dtype, device=meta.device)
    return _gather(meta, [p.data for p in meta.params], model_param_dtype(meta), out, 0, meta.total_numel)


def flatten_param_shard_fp32(meta: FlatParamMetadata, shard_start: int, shard_end: int) -> torch.Tensor:
    return flatten_param_shard_dtype(meta, shard_start, shard_end, torch.float32)


def flatten_param_shard_dtype(meta: FlatParamMetadata, shard_start: int, shard_end: int,
                              dtype: torch.dtype) -> torch.Tensor:
    n = max(0, shard_end - shard_start)
    out = torch.empty(n, dtype=dtype, device=meta.device)
    return _gather(meta, [p.data for p in meta.params], model_param_dtype(meta), out, shard_start, shard_start + n)


def flatten_grads_fp32(meta: FlatParamMetadata) -> torch.Tensor:
    return flatten_grads_dtype(meta, torch.float32)


def flatten_grads_dtype(meta: FlatParamMetadata, dtype: torch.dtype, out: Optional[torch.Tensor] = None,
                        begin: int = 0, end: Optional[int] = None) -> torch.Tensor:
    """Concatenated gradients (zeros for parameters without one), or the
    [begin, end) window of that concatenation written into `out`."""
    end = meta.total_numel if end is None else end
    if out is None:
        out = torch.empty(end - begin, dtype=dtype, device=meta.device)
    grads = [p.grad for p in meta.params]
    src_dtype = next((g.dtype for g in grads if g is not None), model_param_dtype(meta))
    return _gather(meta, grads, src_dtype, out, begin, end)


def assign_flat_params(meta: FlatParamMetadata, flat_params: torch.Tensor) -> None:
    """Writes flat[offset:offset+numel] into every parameter: in place when the
    parameter storage already has the shape, else into a fresh storage
    (zero/common.py:202-216)."""
    if flat_params.numel() < meta.total_numel:
        raise ValueError(f"flat_params too small: {flat_params.numel()} < {meta.total_numel}")
    targets = []
    for p, shape in zip(meta.params, meta.shapes):
        if not (p.data.shape == shape and p.data.device == flat_params.device):
            p.data = torch.empty(shape, dtype=p.dtype, device=flat_params.device)
        targets.append(p.data)
    ops.mt_scatter_host(flat_params, meta.segment_table(targets), model_param_dtype(meta), 0, meta.total_numel)


def assign_flat_grads(meta: FlatParamMetadata, flat_grads: torch.Tensor) -> None:
    if flat_grads.numel() < meta.total_numel:
        raise ValueError(f"flat_grads too small: {flat_grads.numel()} < {meta.total_numel}")
    targets = []
    for p, shape in zip(meta.params, meta.shapes):
        if p.grad is None or p.grad.shape != shape:
            p.grad = torch.empty(shape, dtype=p.dtype, device=flat_grads.device)
        targets.append(p.grad)
    ops.mt_scatter_host(flat_grads, meta.segment_table(targets), model_param_dtype(meta), 0, meta.total_numel)


def views_into(meta: FlatParamMetadata, flat: torch.Tensor) -> None:
    """Re-points every parameter at its slice of `flat` (which must already
    hold the values).  Afterwards q/k/v and gate/up are adjacent in memory and
    an optimizer can write parameters in place through the flat buffer."""
    for p, off, shape in zip(meta.params, meta.offsets, meta.shapes):
        n = math.prod(shape)
        p.data = flat[off : off + n].view(shape)
