"""ZeRO stage 3 — per-module parameter sharding with materialise-on-use and
backward recomputation (reference: zero/stage3_optimizer.py:43-576), single GPU.

Structure and semantics follow the reference: one handle per parameterised
module (`tok_embeddings`, `layers.i`, `norm`; the tied `lm_head` reuses the
embedding's handle), parameters resharded to empty storages between uses, a
custom autograd function that materialises a module's parameters, runs it
under no_grad, and in backward restores the RNG/autocast state, re-materialises,
recomputes and reduce-scatters the parameter gradients into the fp32 shard.

MI355X data path:
  - every handle's fp32 master / exp_avg / exp_avg_sq / grad_shard is a view of
    one engine-wide flat buffer (handle order), so the global norm, the clip
    and AdamW are one kernel launch each over all parameters;
  - materialise = one fp32 -> bf16 cast of the handle's shard into a fresh
    handle buffer whose slices become the parameters (q/k/v and gate/up then
    sit adjacent, which the fused projections use without copies);
  - gradient flatten = multi-tensor gather into 25M-element bf16 buckets (the
    reduce-scatter unit), each bucket accumulated into the fp32 shard.
At world_size 1 the all-gather and reduce-scatter are the identity and are
elided unless a tracing wrapper needs to observe them.

`recompute=False` (world_size 1 only; default True = reference behaviour)
keeps every module's forward autograd graph instead of recomputing it in
backward.  The gradients are the same (the backward of each module call is
taken with autograd.grad over the module's inputs and parameters and
flattened into the fp32 shard per call, exactly as after a recompute), the
forward runs once, and the parameters stay materialised: they live in one
engine-wide bf16 buffer that the fused AdamW rewrites in place, so the
per-module materialise casts and reshards disappear too.
"""
from __future__ import annotations

import time
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Dict, Iterator, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from collectives import CollectiveOps, LocalCollectives
from lzhip import ops
from lzhip.functional import output_unused
from profiler import MemoryTracker

from ._fused import FusedStep
from .common import (
    backward_from_loss,
    GRAD_BUCKET_NUMEL,
    FlatParamMetadata,
    ShardSpec,
    bucket_ranges,
    build_flat_param_metadata_from_params,
    bytes_to_mb,
    compute_shard_spec,
    flatten_params_fp32,
    get_rank_world_size,
    grads_num_bytes,
    model_param_dtype,
    params_num_bytes,
    tensors_num_bytes,
    unique_trainable_params,
    views_into,
)
from .stage0_ddp import _require_single_rank


def _elem_size(dtype: torch.dtype) -> int:
    return torch.tensor([], dtype=dtype).element_size()


def module_specs(model: nn.Module) -> List[Tuple[str, nn.Module]]:
    """Parameterised modules the executor wraps, in handle-creation order
    (zero/stage3_optimizer.py:313-349)."""
    specs: List[Tuple[str, nn.Module]] = [("tok_embeddings", model.tok_embeddings)]
    specs.extend((f"layers.{i}", layer) for i, layer in enumerate(model.layers))
    specs.append(("norm", model.norm))
    specs.append(("lm_head", model.lm_head))
    return specs


def plan_handles(model: nn.Module) -> List[Tuple[str, List[str], List[nn.Parameter]]]:
    """(handle name, module names, parameters) per handle: a module whose
    parameter set equals an earlier module's (the tied LM head) joins that
    handle."""
    plans: List[Tuple[str, List[str], List[nn.Parameter]]] = []
    by_ids: Dict[Tuple[int, ...], int] = {}
    for name, module in module_specs(model):
        params = unique_trainable_params(list(module.parameters(recurse=True)))
        if not params:
            continue
        key = tuple(sorted(id(p) for p in params))
        if key in by_ids:
            names = plans[by_ids[key]][1]
            if name not in names:
                names.append(name)
            continue
        by_ids[key] = len(plans)
        plans.append((name, [name], params))
    return plans


@dataclass
class _Stage3ParamHandle:
    name: str
    meta: FlatParamMetadata
    shard: ShardSpec
    collectives: CollectiveOps
    engine: Optional["ZeROStage3Optimizer"] = None
    module_names: List[str] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.param_dtype = model_param_dtype(self.meta)
        self.materialized = True
        self.pinned = False  # parameters kept materialised (recompute=False)
        # engine-owned flat state; bound by the engine right after creation
        self.local_master_param_shard: Optional[torch.Tensor] = None
        self.exp_avg: Optional[torch.Tensor] = None
        self.exp_avg_sq: Optional[torch.Tensor] = None
        self.grad_shard: Optional[torch.Tensor] = None
        # the shard holds no gradient of this step yet: the first accumulation
        # writes instead of adding (the engine's zero_grad fill is deferred)
        self.grad_fresh = False

    @property
    def world_size(self) -> int:
        return self.shard.world_size

    def materialize(self, phase: str) -> float:
        if self.materialized:
            return 0.0
        t0 = time.perf_counter()
        n = self.meta.total_numel
        if self.collectives.is_identity:
            full = ops.cast(self.local_master_param_shard, self.param_dtype)
        else:
            local = ops.cast(self.local_master_param_shard, self.param_dtype)
            with self.collectives.label_scope(f"stage3.{phase}.allgather.{self.name}"):
                full = self.collectives.allgather(local)
        views_into(self.meta, full[:n])
        self.materialized = True
        return (time.perf_counter() - t0) * 1000.0

    def reshard(self) -> None:
        if not self.materialized or self.pinned:
            return
        for p in self.meta.params:
            p.grad = None
            p.data = torch.empty(0, dtype=p.dtype, device=p.device)
        self.materialized = False

    def reset_grad(self) -> None:
        ops.fill_(self.grad_shard, 0.0)
        self.grad_fresh = False

    def accumulate_grad_shard(self, param_grads: Sequence[Optional[torch.Tensor]]) -> float:
        """Flatten the gradients (zeros for None) bucket by bucket, reduce-scatter
        each bucket, add it to the fp32 shard."""
        grads = []
        for g in param_grads:
            if g is not None and not g.is_contiguous():
                g = g.contiguous()
            grads.append(g)
        table = self.meta.segment_table(grads)
        src_dtype = next((g.dtype for g in grads if g is not None), self.param_dtype)
        if self.collectives.is_identity and self.world_size == 1:
            # One rank: the reduce-scatter returns the bucket unchanged, so the
            # gradients go straight into the fp32 shard in one launch, written
            # on the step's first contribution and added afterwards.  Same
            # values as the bucket path (16-bit -> fp32 is exact, the add is
            # the same fp32 add), without the bucket's write and read.
            ops.mt_gather_host(table, src_dtype, self.grad_shard, 0, self.meta.total_numel,
                               accumulate=not self.grad_fresh)
            self.grad_fresh = False
            return 0.0
        comm_ms = 0.0
        for b0, b1 in bucket_ranges(0, self.meta.total_numel, self.engine.grad_bucket_numel):
            bucket = self.engine._bucket_buffer(b1 - b0, self.param_dtype)
            ops.mt_gather_host(table, src_dtype, bucket, b0, b1)
            t0 = time.perf_counter()
            if self.collectives.is_identity:
                reduced = bucket
            else:
                with self.collectives.label_scope(f"stage3.backward.reduce_scatter.{self.name}"):
                    reduced = self.collectives.reduce_scatter(bucket)
                if reduced.numel() < b1 - b0:
                    raise ValueError(f"reduce_scatter returned too few elements: {reduced.numel()} < {b1 - b0}")
            comm_ms += (time.perf_counter() - t0) * 1000.0
            if self.grad_fresh and self.world_size == 1:
                ops.cast(reduced[: b1 - b0], torch.float32, out=self.grad_shard[b0:b1])
            else:
                ops.axpy_f32_(self.grad_shard[b0:b1], reduced[: b1 - b0], 1.0 / self.world_size)
        self.grad_fresh = False
        return comm_ms


class _ShardedModuleFunction(torch.autograd.Function):
    """Materialise -> no-grad forward -> reshard; in backward restore RNG and
    autocast state, re-materialise, recompute with grad, reduce-scatter the
    parameter gradients (zero/stage3_optimizer.py:106-243)."""

    @staticmethod
    def forward(ctx, runner, autograd_token: torch.Tensor, *args):
        del autograd_token
        ctx.runner = runner
        ctx.arg_is_tensor = [torch.is_tensor(a) for a in args]
        ctx.arg_requires_grad = []
        ctx.non_tensor_args = []
        tensor_args: List[torch.Tensor] = []
        for a in args:
            if torch.is_tensor(a):
                tensor_args.append(a.detach())
                ctx.arg_requires_grad.append(bool(a.requires_grad and (a.is_floating_point() or a.is_complex())))
                ctx.non_tensor_args.append(None)
            else:
                ctx.arg_requires_grad.append(False)
                ctx.non_tensor_args.append(a)
        eng, h = runner.engine, runner.handle
        if not eng.recompute:
            # keep the module's own graph: inputs detached (grad-requiring
            # ones marked), parameters already materialised
            rebuilt: List[object] = []
            grad_inputs: List[torch.Tensor] = []
            it = iter(tensor_args)
            with torch.enable_grad():
                for is_t, rg, nt in zip(ctx.arg_is_tensor, ctx.arg_requires_grad, ctx.non_tensor_args):
                    if not is_t:
                        rebuilt.append(nt)
                        continue
                    t = next(it)
                    if rg:
                        t = t.detach().requires_grad_(True)
                        grad_inputs.append(t)
                    rebuilt.append(t)
                out = runner.module(*rebuilt)
            ctx.inner = (out, grad_inputs)
            eng._record_forward_allgather_ms(0.0, num_bytes=0)
            return out.detach()
        ctx.save_for_backward(*tensor_args)
        ctx.cpu_rng_state = torch.get_rng_state()
        dev = runner.device
        if dev.type == "cuda" and torch.cuda.is_available():
            idx = dev.index if dev.index is not None else torch.cuda.current_device()
            ctx.cuda_rng_state = torch.cuda.get_rng_state(idx)
            ctx.autocast_enabled = torch.is_autocast_enabled()
            ctx.autocast_dtype = torch.get_autocast_dtype("cuda")
        else:
            ctx.cuda_rng_state = None
            ctx.autocast_enabled = torch.is_autocast_cpu_enabled() if dev.type == "cpu" else False
            ctx.autocast_dtype = torch.get_autocast_dtype("cpu") if dev.type == "cpu" else torch.float32

        nbytes = h.meta.total_numel * _elem_size(h.param_dtype)
        eng._record_memory_event(f"measured_step_stage3_{runner.name}_pre_allgather_forward")
        eng._record_forward_allgather_ms(h.materialize("forward"), num_bytes=nbytes)
        eng._record_memory_event(f"measured_step_stage3_{runner.name}_post_allgather_forward")
        with torch.no_grad():
            out = runner.module(*args)
        eng._record_memory_event(f"measured_step_stage3_{runner.name}_after_forward")
        h.reshard()
        eng._record_memory_event(f"measured_step_stage3_{runner.name}_after_forward_discard")
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        runner = ctx.runner
        eng, h = runner.engine, runner.handle
        if not eng.recompute:
            out, grad_inputs = ctx.inner
            del ctx.inner
            params = list(h.meta.params)
            grads = torch.autograd.grad(outputs=out, inputs=grad_inputs + params, grad_outputs=grad_output,
                                        allow_unused=True)
            del out
            nbytes = h.meta.total_numel * _elem_size(h.param_dtype)
            eng._record_backward_allgather_ms(0.0, num_bytes=0)
            eng._record_backward_reduce_scatter_ms(h.accumulate_grad_shard(grads[len(grad_inputs):]),
                                                   num_bytes=nbytes)
            it = iter(grads[: len(grad_inputs)])
            return (None, None, *[next(it) if (is_t and rg) else None
                                  for is_t, rg in zip(ctx.arg_is_tensor, ctx.arg_requires_grad)])
        saved = iter(ctx.saved_tensors)
        rebuilt: List[object] = []
        grad_inputs: List[torch.Tensor] = []
        devices: List[int] = []
        if runner.device.type == "cuda" and torch.cuda.is_available():
            devices.append(runner.device.index if runner.device.index is not None else torch.cuda.current_device())
        with torch.random.fork_rng(devices=devices, enabled=True):
            torch.set_rng_state(ctx.cpu_rng_state)
            if ctx.cuda_rng_state is not None:
                torch.cuda.set_rng_state(ctx.cuda_rng_state, device=devices[0])
            nbytes = h.meta.total_numel * _elem_size(h.param_dtype)
            eng._record_memory_event(f"measured_step_stage3_{runner.name}_pre_allgather_backward")
            eng._record_backward_allgather_ms(h.materialize("backward"), num_bytes=nbytes)
            eng._record_memory_event(f"measured_step_stage3_{runner.name}_post_allgather_backward")
            with torch.enable_grad():
                for is_t, rg, nt in zip(ctx.arg_is_tensor, ctx.arg_requires_grad, ctx.non_tensor_args):
                    if not is_t:
                        rebuilt.append(nt)
                        continue
                    t = next(saved).detach()
                    if rg:
                        t.requires_grad_(True)
                        grad_inputs.append(t)
                    rebuilt.append(t)
                use_ac = ctx.autocast_enabled and runner.device.type in {"cpu", "cuda"}
                # only autograd.grad reads `out` below (its graph, not its
                # value): modules may skip forming the value (output_unused)
                with torch.autocast(device_type=runner.device.type, dtype=ctx.autocast_dtype, enabled=use_ac), \
                        output_unused():
                    out = runner.module(*rebuilt)
                params = list(h.meta.params)
                grads = torch.autograd.grad(outputs=out, inputs=grad_inputs + params, grad_outputs=grad_output,
                                            allow_unused=True)
            input_grads = grads[: len(grad_inputs)]
            param_grads = grads[len(grad_inputs) :]
            eng._record_memory_event(f"measured_step_stage3_{runner.name}_after_layer_backward")
            eng._record_backward_reduce_scatter_ms(h.accumulate_grad_shard(param_grads), num_bytes=nbytes)
            h.reshard()
            eng._record_memory_event(f"measured_step_stage3_{runner.name}_after_reduce_scatter_discard")
        it = iter(input_grads)
        out_grads: List[Optional[torch.Tensor]] = []
        for is_t, rg in zip(ctx.arg_is_tensor, ctx.arg_requires_grad):
            out_grads.append(next(it) if (is_t and rg) else None)
        return (None, None, *out_grads)


@dataclass
class _Stage3ModuleRunner:
    name: str
    module: nn.Module
    handle: _Stage3ParamHandle
    engine: "ZeROStage3Optimizer"

    def __post_init__(self) -> None:
        self.device = self.handle.meta.device
        # a grad-requiring input keeps every module call on the autograd graph
        self.autograd_token = torch.empty(1, dtype=torch.float32, device=self.device).requires_grad_(True)

    def call(self, *args):
        return _ShardedModuleFunction.apply(self, self.autograd_token, *args)


@dataclass
class ZeROStage3Optimizer:
    """Stage 3 with per-module parameter materialization and backward recomputation."""

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
    recompute: bool = True

    def __post_init__(self) -> None:
        self.rank, self.world_size = get_rank_world_size()
        _require_single_rank(self.world_size)
        if self.collectives is None:
            self.collectives = LocalCollectives()
        self.step_count = 0
        self._summon_depth = 0
        self._reset_comm_stats()
        self.handles: Dict[str, _Stage3ParamHandle] = {}
        self._handle_order: List[_Stage3ParamHandle] = []
        self._module_runners: Dict[str, _Stage3ModuleRunner] = {}
        self._bucket: Optional[torch.Tensor] = None
        self._build_module_runners()
        self._bind_flat_state()
        self._param_flat: Optional[torch.Tensor] = None
        if not self.recompute:
            self._pin_params()
        self._fused = FusedStep(self._device)
        self.model._zero3_executor = self
        self._reshard_all_params()

    def _pin_params(self) -> None:
        """recompute=False: every parameter becomes a view of one bf16 buffer in
        handle order (the master's order), filled from the master once and
        afterwards rewritten by the fused AdamW."""
        if not self.collectives.is_identity:
            raise ValueError("recompute=False keeps parameters materialised and needs world_size 1")
        dtypes = {h.param_dtype for h in self._handle_order}
        if len(dtypes) != 1:
            raise ValueError(f"recompute=False needs one parameter dtype across modules, got {sorted(map(str, dtypes))}")
        for h in self._handle_order:
            if h.shard.shard_numel != h.meta.total_numel:
                raise ValueError("recompute=False needs unpadded shards (world_size 1)")
        self._param_flat = ops.cast(self._master_all, dtypes.pop())
        off = 0
        for h in self._handle_order:
            n = h.meta.total_numel
            views_into(h.meta, self._param_flat[off : off + n])
            h.materialized = True
            h.pinned = True
            off += n

    def _reset_comm_stats(self) -> None:
        self._forward_comm_ms = 0.0
        self._backward_comm_ms = 0.0
        self._forward_allgather_ms = 0.0
        self._backward_allgather_ms = 0.0
        self._backward_reduce_scatter_ms = 0.0
        self._forward_allgather_calls = 0
        self._backward_allgather_calls = 0
        self._backward_reduce_scatter_calls = 0
        self._forward_allgather_bytes = 0
        self._backward_allgather_bytes = 0
        self._backward_reduce_scatter_bytes = 0

    def _build_module_runners(self) -> None:
        modules = dict(module_specs(self.model))
        for hname, module_names, params in plan_handles(self.model):
            meta = build_flat_param_metadata_from_params(params)
            shard = compute_shard_spec(meta.total_numel, rank=self.rank, world_size=self.world_size)
            handle = _Stage3ParamHandle(name=hname, meta=meta, shard=shard, collectives=self.collectives, engine=self,
                                        module_names=list(module_names))
            self.handles[hname] = handle
            self._handle_order.append(handle)
            for name in module_names:
                self._module_runners[name] = _Stage3ModuleRunner(name=name, module=modules[name], handle=handle,
                                                                 engine=self)

    def _bind_flat_state(self) -> None:
        """One flat fp32 buffer each for master, moments and gradient shard;
        handle tensors are consecutive views (handle order)."""
        self._device = self._handle_order[0].meta.device
        total = sum(h.shard.shard_numel for h in self._handle_order)
        self._total_numel = total
        self._master_all = torch.empty(total, dtype=torch.float32, device=self._device)
        self._exp_avg_all = ops.zeros((total,), torch.float32, self._device)
        self._exp_avg_sq_all = ops.zeros((total,), torch.float32, self._device)
        self._grad_all = ops.zeros((total,), torch.float32, self._device)
        off = 0
        for h in self._handle_order:
            n = h.shard.shard_numel
            full = flatten_params_fp32(h.meta)
            ops.cast(full[h.shard.shard_start : h.shard.shard_end], torch.float32, out=self._master_all[off : off + n])
            h.local_master_param_shard = self._master_all[off : off + n]
            h.exp_avg = self._exp_avg_all[off : off + n]
            h.exp_avg_sq = self._exp_avg_sq_all[off : off + n]
            h.grad_shard = self._grad_all[off : off + n]
            off += n

    def _bucket_buffer(self, n: int, dtype: torch.dtype) -> torch.Tensor:
        if self._bucket is None or self._bucket.numel() < n or self._bucket.dtype != dtype:
            size = max(n, min(self.grad_bucket_numel, max(h.meta.total_numel for h in self._handle_order)))
            self._bucket = torch.empty(size, dtype=dtype, device=self._device)
        return self._bucket[:n]

    def call_module(self, module_name: str, module: nn.Module, *args):
        runner = self._module_runners.get(module_name)
        if runner is None or runner.module is not module:
            return module(*args)
        return runner.call(*args)

    def _record_forward_comm_ms(self, value: float) -> None:
        self._record_forward_allgather_ms(value=value)

    def _record_backward_comm_ms(self, value: float) -> None:
        del value  # backward time is tracked per phase below

    def _record_forward_allgather_ms(self, value: float, num_bytes: int = 0) -> None:
        self._forward_allgather_ms += value
        self._forward_allgather_calls += 1
        self._forward_allgather_bytes += int(num_bytes)
        self._forward_comm_ms += value

    def _record_backward_allgather_ms(self, value: float, num_bytes: int = 0) -> None:
        self._backward_allgather_ms += value
        self._backward_allgather_calls += 1
        self._backward_allgather_bytes += int(num_bytes)
        self._backward_comm_ms += value

    def _record_backward_reduce_scatter_ms(self, value: float, num_bytes: int = 0) -> None:
        self._backward_reduce_scatter_ms += value
        self._backward_reduce_scatter_calls += 1
        self._backward_reduce_scatter_bytes += int(num_bytes)
        self._backward_comm_ms += value

    def _record_memory_event(self, label: str) -> None:
        if self.memory_tracker is None or not self.memory_trace_active:
            return
        self.memory_tracker.record(label)
        if self.memory_state_timeline is not None:
            self.memory_state_timeline.append({"label": label, **self.live_model_state_breakdown_mb()})

    def _reshard_all_params(self) -> None:
        if self._summon_depth > 0:
            return
        for h in self._handle_order:
            h.reshard()

    @contextmanager
    def summon_full_params(self) -> Iterator[nn.Module]:
        self._summon_depth += 1
        if self._summon_depth == 1:
            for h in self._handle_order:
                h.materialize("summon")
        try:
            yield self.model
        finally:
            self._summon_depth -= 1
            if self._summon_depth == 0:
                self._reshard_all_params()

    def backward(self, loss: torch.Tensor) -> None:
        backward_from_loss(loss)

    def prepare_forward(self) -> Dict[str, float]:
        self._reshard_all_params()
        return {"prepare_comm_ms": 0.0}

    def zero_grad(self) -> None:
        self._reset_comm_stats()
        # zeroing is deferred: each handle's first gradient of the step is
        # written over its shard, and shards that receive none are zeroed
        # before the norm (_finish_grads)
        for h in self._handle_order:
            h.grad_fresh = True
        for p in self.model.parameters():
            p.grad = None
        self._reshard_all_params()

    def step_with_stats(self, max_grad_norm: float = 0.0) -> Dict[str, float]:
        t0 = time.perf_counter()
        self._finish_grads()
        self._fused.grad_norm_and_scale([self._grad_all], max_grad_norm)
        self.step_count += 1
        t_opt0 = time.perf_counter()
        self._fused.adamw(self._master_all, self._exp_avg_all, self._exp_avg_sq_all, self._grad_all, lr=self.lr,
                          betas=self.betas, eps=self.eps, weight_decay=self.weight_decay, step=self.step_count,
                          max_grad_norm=max_grad_norm, p_out=self._param_flat)
        optim_ms = (time.perf_counter() - t_opt0) * 1000.0
        self._reshard_all_params()
        grad_norm = self._fused.read_norm()
        return {
            "grad_norm": grad_norm,
            "comm_ms": self._forward_comm_ms + self._backward_comm_ms,
            "communication_forward_allgather_ms": self._forward_allgather_ms,
            "communication_forward_allgather_calls": float(self._forward_allgather_calls),
            "communication_forward_allgather_bytes": float(self._forward_allgather_bytes),
            "communication_backward_allgather_ms": self._backward_allgather_ms,
            "communication_backward_allgather_calls": float(self._backward_allgather_calls),
            "communication_backward_allgather_bytes": float(self._backward_allgather_bytes),
            "communication_backward_reduce_scatter_ms": self._backward_reduce_scatter_ms,
            "communication_backward_reduce_scatter_calls": float(self._backward_reduce_scatter_calls),
            "communication_backward_reduce_scatter_bytes": float(self._backward_reduce_scatter_bytes),
            "optim_ms": optim_ms,
            "total_ms": (time.perf_counter() - t0) * 1000.0,
        }

    def _finish_grads(self) -> None:
        for h in self._handle_order:
            if h.grad_fresh:
                h.reset_grad()

    def step(self, max_grad_norm: float = 0.0) -> float:
        return float(self.step_with_stats(max_grad_norm=max_grad_norm)["grad_norm"])

    def _logical_bytes(self) -> Tuple[int, int]:
        pb = gb = 0
        for h in self._handle_order:
            pb += h.shard.shard_numel * _elem_size(h.param_dtype)
            gb += h.shard.shard_numel * _elem_size(h.param_dtype)
        return pb, gb

    def _optimizer_tensors(self) -> List[torch.Tensor]:
        out: List[torch.Tensor] = []
        for h in self._handle_order:
            out.extend([h.local_master_param_shard, h.exp_avg, h.exp_avg_sq])
        return out

    def memory_state_breakdown_mb(self) -> Dict[str, float]:
        pb, gb = self._logical_bytes()
        params_mb, grads_mb = bytes_to_mb(pb), bytes_to_mb(gb)
        optimizer_mb = bytes_to_mb(tensors_num_bytes(self._optimizer_tensors()))
        return {"params_mb": params_mb, "grads_mb": grads_mb, "optimizer_mb": optimizer_mb,
                "total_mb": params_mb + grads_mb + optimizer_mb}

    def live_model_state_breakdown_mb(self) -> Dict[str, float]:
        pb, gb = self._logical_bytes()
        params_mb = bytes_to_mb(pb + params_num_bytes(self.model.parameters()))
        grads_mb = bytes_to_mb(gb + grads_num_bytes(self.model.parameters()))
        optimizer_mb = bytes_to_mb(tensors_num_bytes(self._optimizer_tensors()))
        return {"params_mb": params_mb, "grads_mb": grads_mb, "optimizer_mb": optimizer_mb,
                "total_mb": params_mb + grads_mb + optimizer_mb}

    def state_dict(self) -> Dict[str, object]:
        return {
            "step_count": self.step_count,
            "rank": self.rank,
            "world_size": self.world_size,
            "handles": {
                h.name: {
                    "module_names": list(h.module_names),
                    "shard_start": h.shard.shard_start,
                    "shard_end": h.shard.shard_end,
                    "local_master_param_shard": h.local_master_param_shard.detach().cpu(),
                    "exp_avg": h.exp_avg.detach().cpu(),
                    "exp_avg_sq": h.exp_avg_sq.detach().cpu(),
                }
                for h in self._handle_order
            },
            "hparams": {"lr": self.lr, "betas": self.betas, "eps": self.eps, "weight_decay": self.weight_decay},
        }

    def load_state_dict(self, state: Dict[str, object]) -> None:
        self.step_count = int(state["step_count"])
        saved_handles = state["handles"]
        for h in self._handle_order:
            if h.name not in saved_handles:
                raise KeyError(f"missing stage3 handle state for '{h.name}'")
            s = saved_handles[h.name]
            for dst, key in ((h.local_master_param_shard, "local_master_param_shard"), (h.exp_avg, "exp_avg"),
                             (h.exp_avg_sq, "exp_avg_sq")):
                src = s[key]
                if src.numel() != dst.numel():
                    raise ValueError(f"stage3 handle '{h.name}' {key}: {src.numel()} != {dst.numel()} elements")
                dst.copy_(src.to(dtype=torch.float32).view(-1))
            h.reset_grad()
        if self._param_flat is not None:
            ops.cast(self._master_all, self._param_flat.dtype, out=self._param_flat)
        self._reshard_all_params()
