"""ZeRO stage 0-3 trainer (reference: train_zero.py), single GPU.

Flags, defaults, stdout step lines (the experiment harness's contract), the
--profile-json payload and checkpoints follow the reference.  Additions: the
`plumbing`/`125m`/`1b`/`7b` presets, the `synthetic-uniform` data mode,
--grad-bucket-numel (the gradient bucket size of stages 0, 1 and 3) and
--zero3-recompute off (stage 3 keeps each module's forward graph instead of
recomputing it in backward; same gradients, one forward per step).  The
engines run at world_size 1 with LocalCollectives; launching with
WORLD_SIZE > 1 is rejected.
"""
from __future__ import annotations

import argparse
import json
import os
import time
from contextlib import nullcontext
from dataclasses import asdict
from pathlib import Path
from typing import Dict, Iterator, Tuple

import torch
import torch.distributed as dist

from collectives import LocalCollectives, SendRecvCollectives, TorchCollectives, TracingCollectives
from model import MODEL_SIZES, LlamaForCausalLM, build_config, estimate_num_parameters, human_readable_count
from profiler import (
    FlopTracker,
    MemoryTracker,
    TimerRegistry,
    estimate_transformer_train_flops,
    flops_to_tflops_per_second,
    overlap_efficiency,
)
from train import DATA_MODES, batch_from_chunk, make_data_loader, set_seed
from zero import ZeROStage0DDP, ZeROStage1Optimizer, ZeROStage2Optimizer, ZeROStage3Optimizer
from zero.common import GRAD_BUCKET_NUMEL


def log_event(rank: int, message: str, *, force: bool = True) -> None:
    if force:
        print(f"[{time.strftime('%H:%M:%S')}][rank {rank}] {message}", flush=True)


def format_device_memory(device: torch.device) -> str:
    if device.type != "cuda" or not torch.cuda.is_available():
        return "host-only"
    mb = 1024.0 * 1024.0
    return (
        f"cuda_allocated_mb={torch.cuda.memory_allocated(device) / mb:.1f} "
        f"cuda_reserved_mb={torch.cuda.memory_reserved(device) / mb:.1f} "
        f"cuda_max_allocated_mb={torch.cuda.max_memory_allocated(device) / mb:.1f}"
    )


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="ZeRO stages 0-3 training on one MI355X")
    p.add_argument("--zero-stage", type=int, default=0, choices=[0, 1, 2, 3])
    p.add_argument("--collective-impl", type=str, default="torch", choices=["ring", "torch"])
    p.add_argument("--model-size", type=str, default="tiny", choices=MODEL_SIZES)
    p.add_argument("--seq-len", type=int, default=512)
    p.add_argument("--batch-size", type=int, default=2)
    p.add_argument("--grad-accum-steps", type=int, default=1)
    p.add_argument("--max-steps", type=int, default=200)
    p.add_argument("--learning-rate", type=float, default=3e-4)
    p.add_argument("--weight-decay", type=float, default=0.1)
    p.add_argument("--beta1", type=float, default=0.9)
    p.add_argument("--beta2", type=float, default=0.95)
    p.add_argument("--eps", type=float, default=1e-8)
    p.add_argument("--max-grad-norm", type=float, default=0.0)
    p.add_argument("--stage2-grad-bucket-mb", type=float, default=64.0,
                   help="Compatibility knob only; stage 2 uses one contiguous gradient buffer per backward pass.")
    p.add_argument("--grad-bucket-numel", type=int, default=GRAD_BUCKET_NUMEL,
                   help="Elements per gradient bucket of the stage 0/1/3 flatten (reduce-scatter/all-reduce unit).")
    p.add_argument("--zero3-recompute", type=str, default="on", choices=["on", "off"],
                   help="Stage 3: recompute each module in backward (reference behaviour) or keep its forward graph.")
    p.add_argument("--dtype", type=str, default="float32", choices=["float32", "bfloat16"])
    p.add_argument("--seed", type=int, default=1337)
    p.add_argument("--loss-chunk-size", type=int, default=128,
                   help="Sequence chunk size for LM-head projection during training loss; 0 disables chunking.")
    p.add_argument("--activation-checkpointing", dest="activation_checkpointing", action="store_true")
    p.add_argument("--no-activation-checkpointing", dest="activation_checkpointing", action="store_false")
    p.add_argument("--data-mode", type=str, default="synthetic", choices=DATA_MODES)
    p.add_argument("--tokenizer-name", type=str, default="meta-llama/Llama-3.1-8B")
    p.add_argument("--fineweb-subset", type=str, default="sample-10BT")
    p.add_argument("--fineweb-split", type=str, default="train")
    p.add_argument("--shuffle-buffer", type=int, default=10_000)
    p.add_argument("--synthetic-vocab-size", type=int, default=8_192)
    p.add_argument("--allow-synthetic-fallback", action="store_true")
    p.add_argument("--log-interval", type=int, default=10)
    p.add_argument("--checkpoint-interval", type=int, default=100)
    p.add_argument("--save-dir", type=str, default="checkpoints")
    p.add_argument("--profile-json", type=str, default="")
    p.add_argument("--profile-memory-interval", type=int, default=0)
    p.add_argument("--profile-rank0-only", action="store_true")
    p.add_argument("--profile-collectives", action="store_true")
    p.add_argument("--measure-memory-step", action="store_true")
    p.add_argument("--memory-warmup-steps", type=int, default=0)
    p.add_argument("--tflops-mode", type=str, default="estimate", choices=["estimate", "profile", "off"])
    p.add_argument("--verbose", action="store_true")
    p.add_argument("--verbose-memory", action="store_true")
    p.set_defaults(activation_checkpointing=False)
    return p


def parse_args(argv=None) -> argparse.Namespace:
    return build_parser().parse_args(argv)


def init_distributed() -> Tuple[int, int, torch.device]:
    if "RANK" in os.environ and "WORLD_SIZE" in os.environ and int(os.environ["WORLD_SIZE"]) > 1:
        raise RuntimeError("this build runs the ZeRO engines on one GPU; launch without WORLD_SIZE > 1")
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required: the model and engines run on the gfx950 HIP kernels")
    local_rank = int(os.environ.get("LOCAL_RANK", 0))
    torch.cuda.set_device(local_rank)
    return 0, 1, torch.device("cuda", local_rank)


def autocast_context(device: torch.device, dtype_name: str):
    if device.type != "cuda" or dtype_name == "float32":
        return nullcontext()
    return torch.autocast(device_type="cuda", dtype=torch.bfloat16)


def model_param_dtype(device: torch.device, dtype_name: str) -> torch.dtype:
    if device.type != "cuda" or dtype_name == "float32":
        return torch.float32
    return torch.bfloat16


def configure_runtime(device: torch.device) -> None:
    if device.type != "cuda" or not torch.cuda.is_available():
        return
    torch.backends.cuda.matmul.allow_tf32 = True
    torch.set_float32_matmul_precision("high")


def broadcast_model(model: LlamaForCausalLM) -> None:
    if dist.is_available() and dist.is_initialized():
        for p in model.parameters():
            dist.broadcast(p.data, src=0)


def pick_collectives(world_size: int, impl: str):
    if world_size == 1:
        return LocalCollectives()
    return SendRecvCollectives() if impl == "ring" else TorchCollectives()


def aggregate_collective_trace(records: list) -> list:
    by_key: Dict[Tuple[str, str], Dict[str, object]] = {}
    for rec in records:
        key = (str(rec.get("op", "")), str(rec.get("label", "")))
        e = by_key.setdefault(key, {"op": key[0], "label": key[1], "calls": 0, "elapsed_ms": 0.0,
                                    "input_bytes": 0.0, "output_bytes": 0.0})
        e["calls"] = int(e["calls"]) + 1
        e["elapsed_ms"] = float(e["elapsed_ms"]) + float(rec.get("elapsed_ms", 0.0))
        e["input_bytes"] = float(e["input_bytes"]) + float(rec.get("input_bytes", 0.0))
        e["output_bytes"] = float(e["output_bytes"]) + float(rec.get("output_bytes", 0.0))
    return sorted(by_key.values(), key=lambda it: (-float(it["elapsed_ms"]), str(it["label"]), str(it["op"])))


def build_engine(args: argparse.Namespace, model: LlamaForCausalLM, collectives):
    kw = {"model": model, "lr": args.learning_rate, "betas": (args.beta1, args.beta2), "eps": args.eps,
          "weight_decay": args.weight_decay, "collectives": collectives}
    bucket = getattr(args, "grad_bucket_numel", GRAD_BUCKET_NUMEL)
    if args.zero_stage == 0:
        return ZeROStage0DDP(**kw, grad_bucket_numel=bucket)
    if args.zero_stage == 1:
        return ZeROStage1Optimizer(**kw, grad_bucket_numel=bucket)
    if args.zero_stage == 2:
        numel = max(1, int((args.stage2_grad_bucket_mb * 1024.0 * 1024.0) / 4.0))
        return ZeROStage2Optimizer(**kw, grad_bucket_numel=numel)
    if args.zero_stage == 3:
        return ZeROStage3Optimizer(**kw, grad_bucket_numel=bucket,
                                   recompute=getattr(args, "zero3_recompute", "on") == "on")
    raise ValueError(f"Unsupported stage: {args.zero_stage}")


def global_mean_scalar(value: float, device: torch.device, world_size: int) -> float:
    return float(value) / world_size


def save_checkpoint(save_dir: str, step: int, rank: int, model: LlamaForCausalLM, engine, args: argparse.Namespace,
                    extra: Dict[str, object]) -> str:
    os.makedirs(save_dir, exist_ok=True)
    path = os.path.join(save_dir, f"zero_stage{args.zero_stage}_step{step:06d}_rank{rank:03d}.pt")
    ctx = engine.summon_full_params() if hasattr(engine, "summon_full_params") else nullcontext()
    with ctx:
        msd = model.state_dict()
    torch.save({"step": step, "rank": rank, "model_state_dict": msd, "engine_state_dict": engine.state_dict(),
                "train_args": vars(args), "extra": extra}, path)
    return path


def train(args: argparse.Namespace) -> Dict[str, object]:
    rank, world_size, device = init_distributed()
    verbose = bool(args.verbose)
    configure_runtime(device)
    set_seed(args.seed)
    base_vocab = args.synthetic_vocab_size
    cfg = build_config(size=args.model_size, vocab_size=base_vocab, max_seq_len=args.seq_len)
    try:
        loader, detected_vocab, metadata = make_data_loader(args, vocab_size_for_model=base_vocab, rank=rank,
                                                            world_size=world_size)
    except Exception as exc:
        if not args.allow_synthetic_fallback:
            raise
        print(f"[warn] data init failed ({exc}); falling back to synthetic")
        args.data_mode = "synthetic"
        loader, detected_vocab, metadata = make_data_loader(args, vocab_size_for_model=base_vocab, rank=rank,
                                                            world_size=world_size)
    if detected_vocab != cfg.vocab_size:
        cfg = cfg.with_vocab_size(detected_vocab)

    model = LlamaForCausalLM(cfg).to(device=device, dtype=model_param_dtype(device, args.dtype))
    model.set_loss_chunk_size(args.loss_chunk_size)
    model.set_activation_checkpointing(args.activation_checkpointing)
    log_event(rank, f"model moved to device {device} {format_device_memory(device)}", force=verbose or args.verbose_memory)
    broadcast_model(model)
    collectives = pick_collectives(world_size=world_size, impl=args.collective_impl)
    if args.profile_collectives:
        collectives = TracingCollectives(collectives)
    engine = build_engine(args, model, collectives)
    n_params = estimate_num_parameters(cfg)
    print(
        f"[init] stage={args.zero_stage} impl={args.collective_impl} world_size={world_size} model={cfg.name} "
        f"params={human_readable_count(n_params)} ({n_params:,}) vocab={cfg.vocab_size:,} seq_len={cfg.max_seq_len} "
        f"device={device} dtype={args.dtype}",
        flush=True,
    )
    print(f"[init] data_mode={args.data_mode} metadata={json.dumps(metadata)}", flush=True)

    tokens_per_step = args.batch_size * args.grad_accum_steps * args.seq_len * world_size
    data_iter: Iterator[torch.Tensor] = iter(loader)
    timers = TimerRegistry(device=device)
    flop_tracker = FlopTracker(device=device) if args.tflops_mode == "profile" else None
    memory = MemoryTracker(device=device)
    profile_on = bool(args.profile_json)
    record_mem = args.profile_memory_interval > 0 or args.measure_memory_step
    measured_idx = args.memory_warmup_steps + 1 if args.measure_memory_step else None
    if args.measure_memory_step and args.max_steps < measured_idx:
        raise ValueError(f"max_steps={args.max_steps} is too small for memory warmup + measured step; need at least {measured_idx}")
    measured_memory = None
    timeline: list = []
    peak_obs = None
    peak_max = -1.0
    live_breakdown = getattr(engine, "live_model_state_breakdown_mb", None) or getattr(engine, "memory_state_breakdown_mb", None)
    debug_components = getattr(engine, "debug_memory_components_mb", None)
    engine.memory_tracker = memory
    engine.memory_trace_active = False
    engine.memory_state_timeline = timeline
    if record_mem and profile_on and not args.measure_memory_step:
        memory.record("start")

    def snap(label: str, capture_peak: bool) -> None:
        nonlocal peak_obs, peak_max
        s = memory.record(label)
        if live_breakdown is not None and capture_peak:
            timeline.append({"label": label, **live_breakdown()})
        if not capture_peak or s.cuda_max_allocated_mb <= peak_max + 1e-6:
            return
        peak_max = s.cuda_max_allocated_mb
        peak_obs = {"label": label, "timestamp_s": s.timestamp_s, "allocated_mb": s.cuda_allocated_mb,
                    "reserved_mb": s.cuda_reserved_mb, "max_allocated_mb": s.cuda_max_allocated_mb,
                    "max_reserved_mb": s.cuda_max_reserved_mb}
        if live_breakdown is not None:
            peak_obs["live_state_breakdown_mb"] = live_breakdown()
        if callable(debug_components):
            peak_obs["debug_memory_components_mb"] = debug_components()

    step_flops = None
    if args.tflops_mode == "estimate":
        step_flops = estimate_transformer_train_flops(cfg=cfg, batch_size=args.batch_size, seq_len=args.seq_len,
                                                      grad_accum_steps=args.grad_accum_steps, world_size=world_size,
                                                      stage=args.zero_stage)
    recent: list = []
    step_profiles: list = []
    history: list = []
    t_start = time.perf_counter()
    for step in range(1, args.max_steps + 1):
        sample = args.profile_memory_interval > 0 and (step == 1 or step == args.max_steps or step % args.profile_memory_interval == 0)
        measured = measured_idx is not None and step == measured_idx
        if args.profile_collectives:
            collectives.consume_trace()
        it_timer = timers.timer("iteration")
        it_timer.start()
        model.train()
        engine.zero_grad()
        if measured:
            memory.reset_peak_stats()
            engine.memory_trace_active = bool(record_mem and profile_on)
            if record_mem and profile_on:
                snap(f"measured_step_{step}_start", True)
        elif sample and record_mem and profile_on:
            snap(f"step_{step}_start", False)
        prep = engine.prepare_forward()
        prepare_comm_ms = float(prep.get("prepare_comm_ms", 0.0))
        if measured and record_mem and profile_on:
            snap(f"measured_step_{step}_post_prepare", True)
        fb_timer = timers.timer("forward_backward")
        fb_timer.start()

        def run_microbatches() -> list:
            nonlocal data_iter
            losses = []
            for micro in range(args.grad_accum_steps):
                try:
                    chunk = next(data_iter)
                except StopIteration:
                    data_iter = iter(loader)
                    chunk = next(data_iter)
                batch = batch_from_chunk(chunk)
                input_ids = batch.input_ids.to(device, non_blocking=True)
                labels = batch.labels.to(device, non_blocking=True)
                with autocast_context(device, args.dtype):
                    out = model(input_ids=input_ids, labels=labels, return_logits=False)
                    loss = out.loss
                    if loss is None:
                        raise RuntimeError("Model did not return loss even though labels were provided")
                    scaled = loss / args.grad_accum_steps
                if measured and record_mem and profile_on:
                    snap(f"measured_step_{step}_micro_{micro + 1}_after_forward", True)
                losses.append(float(loss.detach().float().item()))
                engine.backward(scaled)
                if measured and record_mem and profile_on:
                    snap(f"measured_step_{step}_micro_{micro + 1}_after_backward", True)
                elif sample and record_mem and profile_on:
                    snap(f"step_{step}_micro_{micro + 1}_post_backward", False)
            return losses

        if flop_tracker is not None and step_flops is None:
            micro_losses, prof_flops = flop_tracker.measure(label=f"step_{step}", fn=run_microbatches)
            if prof_flops is not None:
                step_flops = prof_flops * world_size
        else:
            micro_losses = run_microbatches()
        fb_ms = fb_timer.stop()
        if measured and record_mem and profile_on:
            snap(f"measured_step_{step}_post_backward", True)
        elif sample and record_mem and profile_on:
            snap(f"step_{step}_post_backward", False)

        opt_timer = timers.timer("optimizer_step")
        opt_timer.start()
        stats = engine.step_with_stats(max_grad_norm=args.max_grad_norm)
        opt_timer.stop()
        grad_norm = float(stats["grad_norm"])
        comm_ms = float(stats["comm_ms"]) + prepare_comm_ms
        if measured and record_mem and profile_on:
            snap(f"measured_step_{step}_post_optimizer", True)
        elif sample and record_mem and profile_on:
            snap(f"step_{step}_post_optimizer", False)

        step_loss = global_mean_scalar(sum(micro_losses) / len(micro_losses), device, world_size)
        recent.append(step_loss)
        if len(recent) > 100:
            recent.pop(0)
        iter_ms = it_timer.stop()
        tps = tokens_per_step / max(iter_ms / 1000.0, 1e-8)
        tflops = flops_to_tflops_per_second(step_flops, iter_ms / 1000.0) if step_flops is not None else None
        overlap = overlap_efficiency(step_ms=iter_ms, compute_ms=max(iter_ms - comm_ms, 0.0), communication_ms=comm_ms)
        history.append({"step": step, "loss": step_loss, "grad_norm": grad_norm, "iteration_ms": iter_ms,
                        "tokens_per_second": tps})
        if step % args.log_interval == 0 or step == 1 or step == args.max_steps:
            avg = sum(recent) / len(recent)
            print(
                f"[step {step:05d}] loss={step_loss:.4f} avg100={avg:.4f} tokens/s={tps:,.0f} grad_norm={grad_norm:.3f} "
                f"fb_ms={fb_ms:.2f} comm_ms={comm_ms:.2f} opt_ms={stats['optim_ms']:.2f}"
                + (f" tflops={tflops:.3f}" if tflops is not None else ""),
                flush=True,
            )
        trace, trace_summary = [], []
        if args.profile_collectives:
            trace = collectives.consume_trace()
            trace_summary = aggregate_collective_trace(trace)
        if profile_on:
            prof = {"step": step, "loss": step_loss, "tokens_per_second": tps, "tflops_per_second": tflops,
                    "grad_norm": grad_norm, "forward_backward_ms": fb_ms, "communication_ms": comm_ms,
                    "optimizer_ms": float(stats["optim_ms"]), "iteration_ms": iter_ms}
            for key in ("communication_backward_reduce_scatter_ms", "communication_backward_reduce_scatter_calls",
                        "communication_backward_reduce_scatter_bytes", "communication_post_allgather_ms",
                        "communication_post_allgather_calls", "communication_post_allgather_bytes",
                        "communication_forward_allgather_ms", "communication_forward_allgather_calls",
                        "communication_forward_allgather_bytes", "communication_backward_allgather_ms",
                        "communication_backward_allgather_calls", "communication_backward_allgather_bytes"):
                prof[key] = float(stats.get(key, 0.0))
            prof.update({"collective_trace": trace, "collective_trace_summary": trace_summary, "overlap_ratio": overlap})
            step_profiles.append(prof)
        if measured and record_mem and profile_on:
            snap(f"measured_step_{step}_end", True)
            peaks = memory.peak_stats_mb()
            measured_memory = {"step": step, "warmup_steps": args.memory_warmup_steps,
                               "peak_allocated_mb": float(peaks["peak_allocated_mb"]),
                               "peak_reserved_mb": float(peaks["peak_reserved_mb"])}
            if peak_obs is not None:
                measured_memory["peak_observation"] = peak_obs
            engine.memory_trace_active = False
        elif sample and record_mem and profile_on:
            snap(f"step_{step}_end", False)
        if args.checkpoint_interval > 0 and (step % args.checkpoint_interval == 0 or step == args.max_steps):
            path = save_checkpoint(args.save_dir, step, rank, model, engine, args,
                                   {"model_config": cfg.to_dict(), "step_loss": step_loss})
            print(f"[checkpoint] wrote {path}", flush=True)

    print(f"[done] trained {args.max_steps} steps in {time.perf_counter() - t_start:.1f}s", flush=True)
    if profile_on:
        timer_payload = {n: asdict(s) for n, s in timers.summarize().items()}
        overlap_summary = None
        if step_profiles:
            vals = [float(s["overlap_ratio"]) for s in step_profiles]
            overlap_summary = {"mean": sum(vals) / len(vals), "min": min(vals), "max": max(vals)}
        coll_summary = None
        if step_profiles and args.profile_collectives:
            coll_summary = aggregate_collective_trace([r for s in step_profiles for r in s.get("collective_trace", [])])
        payload = {
            "rank": rank, "world_size": world_size, "stage": args.zero_stage, "collective_impl": args.collective_impl,
            "args": vars(args), "model_config": cfg.to_dict(),
            "optimizer_config": {"lr": args.learning_rate, "betas": [args.beta1, args.beta2], "eps": args.eps,
                                 "weight_decay": args.weight_decay, "max_grad_norm": args.max_grad_norm},
            "global_batch_size": args.batch_size * args.grad_accum_steps * world_size,
            "microbatch_size_per_gpu": args.batch_size, "overlap_enabled": False, "timers": timer_payload,
            "memory": memory.as_dicts() if record_mem else [],
            "flops": {"measurements": flop_tracker.as_dicts() if flop_tracker is not None else [],
                      "profiled_step_flops": step_flops, "tflops_mode": args.tflops_mode},
            "steps": step_profiles, "collective_trace_summary": coll_summary,
            "state_memory_breakdown_mb": engine.memory_state_breakdown_mb(), "overlap_summary": overlap_summary,
            "measured_step_memory": measured_memory, "measured_step_state_timeline": timeline,
        }
        path = Path(args.profile_json)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(payload, indent=2))
        print(f"[profile] wrote {path}", flush=True)
    return {"history": history, "model": model, "engine": engine, "config": cfg}


def main() -> None:
    train(parse_args())


if __name__ == "__main__":
    main()
