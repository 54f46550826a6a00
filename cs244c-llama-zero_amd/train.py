"""Single-process LLaMA trainer (reference: train.py).

Flags, defaults, log lines and checkpoint payloads are the reference's.
Additions: the `plumbing`, `125m`, `1b`, `7b` model presets and the
`synthetic-uniform` data mode (seeded iid ids).  The model and the optimizer
(FusedAdamW, torch.optim.AdamW's update with clip_grad_norm_ folded into the
step) run on the gfx950 HIP kernels; a ROCm GPU is required.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import random
import time
from contextlib import nullcontext
from dataclasses import dataclass
from typing import Dict, Iterator, Tuple

import torch
from torch.utils.data import DataLoader

from data import (
    PackedFineWebDataset,
    RankShardIterableDataset,
    SyntheticPatternDataset,
    SyntheticUniformDataset,
    load_fineweb_stream,
    load_llama_tokenizer,
)
from lzhip.functional import GradSink, pack_parameters_
from lzhip.ops import fill_
from lzhip.optim import FusedAdamW, LossScaler
from model import MODEL_SIZES, LlamaForCausalLM, build_config, estimate_num_parameters, human_readable_count

DATA_MODES = ["fineweb", "synthetic", "synthetic-uniform"]


@dataclass
class TrainBatch:
    input_ids: torch.Tensor
    labels: torch.Tensor


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="Single-GPU LLaMA training baseline (MI355X HIP kernels)")
    p.add_argument("--model-size", type=str, default="tiny", choices=MODEL_SIZES)
    p.add_argument("--seq-len", type=int, default=512)
    p.add_argument("--batch-size", type=int, default=2)
    p.add_argument("--grad-accum-steps", type=int, default=8)
    p.add_argument("--max-steps", type=int, default=200)
    p.add_argument("--learning-rate", type=float, default=3e-4)
    p.add_argument("--weight-decay", type=float, default=0.1)
    p.add_argument("--beta1", type=float, default=0.9)
    p.add_argument("--beta2", type=float, default=0.95)
    p.add_argument("--max-grad-norm", type=float, default=1.0)
    p.add_argument("--dtype", type=str, default="bfloat16", choices=["float32", "float16", "bfloat16"])
    p.add_argument("--device", type=str, default="cuda")
    p.add_argument("--seed", type=int, default=1337)
    p.add_argument("--loss-chunk-size", type=int, default=128,
                   help="Sequence chunk size for LM-head projection during training loss; 0 disables chunking.")
    p.add_argument("--activation-checkpointing", action="store_true",
                   help="Enable per-block activation checkpointing during training.")
    p.add_argument("--data-mode", type=str, default="fineweb", choices=DATA_MODES)
    p.add_argument("--tokenizer-name", type=str, default="meta-llama/Llama-3.1-8B")
    p.add_argument("--fineweb-subset", type=str, default="sample-10BT")
    p.add_argument("--fineweb-split", type=str, default="train")
    p.add_argument("--shuffle-buffer", type=int, default=10_000)
    p.add_argument("--synthetic-vocab-size", type=int, default=8_192)
    p.add_argument("--allow-synthetic-fallback", action="store_true")
    p.add_argument("--log-interval", type=int, default=10)
    p.add_argument("--checkpoint-interval", type=int, default=100)
    p.add_argument("--save-dir", type=str, default="checkpoints")
    return p.parse_args(argv)


def set_seed(seed: int) -> None:
    random.seed(seed)
    torch.manual_seed(seed)
    torch.cuda.manual_seed_all(seed)


def choose_device(device_arg: str) -> torch.device:
    dev = torch.device(device_arg)
    if dev.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(
            f"device '{device_arg}' is not a ROCm GPU: this trainer's compute runs on the gfx950 HIP kernels"
        )
    return dev


def make_data_loader(args: argparse.Namespace, vocab_size_for_model: int, rank: int = 0,
                     world_size: int = 1) -> Tuple[DataLoader, int, Dict[str, str]]:
    meta: Dict[str, str] = {}
    if args.data_mode == "fineweb":
        bundle = load_llama_tokenizer(args.tokenizer_name)
        stream = load_fineweb_stream(subset=args.fineweb_subset, split=args.fineweb_split,
                                     shuffle_buffer=args.shuffle_buffer, seed=args.seed)
        dataset = PackedFineWebDataset(text_iterable=stream, tokenizer=bundle.tokenizer, seq_len=args.seq_len,
                                       eos_token_id=bundle.eos_token_id)
        vocab_size = bundle.vocab_size
        meta["tokenizer"] = args.tokenizer_name
        meta["dataset"] = f"HuggingFaceFW/fineweb-edu:{args.fineweb_subset}/{args.fineweb_split}"
    elif args.data_mode == "synthetic-uniform":
        vocab_size = vocab_size_for_model
        dataset = SyntheticUniformDataset(seq_len=args.seq_len, vocab_size=vocab_size, seed=args.seed)
        meta["tokenizer"] = "synthetic"
        meta["dataset"] = "synthetic_uniform"
    else:
        vocab_size = vocab_size_for_model
        dataset = SyntheticPatternDataset(seq_len=args.seq_len, vocab_size=vocab_size)
        meta["tokenizer"] = "synthetic"
        meta["dataset"] = "synthetic_pattern"
    if world_size > 1:
        dataset = RankShardIterableDataset(dataset=dataset, rank=rank, world_size=world_size)
        meta["data_sharding"] = f"rank_stride:{rank}/{world_size}"
    loader = DataLoader(dataset, batch_size=args.batch_size, num_workers=0, pin_memory=torch.cuda.is_available())
    return loader, vocab_size, meta


def batch_from_chunk(chunk: torch.Tensor) -> TrainBatch:
    # (seq_len + 1)-token chunks; labels == inputs, the shift is inside the loss
    input_ids = chunk[:, :-1].contiguous()
    return TrainBatch(input_ids=input_ids, labels=input_ids.clone())


def autocast_context(device: torch.device, dtype_name: str):
    if device.type != "cuda" or dtype_name == "float32":
        return nullcontext()
    target = torch.float16 if dtype_name == "float16" else torch.bfloat16
    return torch.autocast(device_type="cuda", dtype=target)


def model_param_dtype(device: torch.device, dtype_name: str) -> torch.dtype:
    if device.type != "cuda" or dtype_name == "float32":
        return torch.float32
    return torch.float16 if dtype_name == "float16" else torch.bfloat16


def save_checkpoint(save_dir: str, step: int, model: LlamaForCausalLM, optimizer: torch.optim.Optimizer,
                    args: argparse.Namespace, extra: Dict[str, object]) -> str:
    os.makedirs(save_dir, exist_ok=True)
    path = os.path.join(save_dir, f"step_{step:06d}.pt")
    torch.save({"step": step, "model_state_dict": model.state_dict(), "optimizer_state_dict": optimizer.state_dict(),
                "train_args": vars(args), "extra": extra}, path)
    return path


def train(args: argparse.Namespace) -> None:
    set_seed(args.seed)
    device = choose_device(args.device)

    base_vocab = args.synthetic_vocab_size
    cfg = build_config(size=args.model_size, vocab_size=base_vocab, max_seq_len=args.seq_len)
    try:
        loader, detected_vocab, metadata = make_data_loader(args, vocab_size_for_model=base_vocab)
    except Exception as exc:
        if not args.allow_synthetic_fallback:
            raise
        print(f"[warn] failed to initialize fineweb pipeline ({exc}); falling back to synthetic data")
        args.data_mode = "synthetic"
        loader, detected_vocab, metadata = make_data_loader(args, vocab_size_for_model=base_vocab)
    if detected_vocab != cfg.vocab_size:
        cfg = cfg.with_vocab_size(detected_vocab)

    model = LlamaForCausalLM(cfg).to(device=device, dtype=model_param_dtype(device, args.dtype))
    pack_parameters_(model)  # fused q/k/v and gate/up weights become views, not per-step copies
    model.set_loss_chunk_size(args.loss_chunk_size)
    model.set_activation_checkpointing(args.activation_checkpointing)
    optimizer = FusedAdamW(model.parameters(), lr=args.learning_rate, betas=(args.beta1, args.beta2),
                           weight_decay=args.weight_decay)
    # fp16: dynamic loss scaling (the reference's torch.cuda.amp.GradScaler)
    scaler = LossScaler(enabled=device.type == "cuda" and args.dtype == "float16")
    # the backward kernels write and accumulate the parameter gradients
    # themselves (no autograd accumulation kernels between micro-batches)
    grads = GradSink(model)
    # d(loss / GA) / d(loss), as the backward seed (the same value autograd
    # forms for `(loss / GA).backward()`, without its division kernels)
    seed = fill_(torch.empty((), dtype=torch.float32, device=device), 1.0 / args.grad_accum_steps)

    n_params = estimate_num_parameters(cfg)
    print(
        f"[init] model={cfg.name} params={human_readable_count(n_params)} ({n_params:,}) "
        f"vocab={cfg.vocab_size:,} seq_len={cfg.max_seq_len} device={device.type} dtype={args.dtype}"
    )
    print(f"[init] data_mode={args.data_mode} metadata={json.dumps(metadata)}")

    tokens_per_step = args.batch_size * args.grad_accum_steps * args.seq_len
    data_iter: Iterator[torch.Tensor] = iter(loader)
    recent = []
    t_start = time.perf_counter()
    for step in range(1, args.max_steps + 1):
        model.train()
        grads.begin_step()  # in place of optimizer.zero_grad(set_to_none=True)
        if scaler.is_enabled():  # d(scale * loss / GA) / d(loss)
            fill_(seed, scaler.scale_value() / args.grad_accum_steps)
        t0 = time.perf_counter()
        micro_losses = []
        for _ in range(args.grad_accum_steps):
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
            micro_losses.append(loss.detach().float().item())
            loss.backward(gradient=seed.to(loss.dtype) if loss.dtype != seed.dtype else seed)
        grads.finish()
        if scaler.is_enabled():
            # unscale (and clip) folded into the step; a step whose gradients
            # overflowed is skipped and the scale backed off
            norm_value = float(scaler.unscale_(optimizer, max(args.max_grad_norm, 0.0)).item())
            scaler.step(optimizer, norm_value)
            scaler.update()
            grad_norm_value = norm_value if args.max_grad_norm > 0 else math.nan
        elif args.max_grad_norm > 0:
            norm = optimizer.clip_grad_norm_(args.max_grad_norm)
            optimizer.step()
            grad_norm_value = float(norm.item())
        else:
            optimizer.step()
            grad_norm_value = math.nan
        step_loss = float(sum(micro_losses) / len(micro_losses))
        recent.append(step_loss)
        if len(recent) > 100:
            recent.pop(0)
        tps = tokens_per_step / max(time.perf_counter() - t0, 1e-8)
        if step % args.log_interval == 0 or step == 1 or step == args.max_steps:
            avg = sum(recent) / len(recent)
            print(f"[step {step:05d}] loss={step_loss:.4f} avg100={avg:.4f} tokens/s={tps:,.0f} grad_norm={grad_norm_value:.3f}")
        if args.checkpoint_interval > 0 and (step % args.checkpoint_interval == 0 or step == args.max_steps):
            path = save_checkpoint(args.save_dir, step, model, optimizer, args,
                                   {"model_config": cfg.to_dict(), "step_loss": step_loss})
            print(f"[checkpoint] wrote {path}")
    print(f"[done] trained {args.max_steps} steps in {time.perf_counter() - t_start:.1f}s")


def main() -> None:
    train(parse_args())


if __name__ == "__main__":
    main()
