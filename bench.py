"""Benchmark: the single-GPU LLaMA training step on one MI355X.

Headline (`value`): training tokens/s of the 1B-class model (d2048, 16 layers,
16 query / 8 KV heads, ffn 5632, vocab 32000, tied embeddings) through the
ZeRO-3 engine at world_size 1, micro-batch 8 x 2048 tokens, bf16 compute with
an fp32 flat master, synthetic uniform token ids (seed 0) already resident in
HBM, random-init weights (seed 0).  One step = zero_grad, prepare_forward,
forward + loss, backward (with ZeRO-3's recomputation, which leaves each
block's output, the down projection's product, unformed: only autograd.grad
reads it, so the gradients are the same; at one rank the
reduce-scatter of the flattened gradients is the identity, so each module's
bf16 gradients are gathered straight into the fp32 gradient shard instead of
through 25M-element bf16 buckets), step_with_stats (norm + fused AdamW).

Also reported: MFMA utilisation of that step (model FLOPs, 3x forward, over
2.5 PFLOP/s), the same step with the engine's recompute=False, the
CPU-runnable train.py workload on the HIP path beside the CPU oracle's loop,
the 125M-class ZeRO-1 step (B=16, S=1024), fused AdamW HBM
bandwidth on a 124M-element flat fp32 buffer, the other HBM-bound kernels at
the step's shapes, the dominant GEMM kernel's roofline measured with HIP
events around its launches inside the timed steps (every GEMM plan's share
comes from a separate pass of steps with events around every launch, whose
markers would otherwise add time to the timed steps), and the CPU oracle's
throughput on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "cs244c-llama-zero_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
METRIC = "train tokens/s on 1×MI355X (125M & 1B LLaMA, bf16); MFMA util %; AdamW GB/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_engine(size: str, stage: int, batch: int, seq: int, dev: torch.device, recompute: bool = True):
    from model import LlamaForCausalLM, build_config
    from zero import ZeROStage1Optimizer, ZeROStage3Optimizer

    cfg = build_config(size, vocab_size=32000, max_seq_len=seq)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=dev, dtype=torch.bfloat16)
    model.set_loss_chunk_size(128)
    cls = ZeROStage3Optimizer if stage == 3 else ZeROStage1Optimizer
    kw = {} if stage != 3 else {"recompute": recompute}
    engine = cls(model=model, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, **kw)
    return cfg, model, engine


def run_steps(model, engine, batches, steps: int, warmup: int):
    def one(ids):
        engine.zero_grad()
        engine.prepare_forward()
        loss = model(input_ids=ids, labels=ids, return_logits=False).loss
        engine.backward(loss)
        stats = engine.step_with_stats(max_grad_norm=0.0)
        return float(loss.detach()), stats

    for i in range(warmup):
        one(batches[i % len(batches)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    losses = []
    marks = [t0]
    for i in range(steps):
        loss, _ = one(batches[(warmup + i) % len(batches)])  # reads the loss: the host waits for the step
        losses.append(loss)
        marks.append(time.perf_counter())
    torch.cuda.synchronize()
    run_steps.step_ms = [(b - a) * 1000.0 for a, b in zip(marks, marks[1:])]
    return time.perf_counter() - t0, losses


def bench_125m(dev: torch.device, steps: int, warmup: int, per_plan: bool = False) -> dict:
    """The 125M model (d768, 12 layers, 12 q / 4 kv heads of 64, ffn 2048,
    vocab 32000) through the ZeRO-1 engine at B=16, S=1024; with per_plan,
    each GEMM launch plan's share of the step (HIP events on the launch
    stream, as for the headline)."""
    from lzhip import ops
    from profiler import estimate_transformer_train_flops

    gen = torch.Generator(device=dev).manual_seed(0)
    cfg, model, eng = make_engine("125m", 1, 16, 1024, dev)
    batches = [torch.randint(0, 32000, (16, 1024), device=dev, generator=gen) for _ in range(4)]
    k = max(steps, 5)
    probe = ops.LaunchProbe() if per_plan else None
    run_steps(model, eng, batches, steps=0, warmup=warmup)
    el, _ = run_steps(model, eng, batches, steps=k, warmup=0)
    if probe is not None:
        # per-plan shares from k more steps: the events add host time per
        # launch, so the step time above comes from the steps without them
        ops.set_gemm_probe(probe)
        try:
            run_steps(model, eng, batches, steps=k, warmup=0)
        finally:
            ops.set_gemm_probe(None)
    f = estimate_transformer_train_flops(cfg, 16, 1024, stage=0)
    out = {"tokens_per_s": 16 * 1024 * k / el, "ms_per_step": el * 1000 / k,
           "mfma_util": f * k / el / 1e12 / PEAK_BF16_TFLOPS, "model_tflop_per_step": f / 1e12,
           "workload": "125m ZeRO-1 (d768 L12 12q/4kv ffn2048 V32000), B=16 S=1024"}
    if probe is not None:
        n, fl, ms = probe.summary()
        out["gemm_all_launches"] = {"ms_per_step": ms / k, "TFLOP/s": fl / (ms * 1e-3) / 1e12}
        out["gemm_kernels"] = sorted(
            ({"kernel": ops.gemm_kernel_name(key), "launches": v[0], "ms_per_step": v[2] / k,
              "TFLOP/s": v[1] / (v[2] * 1e-3) / 1e12} for key, v in probe.by_key().items()),
            key=lambda d: -d["ms_per_step"])
    del model, eng
    torch.cuda.empty_cache()
    return out


def bench_adamw(dev: torch.device, ceilings=None, n: int = 124_000_000, iters: int = 10):
    from lzhip import ops

    g = torch.Generator(device=dev).manual_seed(0)
    p = 0.02 * torch.randn(n, device=dev, generator=g)
    grad = 1e-3 * torch.randn(n, device=dev, generator=g)
    m = ops.zeros((n,), torch.float32, dev)
    v = ops.zeros((n,), torch.float32, dev)
    ops.adamw_(p, m, v, grad, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=1)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for t in range(iters):
        ops.adamw_(p, m, v, grad, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=t + 2)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / iters
    gbs = 28.0 * n / (ms * 1e-3) / 1e9
    out = {"elements": n, "bytes_per_elem": 28, "ms": ms, "GB/s": gbs, "frac_of_8TBs": gbs / PEAK_HBM_GBS}
    # the form the ZeRO-3 step launches: the clip factor read from device
    # memory and the bf16 parameters written beside the fp32 master (30 B per
    # element)
    p16 = ops.cast(p, torch.bfloat16)
    scale = torch.ones((1,), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    start.record()
    for t in range(iters):
        ops.adamw_(p, m, v, grad, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=t + 12,
                   grad_scale=scale, p_out=p16)
    end.record()
    torch.cuda.synchronize()
    ms2 = start.elapsed_time(end) / iters
    gbs2 = 30.0 * n / (ms2 * 1e-3) / 1e9
    out["in_step_form"] = {"bytes_per_elem": 30, "ms": ms2, "GB/s": gbs2, "frac_of_8TBs": gbs2 / PEAK_HBM_GBS}
    if ceilings:
        out["frac_of_measured_copy"] = gbs / ceilings["copy_GB/s"]
        out["in_step_form"]["frac_of_measured_copy"] = gbs2 / ceilings["copy_GB/s"]
    return out


def run_no_recompute(args, B, S, dev, batches, tokens, model_flops):
    """The 1B ZeRO-3 step with the engine's recompute=False."""
    log("1B ZeRO-3 with recompute=False")
    _, m_nr, e_nr = make_engine("1b", 3, B, S, dev, recompute=False)
    el_nr, l_nr = run_steps(m_nr, e_nr, batches, steps=args.steps, warmup=args.warmup)
    res = {
        "tokens_per_s": tokens * args.steps / el_nr, "ms_per_step": el_nr * 1000.0 / args.steps,
        "mfma_util": model_flops * args.steps / el_nr / 1e12 / PEAK_BF16_TFLOPS, "loss_first_last": [l_nr[0], l_nr[-1]],
        "workload": "same 1B ZeRO-3 step with the engine's recompute=False (each module's forward graph kept; "
                    "same gradients, one forward per step)",
    }
    log(f"1B ZeRO-3 recompute=False: {res['ms_per_step']:.1f} ms/step")
    del m_nr, e_nr
    torch.cuda.empty_cache()
    return res


def fit_sweep(dev: torch.device, max_batch: int, seq: int = 2048, steps: int = 2, warmup: int = 1):
    """The 7B workload (d4096, 32 layers, 32 q / 8 kv heads, ffn 11008, vocab
    32000, tied) through the ZeRO-3 engine at world size 1, micro-batch 1, 2,
    4, ... until the device runs out of memory (or max_batch): tokens/s and
    peak HBM per size.  Parameters are created on the device."""
    from model import LlamaForCausalLM, build_config
    from profiler import estimate_transformer_train_flops
    from zero import ZeROStage3Optimizer

    cfg = build_config("7b", vocab_size=32000, max_seq_len=seq)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(cfg)
    model = model.to(dtype=torch.bfloat16)
    model.set_loss_chunk_size(128)
    engine = ZeROStage3Optimizer(model=model, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    n_params = sum(h.meta.total_numel for h in engine._handle_order)
    total = torch.cuda.get_device_properties(dev).total_memory
    gen = torch.Generator(device=dev).manual_seed(0)

    def run_one(b):
        log(f"7B fit sweep: micro-batch {b}")
        batches = None
        try:
            torch.cuda.reset_peak_memory_stats(dev)
            batches = [torch.randint(0, cfg.vocab_size, (b, seq), device=dev, generator=gen)]
            el, losses = run_steps(model, engine, batches, steps=steps, warmup=warmup)
            peak = torch.cuda.max_memory_allocated(dev)
            flops = estimate_transformer_train_flops(cfg, b, seq, stage=0)
            row = {"micro_batch": b, "tokens_per_s": b * seq * steps / el, "ms_per_step": el * 1000 / steps,
                   "mfma_util": flops * steps / el / 1e12 / PEAK_BF16_TFLOPS,
                   "peak_hbm_gib": peak / 2**30, "loss": losses[-1]}
            log(f"  {row['ms_per_step']:.0f} ms/step, {row['tokens_per_s']:,.0f} tok/s, "
                f"peak {row['peak_hbm_gib']:.1f} GiB")
            return row
        finally:
            batches = None
            engine.zero_grad()
            torch.cuda.empty_cache()

    rows = sweep_batches(run_one, max_batch)
    return {"metric": "7B ZeRO-3 fit-to-memory sweep (world size 1, S=2048, bf16 + fp32 master)",
            "params": n_params, "device_memory_gib": total / 2**30, "sweep": rows}


def sweep_batches(run_one, max_batch: int):
    """run_one(b) for micro-batch b = 1, 2, 4, ... up to max_batch, one row
    each; the first size that runs out of device memory ends the sweep with
    the row {"micro_batch": b, "oom": True} (any other error propagates)."""
    rows = []
    b = 1
    while b <= max_batch:
        try:
            rows.append(run_one(b))
        except torch.cuda.OutOfMemoryError:
            rows.append({"micro_batch": b, "oom": True})
            log("  out of memory")
            break
        b *= 2
    return rows


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_1b_zero3_traffic.md")
MFMA_PROFILE = os.path.join(ROOT, "profiles", "mfma_busy_1b_zero3_step.md")


def measured_mfma_busy(kernel: str):
    """MFMA-busy fraction of `kernel` (SQ_VALU_MFMA_BUSY_CYCLES over the SIMD
    cycles it occupied) from the committed counter profile of the same step
    (a line `mfma_busy <kernel> = x`), or None."""
    name = kernel.split(" split-K")[0]
    try:
        with open(MFMA_PROFILE) as f:
            for line in f:
                if line.startswith("mfma_busy ") and line[len("mfma_busy "):].rsplit(" = ", 1)[0] == name:
                    return float(line.rsplit("=", 1)[1])
    except OSError:
        pass
    return None


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE/WRITE_SIZE
    profile (a line `traffic_bytes_per_launch <kernel> = N`), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch") and kernel in line:
                    return float(line.rsplit("=", 1)[1])
    except OSError:
        pass
    return None


def bench_plumbing_graph(cfg, dtype, ids_all, B: int, S: int, GA: int, steps: int, dev: torch.device) -> dict:
    """The same workload with the whole step (both micro-batches, clip, AdamW
    with a device-resident step count) replayed from one HIP graph; each timed
    step copies its micro-batch ids into the graph's static inputs."""
    from lzhip.functional import GradSink, pack_parameters_
    from lzhip.graph import GraphedTrainStep
    from lzhip.optim import FusedAdamW
    from model import LlamaForCausalLM

    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=dev, dtype=dtype)
    pack_parameters_(model)
    model.set_loss_chunk_size(128)
    opt = FusedAdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, capturable=True)
    gs = GraphedTrainStep(model, opt, (B, S), GA, 1.0, dev, grads=GradSink(model))
    for i in range(3):
        gs.warmup(ids_all[GA * i:GA * (i + 1)])
    gs.capture()
    for i in range(3, 5):
        gs(ids_all[GA * i:GA * (i + 1)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        loss = gs(ids_all[GA * (5 + i):GA * (6 + i)])
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    return {"hip_graph_tokens_per_s": B * S * GA * steps / el, "hip_graph_ms_per_step": el * 1000 / steps,
            "hip_graph_final_loss": float(loss.detach())}


def bench_plumbing_eager(cfg, dtype, ids_all, B: int, S: int, GA: int, steps: int, dev: torch.device) -> dict:
    """train.py's step as it runs it, launched eagerly: GA micro-batches whose
    kernels write and then accumulate the gradients, clip, fused AdamW."""
    from lzhip import ops
    from lzhip.functional import GradSink, pack_parameters_
    from lzhip.optim import FusedAdamW
    from model import LlamaForCausalLM

    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=dev, dtype=dtype)
    pack_parameters_(model)
    model.set_loss_chunk_size(128)
    opt = FusedAdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    grads = GradSink(model)
    seed = ops.fill_(torch.empty((), dtype=torch.float32, device=dev), 1.0 / GA)

    def one(step):
        grads.begin_step()
        loss = None
        for a in range(GA):
            ids = ids_all[GA * step + a]
            loss = model(input_ids=ids, labels=ids, return_logits=False).loss
            loss.backward(gradient=seed)  # = (loss / GA).backward()
        grads.finish()
        opt.clip_grad_norm_(1.0)
        opt.step()
        return loss

    for i in range(5):
        one(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        loss = one(5 + i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    return {"hip_tokens_per_s": B * S * GA * steps / el, "hip_ms_per_step": el * 1000 / steps,
            "hip_final_loss": float(loss.detach())}


def bench_plumbing(dev: torch.device, cpu: bool, steps: int = 100, cpu_steps: int = 3):
    """The CPU-runnable train.py workload (d256, 4 layers, 8/4 heads, ffn 688,
    vocab 32000, B=4, S=128, grad accumulation 2, AdamW lr 3e-4, clip 1.0,
    uniform ids from torch.Generator seed 0) for `steps` steps on the HIP path,
    eagerly and replayed from a HIP graph, in fp32 (the reference's
    train.py default: parameters, gradients, optimizer state and matmuls in
    fp32) and in bf16 (bf16 parameters over an fp32 master); and the CPU
    oracle's train.py loop (fp32, every host thread) on `cpu_steps` steps of
    the same stream."""
    from model import build_config

    B, S, GA = 4, 128, 2
    cfg = build_config("plumbing", vocab_size=32000, max_seq_len=S)
    gen = torch.Generator().manual_seed(0)
    chunks = [torch.randint(0, 32000, (B, S + 1), generator=gen) for _ in range(GA * (steps + 5))]
    ids_all = [c[:, :-1].contiguous().to(dev) for c in chunks]
    res = {"workload": f"train.py plumbing (d256 L4 8/4 heads ffn688 V32000), B=4 S=128 GA=2, {steps} steps"}
    for name, dtype in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        leg = bench_plumbing_eager(cfg, dtype, ids_all, B, S, GA, steps, dev)
        leg.update(bench_plumbing_graph(cfg, dtype, ids_all, B, S, GA, steps, dev))
        res[name] = leg
    if cpu:
        from oracle import engine as OE
        from oracle import model as OM
        from model import LlamaForCausalLM

        torch.manual_seed(0)
        P = {k: v.detach().clone() for k, v in LlamaForCausalLM(cfg).state_dict().items() if k != "lm_head.weight"}
        ocfg = OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                      n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta)
        out = OE.train_reference(ocfg, P, iter(chunks), steps=cpu_steps, grad_accum_steps=GA, lr=3e-4,
                                 betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=1.0, loss_chunk_size=128)
        sec = sum(out["seconds"])
        res.update({"cpu_oracle_tokens_per_s": B * S * GA * cpu_steps / sec, "cpu_cores": torch.get_num_threads(),
                    "cpu_sample": f"{cpu_steps} steps of the same stream in fp32 ({sec:.1f} s)"})
    return res


def cpu_ops_baseline(rows: int = 16384, dim: int = 2048, ffn: int = 5632, heads: int = 16, n_adam: int = 124_000_000):
    """The CPU oracle's op restatements at the op-level shapes (fp32 on the
    host, every thread), forward + backward through autograd, and its AdamW
    over 124M elements: milliseconds per call."""
    from oracle import ops as O

    def t(fn, reps=2):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) * 1000.0 / reps

    g = torch.Generator().manual_seed(0)
    x = torch.randn(rows, dim, generator=g).requires_grad_(True)
    w = (1 + 0.02 * torch.randn(dim, generator=g)).requires_grad_(True)
    dy = torch.randn(rows, dim, generator=g)
    out = {"cores": torch.get_num_threads()}
    out["rmsnorm fwd+bwd ms"] = t(lambda: O.rmsnorm(x, w, 1e-5).backward(dy))
    hd = dim // heads
    cos, sin = O.rope_tables(2048, hd, 10000.0)
    xr = torch.randn(rows // 2048, heads, 2048, hd, generator=g).requires_grad_(True)
    dr = torch.randn(xr.shape, generator=g)
    out["rope fwd+bwd ms"] = t(lambda: O.apply_rope(xr, cos, sin).backward(dr))
    gg = torch.randn(rows, ffn, generator=g).requires_grad_(True)
    uu = torch.randn(rows, ffn, generator=g).requires_grad_(True)
    dh = torch.randn(rows, ffn, generator=g)
    out["swiglu fwd+bwd ms"] = t(lambda: O.swiglu(gg, uu).backward(dh))
    del x, dy, xr, dr, gg, uu, dh
    p = 0.02 * torch.randn(n_adam, generator=g)
    m, v = torch.zeros(n_adam), torch.zeros(n_adam)
    gr = 1e-3 * torch.randn(n_adam, generator=g)
    st = [0]

    def adam():
        st[0] += 1
        O.adamw_update(p, m, v, gr, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=st[0])

    out["adamw 124M ms"] = t(adam, reps=1)
    out["sample"] = "[16384, 2048] RMSNorm, [8, 16, 2048, 128] RoPE, [16384, 5632] SwiGLU in fp32, AdamW over 124M"
    return out


def _time_ms(fn, iters: int = 20) -> float:
    for _ in range(3):
        fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def _time_graph_ms(fn, iters: int = 20) -> float:
    """Device time per call of `fn` with the host out of the way: `iters`
    calls captured into one HIP graph (after 3 eager warm-up calls, so that
    cached workspaces exist before capture) and the graph replayed between HIP
    events.  Short kernels (tens of microseconds) launched through the Python
    wrappers one by one are otherwise partly host-bound."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / iters
    del graph
    return ms


def _time_graph_cycle_ms(fns, iters: int = 24) -> float:
    """_time_graph_ms over calls that cycle through `fns` (closures over
    different buffer sets), so that a kernel's inputs are not the ones the
    previous call just read: with sets whose total exceeds the 256 MB
    Infinity Cache the inputs come from HBM, as in a training step."""
    n = len(fns)
    return _time_graph_ms(_Cycle(fns), iters - iters % n)


class _Cycle:
    def __init__(self, fns):
        self.fns, self.i = list(fns), 0

    def __call__(self):
        f = self.fns[self.i % len(self.fns)]
        self.i += 1
        return f()


def bench_ceilings(dev: torch.device) -> dict:
    """What this box's HBM and MFMA deliver, measured, beside the published
    8 TB/s and 2.5 PFLOP/s: a STREAM-style 1 GiB -> 1 GiB copy and a 2 GiB
    read-only pass (both this library's kernels: copy2d and the fp32 sum of
    squares), and hipBLASLt's bf16 GEMM (torch.matmul) at the 1B step's QKV,
    gate|up and down projection shapes."""
    from lzhip import ops

    out = {}
    a = torch.ones(1 << 14, 1 << 15, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    ms = _time_ms(lambda: ops.copy2d(a, b), 10)
    out["copy_GB/s"] = 2.0 * 2 * a.numel() / (ms * 1e-3) / 1e9
    del a, b
    r = torch.ones(1 << 29, dtype=torch.float32, device=dev)
    acc = torch.zeros((), dtype=torch.float64, device=dev)
    ms = _time_ms(lambda: ops.sumsq_(r, acc), 10)
    out["read_GB/s"] = 4.0 * r.numel() / (ms * 1e-3) / 1e9
    del r
    out["copy_frac_of_8TBs"] = out["copy_GB/s"] / PEAK_HBM_GBS
    out["read_frac_of_8TBs"] = out["read_GB/s"] / PEAK_HBM_GBS
    g = torch.Generator(device=dev).manual_seed(0)
    shapes = {"qkv 16384x4096x2048": (16384, 4096, 2048), "gate|up 16384x11264x2048": (16384, 11264, 2048),
              "down 16384x2048x5632": (16384, 2048, 5632)}
    lib = {}
    for name, (M, N, K) in shapes.items():
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        w = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
        ms = _time_ms(lambda: torch.matmul(x, w.t()), 20)
        lib[name] = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        del x, w
    out["hipblaslt_bf16_TFLOP/s"] = lib
    out["hipblaslt_best_frac_of_2.5PF"] = max(lib.values()) / PEAK_BF16_TFLOPS
    return out


def bench_pointwise(dev: torch.device, ceilings=None, rows: int = 16384, dim: int = 2048, ffn: int = 5632,
                    heads: int = 16):
    """The step's HBM-bound kernels at the 1B step's shapes (bf16, 8x2048
    tokens): bytes moved (each input read once, each output written once) per
    launch time.  A plain 1 GiB device copy is timed beside them as the
    achievable-bandwidth reference.  Each rate is the device time of calls
    replayed from one HIP graph.  RMSNorm's rates cycle through 4 input sets
    (256-512 MB in all), so its inputs come from HBM as in the step; the
    `*_warm` figures call it on one set, which the 256 MB Infinity Cache
    partly serves, so they can exceed HBM's rate.  The other kernels run on
    one set (warm)."""
    from lzhip import ops

    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    out = {}

    def rec(name, ms, nbytes):
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": ms * 1e3, "bytes": nbytes, "GB/s": gbs, "frac_of_8TBs": gbs / PEAK_HBM_GBS}
        if ceilings:
            out[name]["frac_of_measured_copy"] = gbs / ceilings["copy_GB/s"]

    # plain copy of 1 GiB with this library's copy2d_vec_kernel (also the known-size
    # kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters)
    a = torch.ones(1 << 14, 1 << 15, dtype=bf, device=dev)
    b = torch.empty_like(a)
    rec("device copy 1 GiB (copy2d_vec_kernel)", _time_graph_ms(lambda: ops.copy2d(a, b), 10), 2 * 2 * a.numel())
    del a, b
    w = (1 + 0.02 * torch.randn(dim, device=dev, generator=g)).to(bf)
    sets = []
    for _ in range(4):
        xs = torch.randn(rows, dim, device=dev, generator=g).to(bf)
        sets.append((xs, torch.randn(rows, dim, device=dev, generator=g).to(bf), ops.rmsnorm_fwd(xs, w, 1e-5)[1]))
    x, dy, rstd = sets[0]
    n = rows * dim

    def rec_cycled(name, fns, nbytes):
        rec(name, _time_graph_cycle_ms(fns), nbytes)
        warm = _time_graph_ms(fns[0])
        out[name]["us_warm"] = warm * 1e3
        out[name]["GB/s_warm"] = nbytes / (warm * 1e-3) / 1e9
        out[name]["frac_of_8TBs_warm"] = out[name]["GB/s_warm"] / PEAK_HBM_GBS

    rec_cycled(f"rmsnorm fwd [{rows},{dim}]", [lambda s=s: ops.rmsnorm_fwd(s[0], w, 1e-5) for s in sets], 4 * n)
    rec_cycled(f"rmsnorm bwd [{rows},{dim}]", [lambda s=s: ops.rmsnorm_bwd(s[0], w, s[2], s[1]) for s in sets], 6 * n)
    del sets
    hd = dim // heads
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32, device=dev) / hd))
    cos, sin = ops.rope_table(2048, hd, inv, bf)
    rec(f"rope fwd [{rows},{heads}x{hd}] in place", _time_graph_ms(lambda: ops.rope_(x, 2048, heads, hd, cos, sin)), 4 * n)
    rec(f"rope bwd [{rows},{heads}x{hd}] in place",
        _time_graph_ms(lambda: ops.rope_(x, 2048, heads, hd, cos, sin, backward=True)), 4 * n)
    del x, dy
    gu = torch.randn(rows, 2 * ffn, device=dev, generator=g).to(bf)
    gate, up = gu[:, :ffn], gu[:, ffn:]
    rec(f"swiglu fwd [{rows},{ffn}]", _time_graph_ms(lambda: ops.swiglu_fwd(gate, up)), 6 * rows * ffn)
    dh = torch.randn(rows, ffn, device=dev, generator=g).to(bf)
    dgu = torch.empty_like(gu)
    rec(f"swiglu bwd [{rows},{ffn}]",
        _time_graph_ms(lambda: ops.swiglu_bwd(gate, up, dh, dgu[:, :ffn], dgu[:, ffn:])), 10 * rows * ffn)
    return out


def cpu_baseline(cfg, tokens: int = 2048, seq: int = 2048, warmup: int = 1):
    """The CPU oracle (a port of the reference math) on a bounded sample of the
    same workload: forward+backward over `tokens` tokens (sequences of the
    headline's length) of the 1B model and one AdamW update of all its
    parameters, in fp32 on the host, timed after `warmup` untimed steps."""
    from oracle import engine as OE
    from oracle import model as OM

    threads = len(os.sched_getaffinity(0))  # every CPU this process may run on
    torch.set_num_threads(threads)
    ocfg = OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                  n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta)
    torch.manual_seed(0)
    P = {k: v.requires_grad_(True) for k, v in OM.init_params(ocfg).items()}
    ids = torch.randint(0, cfg.vocab_size, (tokens // seq, seq), generator=torch.Generator().manual_seed(0))
    eng = OE.EngineRef(torch.cat([p.detach().reshape(-1) for p in P.values()]), lr=3e-4)

    def step():
        for p in P.values():
            p.grad = None
        loss = OM.loss(P, ocfg, ids, chunk_size=128)
        loss.backward()
        eng.step(torch.cat([p.grad.reshape(-1) for p in P.values()]))

    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    step()
    sec = time.perf_counter() - t0
    return {
        "value": tokens / sec,
        "unit": "tokens/s",
        "cores": threads,
        "host_cpu_count": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "kind": "port",
        "sample": f"1 step of the same 1B workload on {tokens} tokens ({tokens // seq}x{seq}) in fp32 after "
                  f"{warmup} untimed step: forward, backward and the AdamW update of all "
                  f"{sum(p.numel() for p in P.values()):,} parameters ({sec:.1f} s)",
    }


def gemm_sweep(dev: torch.device) -> dict:
    """The 1B step's GEMM shapes (16384 tokens) one product at a time, with HIP
    events around 20 launches each: forward x.W^T (with and without the
    block's residual), input gradient dy.W and weight gradient dy^T.x, each
    next to hipBLASLt (torch.matmul) on the same operands; the 125M step's
    weight gradients the same way; and the O-projection shape at K = 64 ...
    2048, whose intercept is the fixed per-launch cost (prologue, epilogue,
    launch) and whose slope is the main loop's rate."""
    from lzhip import ops

    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    T = 16384
    out = {"tokens": T, "products_TFLOP/s": {}, "k_sweep_us": {}}
    for name, (N, K) in {"qkv": (4096, 2048), "gate|up": (11264, 2048), "o": (2048, 2048), "down": (2048, 5632),
                         "lm_head": (32000, 2048)}.items():
        x = torch.randn(T, K, device=dev, generator=g).to(bf)
        w = (0.02 * torch.randn(N, K, device=dev, generator=g)).to(bf)
        dy = torch.randn(T, N, device=dev, generator=g).to(bf)
        f = 2.0 * T * N * K / 1e9
        r = {"forward": f / _time_ms(lambda: ops.gemm(x, w)),
             "input_grad": f / _time_ms(lambda: ops.gemm(dy, w, b_kmajor=False)),
             "weight_grad": f / _time_ms(lambda: ops.gemm(dy, x, a_kmajor=False, b_kmajor=False)),
             "hipblaslt_forward": f / _time_ms(lambda: torch.matmul(x, w.t())),
             "hipblaslt_input_grad": f / _time_ms(lambda: torch.matmul(dy, w)),
             "hipblaslt_weight_grad": f / _time_ms(lambda: torch.matmul(dy.t(), x))}
        if N == 2048:
            res = torch.randn(T, N, device=dev, generator=g).to(bf)
            r["forward_residual"] = f / _time_ms(lambda: ops.gemm(x, w, residual=res))
        out["products_TFLOP/s"][name] = {k: round(v, 1) for k, v in r.items()}
        del x, w, dy
    out["weight_grad_125m_TFLOP/s"] = {}
    for name, (M, N) in {"qkv": (1280, 768), "o": (768, 768), "gate|up": (4096, 768), "down": (768, 2048),
                         "lm_head": (32000, 768)}.items():
        dy = torch.randn(T, M, device=dev, generator=g).to(bf)
        x = torch.randn(T, N, device=dev, generator=g).to(bf)
        f = 2.0 * T * M * N / 1e9
        out["weight_grad_125m_TFLOP/s"][name] = {
            "ours": round(f / _time_ms(lambda: ops.gemm(dy, x, a_kmajor=False, b_kmajor=False)), 1),
            "hipblaslt": round(f / _time_ms(lambda: torch.matmul(dy.t(), x)), 1)}
        del dy, x
    N = 2048
    for K in (64, 128, 256, 512, 1024, 2048):
        x = torch.randn(T, K, device=dev, generator=g).to(bf)
        w = torch.randn(N, K, device=dev, generator=g).to(bf)
        res = torch.randn(T, N, device=dev, generator=g).to(bf)
        y = torch.empty(T, N, device=dev, dtype=bf)
        out["k_sweep_us"][K] = {"plain": round(1000 * _time_ms(lambda: ops.gemm(x, w, out=y)), 2),
                                "residual": round(1000 * _time_ms(lambda: ops.gemm(x, w, out=y, residual=res)), 2)}
    ks = sorted(out["k_sweep_us"])
    k0, k1 = ks[-3], ks[-1]
    t0, t1 = out["k_sweep_us"][k0]["plain"], out["k_sweep_us"][k1]["plain"]
    slope = (t1 - t0) / (k1 - k0)  # us per unit of K
    out["fixed_cost_us"] = round(t1 - slope * k1, 2)
    out["main_loop_TFLOP/s"] = round(2.0 * T * N / (slope * 1e-6) / 1e12, 1)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-125m", action="store_true")
    ap.add_argument("--fit-sweep", action="store_true",
                    help="7B ZeRO-3 fit-to-memory sweep: micro-batch 1, 2, 4, ... (S=2048) until the device is "
                         "out of memory or --fit-max-batch; prints one JSON line and exits")
    ap.add_argument("--fit-max-batch", type=int, default=64)
    ap.add_argument("--skip-plumbing", action="store_true", help="skip the train.py plumbing leg")
    ap.add_argument("--plumbing-only", action="store_true",
                    help="only the train.py plumbing leg (eager and HIP-graph replay); prints its JSON and exits")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="the 1B step's GEMM shapes one product at a time (with hipBLASLt beside them) and a K "
                         "sweep of the O projection; prints one JSON line and exits")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the 1B ZeRO-3 step (no recompute=False, 125M, AdamW or pointwise legs)")
    ap.add_argument("--125m-only", dest="only_125m", action="store_true",
                    help="only the 125M ZeRO-1 step (B=16, S=1024), with its GEMM launches timed per plan; prints "
                         "one JSON line and exits")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's engines run at world_size 1 (got --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    import lzhip
    from lzhip import ops
    from profiler import estimate_transformer_train_flops

    if args.plumbing_only:
        lzhip.load()
        print(json.dumps({"plumbing_train_py": bench_plumbing(torch.device("cuda:0"),
                                                              cpu=not args.no_cpu_baseline)}), flush=True)
        return 0

    lzhip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.fit_sweep:
        print(json.dumps(fit_sweep(dev, args.fit_max_batch)), flush=True)
        return 0
    if args.gemm_sweep:
        print(json.dumps({"gemm_sweep": gemm_sweep(dev)}), flush=True)
        return 0
    if args.only_125m:
        print(json.dumps({"llama_125m_zero1": bench_125m(dev, args.steps, args.warmup, per_plan=True)}), flush=True)
        return 0
    B, S = 8, 2048
    log("building 1B model + ZeRO-3 engine")
    cfg, model, engine = make_engine("1b", 3, B, S, dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    batches = [torch.randint(0, cfg.vocab_size, (B, S), device=dev, generator=gen) for _ in range(4)]
    log(f"warmup {args.warmup} + timed {args.steps} steps")
    # warmup without the probe; then a pass that times every GEMM launch with
    # HIP events (their markers add time between launches, so these steps
    # are not the timed ones), which ranks the launch plans by their share of
    # the step; then the timed steps, with events only around the dominant
    # plan's launches for the roofline
    run_steps(model, engine, batches, steps=0, warmup=args.warmup)
    plan_steps = max(2, min(args.steps, 5))
    all_plans = ops.LaunchProbe()
    ops.set_gemm_probe(all_plans)
    try:
        run_steps(model, engine, batches, steps=plan_steps, warmup=0)
    finally:
        ops.set_gemm_probe(None)
    per_kernel = all_plans.by_key()
    top_key = max(per_kernel, key=lambda k: per_kernel[k][2])
    probe = ops.LaunchProbe(only=top_key)
    ops.set_gemm_probe(probe)
    try:
        elapsed, losses = run_steps(model, engine, batches, steps=args.steps, warmup=0)
    finally:
        ops.set_gemm_probe(None)
    ms = elapsed * 1000.0 / args.steps
    step_ms = sorted(run_steps.step_ms)
    ms_median = step_ms[len(step_ms) // 2]
    tokens = B * S
    value = tokens * args.steps / elapsed
    model_flops = estimate_transformer_train_flops(cfg, B, S, stage=0)
    # executed flops: the stage-3 formula's recompute (a fourth forward) less
    # each layer's down projection, which the recompute leaves unformed (only
    # autograd.grad reads the recomputed block output)
    hw_flops = estimate_transformer_train_flops(cfg, B, S, stage=3) - 2.0 * B * S * cfg.ffn_dim * cfg.dim * cfg.n_layers
    n_launch, gemm_flops, gemm_ms = all_plans.summary()
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12
    # the dominant GEMM kernel (the most launch time in the plan pass), timed
    # over the timed steps
    top_n, top_flops, top_ms = probe.summary(top_key)
    top_tflops = top_flops / (top_ms * 1e-3) / 1e12
    gemm_kernels = sorted(
        ({"kernel": ops.gemm_kernel_name(k), "launches": v[0], "ms_per_step": v[2] / plan_steps,
          "TFLOP/s": v[1] / (v[2] * 1e-3) / 1e12} for k, v in per_kernel.items()),
        key=lambda d: -d["ms_per_step"])
    log(f"1B ZeRO-3: {ms:.1f} ms/step, {value:,.0f} tok/s, loss {losses[0]:.3f}->{losses[-1]:.3f}")
    peak_mem = torch.cuda.max_memory_allocated(dev) / 2**30

    del model, engine
    torch.cuda.empty_cache()
    if args.headline_only:
        args.skip_125m = True
    res_norecompute = adamw = pointwise = None
    if not args.headline_only:
        res_norecompute = run_no_recompute(args, B, S, dev, batches, tokens, model_flops)
    res_125m = None
    if not args.skip_125m:
        log("125M ZeRO-1")
        res_125m = bench_125m(dev, args.steps, args.warmup)
    plumbing = ceilings = None
    if not args.headline_only and not args.skip_plumbing:
        log("plumbing workload (train.py config)")
        plumbing = bench_plumbing(dev, cpu=not args.no_cpu_baseline)
    if not args.headline_only:
        log("measured ceilings")
        ceilings = bench_ceilings(dev)
        log("AdamW 124M")
        adamw = bench_adamw(dev, ceilings)
        log("pointwise kernels")
        pointwise = bench_pointwise(dev, ceilings)

    cpu = cpu_ops = None
    if not args.no_cpu_baseline:
        log("CPU oracle baseline")
        cpu = cpu_baseline(cfg)
        if not args.headline_only:
            log("CPU oracle ops")
            cpu_ops = cpu_ops_baseline()

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_median": ms_median,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic uniform token ids (seed 0) resident in HBM; random-init weights (seed 0)",
        "config": {
            "workload": "llama-1b ZeRO-3 train step at world_size 1 (d2048 L16 16q/8kv hd128 ffn5632 V32000 tied, "
                        "820,578,304 params), bf16 + fp32 master; at one rank each module's bf16 gradients are "
                        "gathered straight into the fp32 gradient shard (the reduce-scatter of 25M-element buckets "
                        "is the identity there)",
            "global_batch": B,
            "seq_len": S,
            "zero_stage": 3,
        },
        "mfma_util": model_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "model_tflop_per_step": model_flops / 1e12,
        "hardware_tflop_per_step_with_recompute": hw_flops / 1e12,
        "peak_hbm_gib": peak_mem,
        "loss_first_last": [losses[0], losses[-1]],
        "llama_1b_zero3_recompute_off": res_norecompute,
        "plumbing_train_py": plumbing,
        "llama_125m_zero1": res_125m,
        "measured_ceilings": ceilings,
        "adamw_124m": adamw,
        "pointwise": pointwise,
        "gemm_all_launches": {"launches": n_launch, "steps": plan_steps, "ms_per_step": gemm_ms / plan_steps,
                              "TFLOP/s": gemm_tflops, "frac": gemm_tflops / PEAK_BF16_TFLOPS},
        "gemm_kernels": gemm_kernels,
        "roofline": {
            "kernel": ops.gemm_kernel_name(top_key),
            "bound": "mfma",
            "achieved": top_tflops,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": top_tflops / PEAK_BF16_TFLOPS,
            "traffic": measured_traffic(ops.gemm_kernel_name(top_key)),
            "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
            "mfma_busy": measured_mfma_busy(ops.gemm_kernel_name(top_key)),
            "mfma_busy_source": os.path.relpath(MFMA_PROFILE, ROOT),
            "launches": top_n,
            "avg_launch_ms": top_ms / max(top_n, 1),
            "flop_per_launch": top_flops / max(top_n, 1),
        },
        "cpu_baseline": cpu,
        "cpu_ops_baseline": cpu_ops,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
