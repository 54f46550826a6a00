"""CPU oracle for the llama-zero single-GPU training step.

TEST INFRASTRUCTURE ONLY.  This package restates the reference's algorithms
(dannyadkins/cs244c-llama-zero) in plain PyTorch on the CPU so the HIP product
path can be checked against them.  Only tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg may import it, and only as the checker (or the
timed CPU baseline) — never as a compute path of the product.

Modules and the reference code each follows:
  ops.py    model/llama.py:14-39,42-69,88-117,136-146,273-302 (RMSNorm, RoPE,
            causal GQA attention, SwiGLU, shifted cross entropy) and the
            AdamW/clip arithmetic of zero/stage0_ddp.py:66-88.
  model.py  model/llama.py:149-308 (block composition, init order, chunked
            loss) and model/config.py:129-151 (parameter count).
  flat.py   zero/common.py:13-111 (flat parameter order, offsets, shard spec),
            zero/stage3_optimizer.py:313-349 (per-module handles), and the
            25M-element gradient bucket plan.
  engine.py zero/stage{0,1,2,3}*.py step semantics at world_size=1.
  data.py   data/fineweb.py:100-139 and train.py:139-145 (synthetic data).

How each part is pinned (tests/test_oracle.py):
  - the reference's golden loss 4.901787757873535 (tests/test_model.py:46-64)
    pins init order, RMSNorm, RoPE, attention, SwiGLU and the chunked loss;
  - library routines: F.scaled_dot_product_attention, F.cross_entropy,
    F.rms_norm, F.silu, torch.optim.AdamW + clip_grad_norm_;
  - invariants: RoPE norm preservation and relative-position dependence,
    causal masking, chunked == full loss, parameter counts vs the closed form,
    flat offsets vs brute force over the module tree.
"""
