"""fp16 models on the GPU (reference train.py --dtype float16: parameters in
fp16 under fp16 autocast, torch.cuda.amp.GradScaler; train.py:148-160,
213-214,254-269).

- The fp16 MFMA GEMM (v_mfma_f32_32x32x16_f16, the bf16 kernels' loops) in
  every operand layout against float64: fp32 output within 1e-5 (fp16
  products are exact in fp32), fp16 output within one fp16 rounding (1e-3
  relative), residual and accumulation (beta) as the bf16 kernels do them.
- RoPE tables and rotation bit-exact against the oracle's op sequence in
  fp16 arithmetic (angles formed in the fp16 inv_freq buffer's dtype).
- Attention (one-wave-per-row and quad kernels) against float64.
- The model's loss and gradients against the float64 oracle at the fp16
  parameters: loss within 1e-2, gradient cosine >= 0.999.
- Training with the loss scaler: 30 steps teacher-forced against the
  oracle's train.py loop with fp16 parameter semantics (loss within 1e-2,
  unscaled gradient cosine >= 0.999 per step); an overflowing step is
  skipped and backs the scale off; train.py --dtype float16 runs.
"""
from __future__ import annotations

import math
import os
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from lzhip import ops
from lzhip.optim import FusedAdamW, LossScaler
from model import LlamaForCausalLM, ModelConfig, build_config
from oracle import data as OD
from oracle import engine as OE
from oracle import model as OM
from oracle import ops as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
H16 = torch.float16
ROOT = Path(__file__).resolve().parents[1]


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (300, 200, 136), (256, 256, 16384), (1024, 2048, 64)])
@pytest.mark.parametrize("ak,bk", [(True, True), (True, False), (False, True), (False, False)])
def test_gemm_f16_vs_float64(M, N, K, ak, bk):
    g = torch.Generator().manual_seed(M + N + K + 2 * ak + bk)
    A = torch.randn(M, K, generator=g).to(H16)
    B = torch.randn(N, K, generator=g).to(H16)
    ref = A.double() @ B.double().t()
    a = (A if ak else A.t().contiguous()).to(DEV)
    b = (B if bk else B.t().contiguous()).to(DEV)
    c32 = ops.gemm(a, b, ak, bk, out_dtype=torch.float32)
    assert _rel(c32, ref) < 1e-5
    c16 = ops.gemm(a, b, ak, bk)
    assert c16.dtype == H16 and _rel(c16, ref) < 1e-3
    # the block's residual: product rounded to fp16, then the sum rounded
    res = torch.randn(M, N, generator=g).to(H16)
    cr = ops.gemm(a, b, ak, bk, residual=res.to(DEV))
    assert _rel(cr, (ref.to(H16).double() + res.double()).to(H16)) < 1e-3
    # accumulation into an existing fp16 gradient (beta = 1)
    acc = torch.randn(M, N, generator=g).to(H16)
    out = acc.to(DEV)
    ops.gemm(a, b, ak, bk, out=out, beta=1.0)
    assert _rel(out, ref + acc.double()) < 1e-3
    with pytest.raises(TypeError):
        ops.gemm(a, b.to(torch.bfloat16), ak, bk)


def test_rope_f16_tables_and_rotation():
    """fp16 cos/sin tables (angles in the fp16 inv_freq buffer, positions past
    2048 rounded as torch.arange in fp16 rounds them) within one fp16 ulp of
    the oracle's (the device's and the host's sin/cos may differ in the last
    fp32 bit), and the rotation bit-exact against the oracle's fp16 op
    sequence on the same tables."""
    S, Hh, hd, theta = 2304, 4, 64, 10_000.0
    inv = R.inv_freq(hd, theta).to(H16)
    cos, sin = ops.rope_table(S, hd, inv.to(DEV), H16)
    rc, rs = R.rope_tables(S, hd, theta, dtype=H16, angle_dtype=H16)
    for got, want in ((cos.cpu(), rc), (sin.cpu(), rs)):
        ulp = want.abs().float() * 2.0 ** -10 + 2.0 ** -24  # at least one fp16 ulp of the value
        assert bool(((got.float() - want.float()).abs() <= ulp).all())
        assert (got != want).float().mean() < 1e-3
    g = torch.Generator().manual_seed(4)
    x = torch.randn(S, Hh * hd, generator=g).to(H16)
    c, s = cos.cpu(), sin.cpu()
    for backward in (False, True):
        y = x.to(DEV)
        ops.rope_(y, S, Hh, hd, cos, sin, backward=backward)
        xh = x.view(1, S, Hh, hd).transpose(1, 2)
        if backward:  # the transpose of the rotation: x*cos + rotate_half^T(x*sin)
            half = hd // 2
            xs = xh * s
            rot_t = torch.cat((xs[..., half:], -xs[..., :half]), dim=-1)
            ref = xh * c + rot_t
        else:
            ref = R.apply_rope(xh, c, s)
        assert torch.equal(y.cpu(), ref.transpose(1, 2).reshape(S, Hh * hd))


@pytest.mark.parametrize("B,S,Hq,KV,hd", [(2, 64, 4, 2, 64), (1, 256, 8, 4, 128), (1, 96, 4, 2, 32),
                                          (2, 40, 6, 2, 128)])
def test_attention_f16_vs_float64(B, S, Hq, KV, hd):
    """Causal GQA attention in fp16 forward and backward against float64: the
    MFMA tile kernels (v_mfma_f32_32x32x16_f16; head dim 64 or 128, S a
    multiple of 64), the quad kernels (head dim 32) and the one-wave-per-row
    kernels (the rest); and with an fp16 additive mask."""
    g = torch.Generator().manual_seed(B * S + hd)
    ld = (Hq + 2 * KV) * hd
    qkv = torch.randn(B * S, ld, generator=g).to(H16)
    d = qkv.to(DEV)
    q2, k2, v2 = d[:, : Hq * hd], d[:, Hq * hd : (Hq + KV) * hd], d[:, (Hq + KV) * hd :]
    scale = hd**-0.5
    assert ops.attn_path(H16, S, hd, ld, ld, ld, Hq * hd) == (2 if hd in (64, 128) and S % 64 == 0 else 0)
    o, lse = ops.attn_fwd(q2, k2, v2, B, S, Hq, KV, hd, scale, None)

    def heads(t, n):
        return t.double().view(B, S, n, hd).transpose(1, 2).requires_grad_(True)

    qr, kr, vr = heads(qkv[:, : Hq * hd], Hq), heads(qkv[:, Hq * hd : (Hq + KV) * hd], KV), heads(qkv[:, (Hq + KV) * hd :], KV)
    oref = R.causal_gqa_attention(qr, kr, vr, scale)
    assert _rel(o.view(B, S, Hq, hd).transpose(1, 2), oref) < 2e-3
    do = torch.randn(B * S, Hq * hd, generator=g).to(H16)
    dqkv = torch.zeros_like(d)
    ops.attn_bwd(q2, k2, v2, o, do.to(DEV), lse, B, S, Hq, KV, hd, scale, dqkv[:, : Hq * hd],
                 dqkv[:, Hq * hd : (Hq + KV) * hd], dqkv[:, (Hq + KV) * hd :])
    oref.backward(do.double().view(B, S, Hq, hd).transpose(1, 2))
    for got, want in ((dqkv[:, : Hq * hd], qr.grad), (dqkv[:, Hq * hd : (Hq + KV) * hd], kr.grad),
                      (dqkv[:, (Hq + KV) * hd :], vr.grad)):
        n = want.shape[1]
        assert _rel(got.view(B, S, n, hd).transpose(1, 2), want) < 5e-3
    mask = torch.randn(S, S, generator=g).masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1),
                                                      float("-inf")).to(H16)
    om, _ = ops.attn_fwd_general(q2, k2, v2, B, S, Hq, KV, hd, scale, mask.to(DEV))
    with torch.no_grad():
        mref = R.causal_gqa_attention(qr, kr, vr, scale, attn_mask=mask.double())
    assert _rel(om.view(B, S, Hq, hd).transpose(1, 2), mref) < 2e-3


def _ocfg(cfg: ModelConfig) -> OM.Cfg:
    return OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                  n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta,
                  rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings, rope_angle_dtype=H16)


@pytest.mark.parametrize("dim,Hq,KV,S,chunk", [(128, 4, 2, 64, 0), (256, 4, 2, 128, 64), (512, 4, 2, 256, 0)])
def test_model_f16_vs_oracle(dim, Hq, KV, S, chunk):
    cfg = ModelConfig(name="f16", vocab_size=1000, max_seq_len=S, dim=dim, n_layers=2, n_heads=Hq, n_kv_heads=KV,
                      ffn_dim=2 * dim, rope_theta=10_000.0)
    torch.manual_seed(dim + S)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=H16)
    model.set_loss_chunk_size(chunk)
    P = {k: v.detach().double().cpu().requires_grad_(True) for k, v in model.state_dict().items()
         if k != "lm_head.weight"}
    ids = torch.randint(0, cfg.vocab_size, (2, S), generator=torch.Generator().manual_seed(S))
    out = model(input_ids=ids.to(DEV), labels=ids.to(DEV), return_logits=False)
    out.loss.backward()
    ref = OM.loss(P, _ocfg(cfg), ids, chunk_size=chunk)
    ref.backward()
    assert abs(float(out.loss.detach()) - float(ref.detach())) <= 1e-2 * abs(float(ref.detach()))
    for name, p in model.named_parameters():
        assert p.grad.dtype == H16
        cos = float(F.cosine_similarity(p.grad.double().cpu().view(-1), P[name].grad.view(-1), dim=0))
        assert cos >= 0.999, (name, cos)


def test_loss_scaled_training_vs_oracle():
    """30 steps of the plumbing workload in fp16 with the loss scaler at
    GradScaler's default scale (backward seeded with scale / GA, unscale and
    clip folded into FusedAdamW; a scale whose gradients overflow is backed
    off and the step taken again), teacher-forced: at each step the HIP path starts from the oracle
    trainer's parameters rounded to fp16; loss within 1e-2, unscaled
    gradient cosine >= 0.999, and the norm the scaler reports equals the
    norm of the unscaled gradients."""
    steps, B, S, GA = 30, 4, 128, 2
    cfg = build_config("plumbing", vocab_size=32000, max_seq_len=S)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg)
    P = {k: v.detach().clone() for k, v in model.state_dict().items() if k != "lm_head.weight"}
    order = [n for n, _ in model.named_parameters()]
    model = model.to(device=DEV, dtype=H16)
    model.set_loss_chunk_size(128)
    opt = FusedAdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    scaler = LossScaler()  # GradScaler's defaults: 2^16 first
    batches = [next(gen) for gen in [OD.uniform_chunks(S, cfg.vocab_size, B, seed=0)] for _ in range(steps * GA)]
    rel, cos, norm_rel, overflows = [], [], [], []

    def on_step(step, loss, gn, grads, params):
        with torch.no_grad():
            model.load_state_dict({k: v.to(H16) for k, v in params.items()}, strict=False)
        while True:  # an overflowing scale backs off and the step is taken again
            model.zero_grad(set_to_none=True)
            seed = torch.full((), scaler.scale_value() / GA, dtype=torch.float32, device=DEV)
            losses = []
            for i in range(GA):
                ids = batches[(step - 1) * GA + i][:, :-1].contiguous().to(DEV)
                l = model(input_ids=ids, labels=ids, return_logits=False).loss
                losses.append(float(l.detach()))
                l.backward(gradient=seed)
            norm = float(scaler.unscale_(opt, 1.0))
            if math.isfinite(norm):
                break
            assert scaler.step(opt, norm) is False
            scaler.update()
            overflows.append(step)
        opt.discard_step()
        g = torch.cat([p.grad.double().reshape(-1).cpu() for p in model.parameters()]) / scaler.scale_value()
        rel.append(abs(sum(losses) / GA - loss) / abs(loss))
        ref = torch.cat([grads[n].double().reshape(-1).cpu() for n in order])
        cos.append(float(F.cosine_similarity(g, ref, dim=0)))
        norm_rel.append(abs(norm - float(g.norm())) / float(g.norm()))

    OE.train_reference(_ocfg(cfg), P, iter(batches), steps=steps, grad_accum_steps=GA, lr=3e-4, betas=(0.9, 0.95),
                       weight_decay=0.1, max_grad_norm=1.0, loss_chunk_size=128, on_step=on_step, param_dtype=H16)
    print("per-step grad cosine:", " ".join(f"{c:.5f}" for c in cos))
    print(f"overflowing scales at steps {overflows}, final scale {scaler.scale_value()}")
    assert len(cos) == steps and max(rel) <= 1e-2 and min(cos) >= 0.999
    assert max(norm_rel) < 1e-3


def test_loss_scaler_skips_overflow_and_backs_off():
    """A scale large enough to overflow fp16 gradients gives an inf/NaN norm:
    the step is skipped (parameters unchanged), the scale halves; with a
    finite norm the step runs, reports the unscaled norm and moves the
    parameters as FusedAdamW's step on unscaled gradients does."""
    cfg = build_config("plumbing", vocab_size=32000, max_seq_len=64)
    torch.manual_seed(1)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=H16)
    opt = FusedAdamW(model.parameters(), lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1)
    ids = torch.randint(0, cfg.vocab_size, (2, 64), generator=torch.Generator().manual_seed(2)).to(DEV)
    scaler = LossScaler(init_scale=2.0 ** 40)
    before = [p.detach().clone() for p in model.parameters()]
    loss = model(input_ids=ids, labels=ids, return_logits=False).loss
    loss.backward(gradient=torch.full((), scaler.scale_value(), dtype=torch.float32, device=DEV))
    norm = float(scaler.unscale_(opt, 1.0))
    assert not math.isfinite(norm)
    assert scaler.step(opt, norm) is False
    scaler.update()
    assert scaler.scale_value() == 2.0 ** 39
    assert all(torch.equal(a, p) for a, p in zip(before, model.parameters()))
    # a finite scale: the same update as stepping on the unscaled gradients
    twin = LlamaForCausalLM(cfg).to(device=DEV, dtype=H16)
    twin.load_state_dict(model.state_dict())
    start = torch.cat([p.detach().double().reshape(-1) for p in model.parameters()])
    topt = FusedAdamW(twin.parameters(), lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1)
    s = 2.0 ** 8
    model.zero_grad(set_to_none=True)
    model(input_ids=ids, labels=ids, return_logits=False).loss.backward(
        gradient=torch.full((), s, dtype=torch.float32, device=DEV))
    twin(input_ids=ids, labels=ids, return_logits=False).loss.backward()
    sc = LossScaler(init_scale=s)
    n1 = float(sc.unscale_(opt, 0.0))
    assert sc.step(opt, n1)
    n2 = float(topt.clip_grad_norm_(0.0))
    topt.step()
    assert abs(n1 - n2) <= 2e-3 * n2
    # Adam's first step moves every element by about lr * sign(g), so compare
    # the update directions (elements whose tiny gradients differ in sign
    # between the scaled and the unscaled fp16 backward move oppositely)
    d1 = torch.cat([p.detach().double().reshape(-1) for p in model.parameters()]) - start
    d2 = torch.cat([p.detach().double().reshape(-1) for p in twin.parameters()]) - start
    assert float(F.cosine_similarity(d1, d2, dim=0)) > 0.99


def test_train_py_float16_cli(tmp_path):
    """train.py --dtype float16 (the reference's GradScaler path) runs and
    prints finite step lines."""
    env = dict(os.environ)
    pkg = ROOT / "cs244c-llama-zero_amd"
    env["PYTHONPATH"] = f"{pkg}:{ROOT}:" + env.get("PYTHONPATH", "")
    cmd = [sys.executable, "train.py", "--model-size", "plumbing", "--data-mode", "synthetic-uniform",
           "--synthetic-vocab-size", "32000", "--batch-size", "2", "--seq-len", "64", "--grad-accum-steps", "2",
           "--max-steps", "6", "--log-interval", "1", "--dtype", "float16", "--save-dir", str(tmp_path),
           "--checkpoint-interval", "0"]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=300, cwd=str(pkg), env=env)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    losses = [float(m) for m in re.findall(r"\[step\s+\d+\]\s+loss=(\S+)", proc.stdout)]
    assert len(losses) == 6 and all(math.isfinite(x) for x in losses), proc.stdout
    assert "dtype=float16" in proc.stdout
