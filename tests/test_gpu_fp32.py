"""The float32 path on the GPU: the fp32 MFMA GEMM and the models and
trainers run in float32 (the reference's `--dtype float32`: train.py:148-160,
train_zero.py:74,150-164).

Tolerances:
  - fp32 GEMM: 1e-5 relative (Frobenius) to the float64 product;
  - fp32 model forward/backward: loss 1e-5 relative to the float64 oracle,
    per-parameter gradient cosine >= 0.99999;
  - the train.py workload (plumbing model, B=4 S=128 GA=2, clip 1.0) in fp32
    for 100 steps against the oracle's train.py loop in fp32: teacher-forced
    (the oracle's parameters loaded each step) loss within 1e-4 relative and
    gradient cosine >= 0.9999 at every step.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from lzhip import ops
from lzhip.functional import GradSink
from model import LlamaForCausalLM, ModelConfig, build_config
from oracle import data as OD
from oracle import engine as OE
from oracle import model as OM

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "cs244c-llama-zero_amd"
STEP_RE = re.compile(r"\[step\s+(\d+)\]\s+loss=([0-9.]+).*tokens/s=([0-9,]+)")


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _operand(t: torch.Tensor, kmajor: bool) -> torch.Tensor:
    """t is [R, K]; the stored operand is t itself (K-major) or t^T laid
    out contiguously ([K, R], R-major)."""
    return t if kmajor else t.t().contiguous()


@pytest.mark.parametrize("ak,bk", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (37, 29, 13), (128, 128, 32), (300, 200, 72), (515, 257, 1031),
                                   (1024, 768, 2048), (256, 5632, 2048), (200, 100, 5000), (512, 256, 32000)])
def test_gemm_f32_layouts_vs_float64(ak, bk, M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K + 2 * ak + bk)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(N, K, generator=g)
    ref = a.double() @ b.double().t()
    out = ops.gemm(_operand(a, ak).to(DEV), _operand(b, bk).to(DEV), ak, bk)
    assert out.dtype == torch.float32 and out.shape == (M, N)
    assert _rel(out, ref) <= 1e-5


def test_gemm_f32_split_plan():
    """Few output tiles with a long K (a language-model head's input
    gradient: 512 tokens x 256 features over a 32000 vocabulary) are split
    along K; large products are not."""
    from lzhip import _lib

    lib = _lib.load()
    assert lib.lz_gemm_f32_plan(512, 256, 32000) >= 16
    assert lib.lz_gemm_f32_workspace(512, 256, 32000) == lib.lz_gemm_f32_plan(512, 256, 32000) * 512 * 256 * 4
    assert lib.lz_gemm_f32_plan(333, 190, 517) > 1      # the epilogue test below runs split
    assert lib.lz_gemm_f32_plan(4096, 4096, 4096) == 1 and lib.lz_gemm_f32_workspace(4096, 4096, 4096) == 0
    assert lib.lz_gemm_f32_plan(64, 64, 64) == 1


def test_gemm_f32_epilogue_and_views():
    g = torch.Generator().manual_seed(5)
    M, N, K = 333, 190, 517
    big = torch.randn(M, K + 7, generator=g)            # row stride K + 7: scalar loads
    a = big[:, 3:3 + K]
    b = torch.randn(N, K, generator=g)
    r = torch.randn(M, N, generator=g)
    c0 = torch.randn(M, N + 5, generator=g)[:, :N]      # strided output view
    ab = a.double() @ b.double().t()
    out = ops.gemm(a.to(DEV), b.to(DEV), residual=r.to(DEV))
    assert _rel(out, ab + r.double()) <= 1e-5
    cd = c0.to(DEV)
    ops.gemm(a.to(DEV), b.to(DEV), out=cd, alpha=0.5, beta=-2.0)
    assert _rel(cd, 0.5 * ab - 2.0 * c0.double()) <= 1e-5
    # bf16 output: one bf16 rounding of the fp32 product
    o16 = ops.gemm(a.to(DEV), b.to(DEV), out_dtype=torch.bfloat16)
    assert o16.dtype == torch.bfloat16
    assert torch.allclose(o16.double().cpu(), ab, rtol=2 ** -8, atol=1e-5)
    # K = 0: C = beta * C + R
    z = ops.gemm(torch.empty(4, 0, device=DEV), torch.empty(3, 0, device=DEV), residual=torch.ones(4, 3, device=DEV))
    assert torch.equal(z.cpu(), torch.ones(4, 3))
    with pytest.raises(TypeError):
        ops.gemm(a.to(DEV), b.to(DEV).to(torch.bfloat16))


def _ocfg(cfg: ModelConfig) -> OM.Cfg:
    return OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                  n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta,
                  rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings)


@pytest.mark.parametrize(
    "dim,H,KV,ffn,L,V,B,S,chunk",
    [
        (256, 8, 4, 688, 2, 32000, 4, 128, 128),   # the train.py plumbing layout (head dim 32)
        (768, 12, 4, 2048, 1, 32000, 2, 256, 0),   # the 125M layout (head dim 64)
        (512, 4, 2, 1024, 1, 1000, 1, 200, 0),     # head dim 128, ragged sequence, odd vocab
    ],
)
def test_fp32_model_vs_oracle(dim, H, KV, ffn, L, V, B, S, chunk):
    cfg = ModelConfig(name="f32", vocab_size=V, max_seq_len=S, dim=dim, n_layers=L, n_heads=H, n_kv_heads=KV,
                      ffn_dim=ffn, rope_theta=10_000.0)
    torch.manual_seed(dim + S)
    model = LlamaForCausalLM(cfg).to(DEV)
    assert next(model.parameters()).dtype == torch.float32
    model.set_loss_chunk_size(chunk)
    P = {k: v.detach().double().cpu().requires_grad_(True) for k, v in model.state_dict().items()
         if k != "lm_head.weight"}
    ids = torch.randint(0, V, (B, S), generator=torch.Generator().manual_seed(S))
    out = model(input_ids=ids.to(DEV), labels=ids.to(DEV), return_logits=False)
    out.loss.backward()
    ref = OM.loss(P, _ocfg(cfg), ids, chunk_size=chunk)
    ref.backward()
    assert abs(float(out.loss.detach()) - float(ref.detach())) <= 1e-5 * abs(float(ref.detach()))
    worst = min((float(F.cosine_similarity(p.grad.double().cpu().view(-1), P[n].grad.view(-1), dim=0)), n)
                for n, p in model.named_parameters())
    assert worst[0] >= 0.99999, worst


def test_plumbing_fp32_100_steps_vs_oracle():
    """The train.py workload in float32, as the reference's CPU run is:
    every step, the HIP path (FusedAdamW on fp32 parameters) is given the
    oracle trainer's current parameters and must reproduce its loss and
    gradient; the free-running HIP trainer must track the oracle's loss."""
    from lzhip.optim import FusedAdamW

    steps, B, S, GA = 100, 4, 128, 2
    cfg = build_config("plumbing", vocab_size=32000, max_seq_len=S)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg)
    P = {k: v.detach().clone() for k, v in model.state_dict().items() if k != "lm_head.weight"}
    order = [n for n, _ in model.named_parameters()]
    model = model.to(DEV)
    model.set_loss_chunk_size(128)
    free = LlamaForCausalLM(cfg).to(DEV)
    free.load_state_dict(model.state_dict())
    free.set_loss_chunk_size(128)
    opt = FusedAdamW(free.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    sink = GradSink(free)  # the free-running trainer accumulates as train.py does
    seed = torch.full((), 1.0 / GA, device=DEV)
    batches = []
    gen = OD.uniform_chunks(S, cfg.vocab_size, B, seed=0)
    for _ in range(steps * GA):
        batches.append(next(gen))
    rel, cos, free_rel = [], [], []

    def on_step(step, loss, gn, grads, params):
        with torch.no_grad():
            model.load_state_dict({k: v.to(DEV) for k, v in params.items()}, strict=False)
        model.zero_grad(set_to_none=True)
        sink.begin_step()
        losses, flosses = [], []
        for i in range(GA):
            ids = batches[(step - 1) * GA + i][:, :-1].contiguous().to(DEV)
            l = model(input_ids=ids, labels=ids, return_logits=False).loss
            losses.append(float(l.detach()))
            (l / GA).backward()
            fl = free(input_ids=ids, labels=ids, return_logits=False).loss
            flosses.append(float(fl.detach()))
            fl.backward(gradient=seed)
        sink.finish()
        opt.clip_grad_norm_(1.0)
        opt.step()
        g = torch.cat([p.grad.double().reshape(-1).cpu() for p in model.parameters()])
        r = torch.cat([grads[n].double().reshape(-1) for n in order])
        # the oracle hands over clipped gradients; compare directions
        rel.append(abs(sum(losses) / GA - loss) / abs(loss))
        cos.append(float(F.cosine_similarity(g, r, dim=0)))
        free_rel.append(abs(sum(flosses) / GA - loss) / abs(loss))

    OE.train_reference(_ocfg(cfg), P, iter(batches), steps=steps, grad_accum_steps=GA, lr=3e-4, betas=(0.9, 0.95),
                       weight_decay=0.1, max_grad_norm=1.0, loss_chunk_size=128, on_step=on_step)
    print(f"teacher-forced: max loss rel {max(rel):.2e}, min grad cosine {min(cos):.7f}; "
          f"free-running: max loss rel {max(free_rel):.2e}")
    assert len(cos) == steps
    assert max(rel) <= 1e-4
    assert min(cos) >= 0.9999
    assert max(free_rel) <= 1e-3


def _run(args, timeout=600):
    env = dict(os.environ)
    env["PYTHONPATH"] = f"{PKG}:{ROOT}:" + env.get("PYTHONPATH", "")
    proc = subprocess.run([sys.executable, *args], cwd=str(PKG), env=env, capture_output=True, text=True,
                          timeout=timeout)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-3000:]
    return proc.stdout


def test_train_zero_cli_reference_defaults(tmp_path):
    """train_zero.py with the reference's defaults (--dtype float32, ZeRO
    stage 0) runs on the GPU: three finite step lines."""
    out = _run(["train_zero.py", "--model-size", "plumbing", "--data-mode", "synthetic-uniform",
                "--synthetic-vocab-size", "32000", "--seq-len", "128", "--batch-size", "4", "--max-steps", "3",
                "--log-interval", "1", "--save-dir", str(tmp_path)])
    steps = STEP_RE.findall(out)
    assert len(steps) == 3, out
    assert all(float(loss) > 0 and float(loss) < 20 for _, loss, _ in steps)
    assert "dtype=float32" in out


def test_train_py_cli_fp32(tmp_path):
    out = _run(["train.py", "--model-size", "plumbing", "--dtype", "float32", "--data-mode", "synthetic-uniform",
                "--synthetic-vocab-size", "32000", "--seq-len", "128", "--batch-size", "4", "--grad-accum-steps", "2",
                "--max-steps", "3", "--seed", "0", "--log-interval", "1", "--save-dir", str(tmp_path)])
    assert len(STEP_RE.findall(out)) == 3, out
    payload = torch.load(tmp_path / "step_000003.pt", map_location="cpu", weights_only=True)
    assert all(v.dtype == torch.float32 for v in payload["model_state_dict"].values())
