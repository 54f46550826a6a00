"""Model-level parity on the GPU: the HIP forward/backward of
LlamaForCausalLM in bf16 against the float64 CPU oracle evaluated at the same
(bf16-rounded) parameters.

Tolerances (bf16 training bar): loss within 1e-2 relative, per-parameter
gradient cosine similarity >= 0.999.  The oracle uses bf16 RoPE angles, which
is what the reference computes once Module.to(bfloat16) has cast its inv_freq
buffer.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from model import LlamaForCausalLM, ModelConfig
from oracle import model as OM

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _ocfg(cfg: ModelConfig, angle=torch.bfloat16) -> OM.Cfg:
    return OM.Cfg(vocab_size=cfg.vocab_size, dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
                  n_kv_heads=cfg.n_kv_heads, ffn_dim=cfg.ffn_dim, rope_theta=cfg.rope_theta,
                  rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings, rope_angle_dtype=angle)


def _oracle_params(model: LlamaForCausalLM):
    return {k: v.detach().double().cpu().requires_grad_(True) for k, v in model.state_dict().items()
            if not (k == "lm_head.weight" and model.cfg.tie_word_embeddings)}


def _compare(model, P, ocfg, ids, chunk):
    out = model(input_ids=ids.to(DEV), labels=ids.to(DEV), return_logits=False)
    out.loss.backward()
    ref = OM.loss(P, ocfg, ids, chunk_size=chunk)
    ref.backward()
    loss, rloss = float(out.loss.detach()), float(ref.detach())
    assert abs(loss - rloss) <= 1e-2 * abs(rloss), (loss, rloss)
    worst = (1.0, "")
    for name, p in model.named_parameters():
        g = p.grad.detach().double().cpu().view(-1)
        r = P[name].grad.view(-1)
        cos = float(F.cosine_similarity(g, r, dim=0))
        worst = min(worst, (cos, name))
    assert worst[0] >= 0.999, worst
    return loss, rloss, worst


@pytest.mark.parametrize(
    "dim,H,KV,L,V,B,S,chunk",
    [
        (128, 4, 2, 2, 256, 2, 64, 0),      # hd 32: generic attention path
        (256, 4, 2, 2, 512, 2, 128, 128),   # hd 64 MFMA, chunked loss
        (512, 4, 2, 2, 1000, 2, 256, 0),    # hd 128 MFMA, odd vocab
        (768, 12, 4, 2, 32000, 2, 300, 0),  # 125M head layout, ragged sequence
    ],
)
def test_forward_backward_vs_oracle(dim, H, KV, L, V, B, S, chunk):
    cfg = ModelConfig(name="t", vocab_size=V, max_seq_len=S, dim=dim, n_layers=L, n_heads=H, n_kv_heads=KV,
                      ffn_dim=dim * 2, rope_theta=10_000.0)
    torch.manual_seed(dim + S)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    model.set_loss_chunk_size(chunk)
    P = _oracle_params(model)
    ids = torch.randint(0, V, (B, S), generator=torch.Generator().manual_seed(S))
    _compare(model, P, _ocfg(cfg), ids, chunk)


@pytest.mark.parametrize("chunk", [0, 128])
def test_fused_lm_head_loss_matches_unfused(chunk):
    """The fused LM-head + loss (logits formed one sequence at a time here, so
    several chunks) against the unfused LM head + cross entropy, with ignored
    targets in the labels: same loss, same gradients up to the fp32
    summation order of the chunked dW."""
    cfg = ModelConfig(name="t", vocab_size=1000, dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=688,
                      max_seq_len=128)
    torch.manual_seed(3)
    ma = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    mb = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    mb.load_state_dict(ma.state_dict())
    for m in (ma, mb):
        m.set_loss_chunk_size(chunk)
    ma.fused_lm_head_loss = True
    ma.lm_head.fused_chunk_bytes = 128 * 1000 * 2  # one sequence of logits per chunk
    mb.fused_lm_head_loss = False
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 1000, (3, 128), generator=g)
    labels = ids.clone()
    labels[0, 10:20] = -100
    labels[2, 100:] = -100
    out_a = ma(input_ids=ids.to(DEV), labels=labels.to(DEV), return_logits=False)
    out_b = mb(input_ids=ids.to(DEV), labels=labels.to(DEV), return_logits=False)
    assert out_a.logits is None
    (0.5 * out_a.loss).backward()
    (0.5 * out_b.loss).backward()
    la, lb = float(out_a.loss.detach()), float(out_b.loss.detach())
    assert abs(la - lb) <= 1e-6 * abs(lb), (la, lb)
    with torch.no_grad():  # the no-grad pass forms no gradients and gives the same loss
        assert float(ma(input_ids=ids.to(DEV), labels=labels.to(DEV), return_logits=False).loss.detach()) == la
    for (n, pa), (_, pb) in zip(ma.named_parameters(), mb.named_parameters()):
        ga, gb = pa.grad.double().view(-1), pb.grad.double().view(-1)
        assert float(F.cosine_similarity(ga, gb, dim=0)) >= 0.9999, n
        assert float((ga - gb).norm() / gb.norm()) <= 1e-2, n


def test_reference_golden_config_in_bf16():
    """The reference's golden case (seed 123, chunk 4) through the HIP path in
    bf16: within 1e-2 of 4.901787757873535."""
    cfg = ModelConfig(name="unit_test", vocab_size=128, max_seq_len=16, dim=64, n_layers=2, n_heads=4, n_kv_heads=2,
                      ffn_dim=128)
    torch.manual_seed(123)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    model.set_loss_chunk_size(4)
    ids = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7, 9, 3], [2, 7, 1, 8, 2, 8, 1, 8, 2, 8, 4, 5, 9, 0, 4, 5]])
    out = model(input_ids=ids.to(DEV), labels=ids.to(DEV), return_logits=False)
    assert out.logits is None
    assert abs(float(out.loss.detach()) - 4.901787757873535) <= 1e-2 * 4.901787757873535


def test_logits_and_causality():
    cfg = ModelConfig(name="t", vocab_size=300, max_seq_len=64, dim=256, n_layers=2, n_heads=4, n_kv_heads=2,
                      ffn_dim=512, rope_theta=10_000.0)
    torch.manual_seed(2)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16).eval()
    a = torch.randint(0, 300, (1, 64), generator=torch.Generator().manual_seed(1))
    b = a.clone()
    b[0, -1] = (b[0, -1] + 7) % 300
    with torch.no_grad():
        la = model(a.to(DEV)).logits
        lb = model(b.to(DEV)).logits
    assert la.shape == (1, 64, 300)
    assert torch.equal(la[:, :-1], lb[:, :-1])
    P = _oracle_params(model)
    ref = OM.logits({k: v.detach() for k, v in P.items()}, _ocfg(cfg), a)
    assert float((la.double().cpu() - ref).norm() / ref.norm()) < 2e-2


def test_activation_checkpointing_matches_plain():
    cfg = ModelConfig(name="t", vocab_size=256, max_seq_len=128, dim=256, n_layers=3, n_heads=4, n_kv_heads=2,
                      ffn_dim=512, rope_theta=10_000.0)
    torch.manual_seed(9)
    m1 = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    m2 = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    m2.load_state_dict(m1.state_dict())
    m2.set_activation_checkpointing(True)
    ids = torch.randint(0, 256, (2, 128), generator=torch.Generator().manual_seed(3)).to(DEV)
    l1 = m1(ids, labels=ids).loss
    l2 = m2(ids, labels=ids).loss
    assert float(l1.detach()) == float(l2.detach())
    l1.backward()
    l2.backward()
    for (n, p1), (_, p2) in zip(m1.named_parameters(), m2.named_parameters()):
        assert torch.allclose(p1.grad.float(), p2.grad.float(), rtol=1e-2, atol=1e-4), n


def test_unsupported_dtype_is_refused_clearly():
    cfg = ModelConfig(name="t", vocab_size=64, max_seq_len=16, dim=64, n_layers=1, n_heads=2, n_kv_heads=1,
                      ffn_dim=128)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.float64)
    with pytest.raises(TypeError, match="float32, bfloat16 and float16"):
        model(torch.zeros(1, 16, dtype=torch.long, device=DEV))


def test_generate_runs():
    """generate (model/llama.py:311-335): greedy tokens are the arg-max of the
    model's last logits over the last max_seq_len tokens (the window slides
    once the sequence outgrows it); top_k=1 sampling is greedy; a seeded
    sampling run repeats."""
    cfg = ModelConfig(name="t", vocab_size=64, max_seq_len=32, dim=128, n_layers=1, n_heads=2, n_kv_heads=1,
                      ffn_dim=256, rope_theta=10_000.0)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    prompt = torch.randint(0, 64, (2, 29), generator=torch.Generator().manual_seed(1)).to(DEV)
    out = model.generate(prompt, max_new_tokens=6, temperature=0.0)
    assert out.shape == (2, 35) and torch.equal(out[:, :29], prompt)
    with torch.no_grad():
        for t in range(29, 35):
            ctx = out[:, max(0, t - 32) : t].contiguous()
            assert torch.equal(out[:, t], model(ctx).logits[:, -1, :].float().argmax(dim=-1))
    assert torch.equal(model.generate(prompt, 6, temperature=0.7, top_k=1), out)
    torch.manual_seed(5)
    s1 = model.generate(prompt, 4, temperature=1.0, top_k=10)
    torch.manual_seed(5)
    s2 = model.generate(prompt, 4, temperature=1.0, top_k=10)
    assert torch.equal(s1, s2) and s1.shape == (2, 33)


@pytest.mark.parametrize("stage3", [False, True])
def test_model_with_attention_mask(stage3):
    """The model called with attention_mask (model/llama.py:203-216 ->
    SDPA attn_mask): an explicit causal mask gives the causal model's loss
    and gradients (the masked kernels accumulate in another order: bf16
    bars), a padding mask changes the loss and keeps everything finite; the
    same through the ZeRO-3 executor, which carries the mask into its
    recompute."""
    from zero import ZeROStage3Optimizer

    cfg = ModelConfig(name="mask", vocab_size=1000, max_seq_len=64, dim=256, n_layers=2, n_heads=8, n_kv_heads=4,
                      ffn_dim=512)
    torch.manual_seed(5)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    B, S = 2, 64
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(1)).to(DEV)
    causal = ~torch.triu(torch.ones(S, S, dtype=torch.bool, device=DEV), 1)
    pad = causal.expand(B, 1, S, S).clone()
    pad[1, :, :, S // 2:] = False
    pad[..., 0] = True
    engine = ZeROStage3Optimizer(model=model, lr=1e-3) if stage3 else None

    def run(mask):
        if engine is not None:
            engine.zero_grad()
            engine.prepare_forward()
        else:
            model.zero_grad(set_to_none=True)
        loss = model(input_ids=ids, labels=ids, attention_mask=mask, return_logits=False).loss
        if engine is not None:
            engine.backward(loss)
            g = engine._grad_all.detach().double().cpu().clone()  # every handle's fp32 gradient shard
        else:
            loss.backward()
            g = torch.cat([p.grad.double().reshape(-1).cpu() for p in model.parameters()])
        return float(loss.detach()), g

    l0, g0 = run(None)
    l1, g1 = run(causal)
    assert abs(l1 - l0) <= 1e-2 * abs(l0)
    assert float(F.cosine_similarity(g0, g1, dim=0)) >= 0.999
    l2, g2 = run(pad)
    assert torch.isfinite(torch.tensor(l2)) and abs(l2 - l0) > 1e-4
    assert bool(torch.isfinite(g2).all())


def _record_dropout_keys(monkeypatch):
    """Records the stream key of every dropout call the model makes."""
    from lzhip import ops

    keys = []
    draw = ops.dropout_seed

    def recording(device):
        k = draw(device)
        keys.append(k)
        return k

    monkeypatch.setattr(ops, "dropout_seed", recording)
    return keys


def _oracle_drop(cfg: ModelConfig, keys, B: int, S: int):
    """The keep masks the model's dropout calls used, in call order: token
    embeddings, then per layer attention probabilities and MLP activations."""
    from lzhip import ops

    p = cfg.dropout
    assert len(keys) == 1 + 2 * cfg.n_layers
    mask = lambda k, shape: ops.dropout_mask(math.prod(shape), p, k, DEV).cpu().view(shape).bool()
    drop = {"p": p, "embed": mask(keys[0], (B, S, cfg.dim))}
    for i in range(cfg.n_layers):
        drop[(i, "attn")] = mask(keys[1 + 2 * i], (B, cfg.n_heads, S, S))
        drop[(i, "mlp")] = mask(keys[2 + 2 * i], (B, S, cfg.ffn_dim))
    return drop


@pytest.mark.parametrize("dim,H,KV,S", [(128, 4, 2, 64), (256, 4, 2, 96)])
def test_model_dropout_vs_oracle(monkeypatch, dim, H, KV, S):
    """Training-mode dropout (model/llama.py:107-115 attention, :146 MLP,
    :213 embeddings) against the float64 oracle given the keep masks the
    model's calls drew: loss within 1e-2, gradients cosine >= 0.999."""
    cfg = ModelConfig(name="drop", vocab_size=300, max_seq_len=S, dim=dim, n_layers=2, n_heads=H, n_kv_heads=KV,
                      ffn_dim=2 * dim, rope_theta=10_000.0, dropout=0.2)
    torch.manual_seed(dim + S)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16)
    model.train()
    P = _oracle_params(model)
    B = 2
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(S))
    keys = _record_dropout_keys(monkeypatch)
    out = model(input_ids=ids.to(DEV), labels=ids.to(DEV), return_logits=False)
    out.loss.backward()
    drop = _oracle_drop(cfg, keys, B, S)
    ref = OM.loss(P, _ocfg(cfg), ids, drop=drop)
    ref.backward()
    assert abs(float(out.loss.detach()) - float(ref.detach())) <= 1e-2 * abs(float(ref.detach()))
    nodrop = OM.loss({k: v.detach() for k, v in P.items()}, _ocfg(cfg), ids)
    assert abs(float(nodrop) - float(ref.detach())) > 1e-4 * abs(float(ref.detach()))  # the masks matter
    for name, prm in model.named_parameters():
        cos = float(F.cosine_similarity(prm.grad.detach().double().cpu().view(-1), P[name].grad.view(-1), dim=0))
        assert cos >= 0.999, (name, cos)


def test_model_dropout_replay_and_eval():
    """torch.manual_seed replays a dropout forward bit for bit, activation
    checkpointing's recompute replays the masks (same loss bits, gradients
    as without it), eval mode and dropout=0 skip dropout."""
    kw = dict(name="drop", vocab_size=256, max_seq_len=128, dim=256, n_layers=3, n_heads=4, n_kv_heads=2,
              ffn_dim=512, rope_theta=10_000.0)
    torch.manual_seed(9)
    m1 = LlamaForCausalLM(ModelConfig(dropout=0.1, **kw)).to(device=DEV, dtype=torch.bfloat16)
    m2 = LlamaForCausalLM(ModelConfig(dropout=0.1, **kw)).to(device=DEV, dtype=torch.bfloat16)
    m0 = LlamaForCausalLM(ModelConfig(dropout=0.0, **kw)).to(device=DEV, dtype=torch.bfloat16)
    m2.load_state_dict(m1.state_dict())
    m0.load_state_dict(m1.state_dict())
    m2.set_activation_checkpointing(True)
    ids = torch.randint(0, 256, (2, 128), generator=torch.Generator().manual_seed(3)).to(DEV)
    torch.manual_seed(100)
    l1 = m1(ids, labels=ids).loss
    torch.manual_seed(100)
    l2 = m2(ids, labels=ids).loss
    assert float(l1.detach()) == float(l2.detach())
    l1.backward()
    l2.backward()
    for (n, p1), (_, p2) in zip(m1.named_parameters(), m2.named_parameters()):
        assert torch.allclose(p1.grad.float(), p2.grad.float(), rtol=1e-2, atol=1e-4), n
    torch.manual_seed(100)
    again = m1(ids, labels=ids).loss
    other = m1(ids, labels=ids).loss
    base = m0(ids, labels=ids).loss
    m1.eval()
    ev = m1(ids, labels=ids).loss
    assert float(again.detach()) == float(l1.detach()) and float(other.detach()) != float(l1.detach())
    assert float(ev.detach()) == float(base.detach()) and float(ev.detach()) != float(l1.detach())
