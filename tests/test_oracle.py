"""Pins the CPU oracle before anything is compared against it (CPU only).

Each oracle function is checked against a value the reference itself holds
(the golden loss), a library routine computing the same quantity, or an
invariant/closed form that a plausible mistake would break.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import data as OD
from oracle import engine as OE
from oracle import flat as OF
from oracle import model as OM
from oracle import ops as R


def tiny_cfg(**kw) -> OM.Cfg:
    # tests/test_model.py:7-18 of the reference
    base = dict(vocab_size=128, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128)
    base.update(kw)
    return OM.Cfg(**base)


GOLDEN_IDS = torch.tensor(
    [[3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7, 9, 3], [2, 7, 1, 8, 2, 8, 1, 8, 2, 8, 4, 5, 9, 0, 4, 5]]
)


@pytest.mark.parametrize("attn_impl", ["sdpa", "explicit"])
def test_golden_chunked_loss(attn_impl):
    """reference tests/test_model.py:46-64: seed 123, chunk 4 -> 4.901787757873535."""
    cfg = tiny_cfg()
    torch.manual_seed(123)
    P = OM.init_params(cfg)
    loss = OM.loss(P, cfg, GOLDEN_IDS, chunk_size=4, attn_impl=attn_impl)
    torch.testing.assert_close(loss.detach(), torch.tensor(4.901787757873535), atol=1e-6, rtol=0.0)


def test_golden_breaks_under_planted_mistakes():
    """A wrong init order, RoPE sign or missing residual moves the golden loss."""
    cfg = tiny_cfg()
    torch.manual_seed(123)
    P = OM.init_params(cfg)
    good = float(OM.loss(P, cfg, GOLDEN_IDS, chunk_size=4))
    bad = dict(P)
    bad["layers.0.attn.q_proj.weight"], bad["layers.0.attn.k_proj.weight"] = (
        P["layers.0.attn.k_proj.weight"].repeat(2, 1), P["layers.0.attn.q_proj.weight"][:32])
    assert abs(float(OM.loss(bad, cfg, GOLDEN_IDS, chunk_size=4)) - good) > 1e-4
    orig = R.rotate_half
    try:
        R.rotate_half = lambda x: torch.cat((x[..., x.shape[-1] // 2:], -x[..., : x.shape[-1] // 2]), dim=-1)
        assert abs(float(OM.loss(P, cfg, GOLDEN_IDS, chunk_size=4)) - good) > 1e-4
    finally:
        R.rotate_half = orig


def test_chunked_equals_full_loss_and_grads():
    cfg = tiny_cfg()
    torch.manual_seed(5)
    P = {k: v.requires_grad_(True) for k, v in OM.init_params(cfg).items()}
    x = torch.randint(0, cfg.vocab_size, (2, 16))
    full = OM.loss(P, cfg, x, chunk_size=0)
    g_full = torch.autograd.grad(full, list(P.values()))
    chunked = OM.loss(P, cfg, x, chunk_size=4)
    g_ch = torch.autograd.grad(chunked, list(P.values()))
    torch.testing.assert_close(full, chunked, atol=1e-5, rtol=1e-5)
    for a, b in zip(g_full, g_ch):
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)
    # the explicit restatement of the loss agrees with F.cross_entropy
    lg = OM.logits(P, cfg, x)
    torch.testing.assert_close(R.shifted_cross_entropy(lg, x), full, atol=1e-6, rtol=1e-6)


def test_causal_mask_blocks_future():
    cfg = tiny_cfg()
    torch.manual_seed(1)
    P = OM.init_params(cfg)
    a = torch.tensor([[1, 2, 3, 4, 5, 6, 7, 8]])
    b = a.clone()
    b[0, -1] = 99
    la, lb = OM.logits(P, cfg, a), OM.logits(P, cfg, b)
    torch.testing.assert_close(la[:, :-1], lb[:, :-1], atol=1e-6, rtol=1e-5)
    assert not torch.allclose(la[:, -1], lb[:, -1])


def test_rope_norm_preserving_and_relative():
    hd, S = 32, 40
    cos, sin = R.rope_tables(S, hd, 500_000.0)
    q = torch.randn(2, 4, S, hd, dtype=torch.float64)
    k = torch.randn(2, 4, S, hd, dtype=torch.float64)
    qr = R.apply_rope(q, cos.double(), sin.double())
    torch.testing.assert_close(q.norm(dim=-1), qr.norm(dim=-1), atol=1e-5, rtol=1e-4)
    # <rope(q)_i, rope(k)_j> depends on i - j only
    c64, s64 = R.rope_tables(S, hd, 10_000.0)
    v = torch.randn(hd, dtype=torch.float64)
    w = torch.randn(hd, dtype=torch.float64)
    rq = R.apply_rope(v.expand(S, hd), c64.double(), s64.double())
    rk = R.apply_rope(w.expand(S, hd), c64.double(), s64.double())
    assert abs(float(rq[10] @ rk[7]) - float(rq[25] @ rk[22])) < 1e-5
    assert abs(float(rq[10] @ rk[7]) - float(rq[10] @ rk[8])) > 1e-3


def test_rope_bf16_angle_tables_follow_bf16_arithmetic():
    cos, _ = R.rope_tables(1024, 64, 10_000.0, angle_dtype=torch.bfloat16)
    # bf16 positions: 1022 and 1023 round to 1024, 1021 to 1020
    assert torch.equal(cos[1022], cos[1023])
    assert not torch.equal(cos[1021], cos[1022])
    c32, _ = R.rope_tables(1024, 64, 10_000.0)
    assert not torch.equal(c32[1022], c32[1023])


@pytest.mark.parametrize("H,KV", [(4, 2), (4, 4), (8, 1)])
def test_attention_matches_sdpa(H, KV):
    g = torch.Generator().manual_seed(H * 10 + KV)
    q = torch.randn(2, H, 33, 16, generator=g, dtype=torch.float64)
    k = torch.randn(2, KV, 33, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, KV, 33, 16, generator=g, dtype=torch.float64)
    out = R.causal_gqa_attention(q, k, v)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(H // KV, 1), v.repeat_interleave(H // KV, 1),
                                         is_causal=True)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)


def test_rmsnorm_swiglu_ce_match_library():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 48, generator=g, dtype=torch.float64)
    w = torch.randn(48, generator=g, dtype=torch.float64)
    torch.testing.assert_close(R.rmsnorm(x, w, 1e-5), F.rms_norm(x, (48,), w, eps=1e-5))
    a, b = torch.randn(9, 11, generator=g, dtype=torch.float64), torch.randn(9, 11, generator=g, dtype=torch.float64)
    torch.testing.assert_close(R.swiglu(a, b), F.silu(a) * b)
    lg = torch.randn(3, 10, 50, generator=g, dtype=torch.float64)
    lab = torch.randint(0, 50, (3, 10), generator=g)
    lab[1, 4] = -100
    ref = F.cross_entropy(lg[:, :-1].transpose(1, 2), lab[:, 1:], ignore_index=-100)
    torch.testing.assert_close(R.shifted_cross_entropy(lg, lab), ref)
    none = torch.full((3, 10), -100)
    assert float(R.shifted_cross_entropy(lg, none, clamp=True)) == 0.0
    assert math.isnan(float(R.shifted_cross_entropy(lg, none, clamp=False)))


@pytest.mark.parametrize("max_norm", [0.0, 0.05, 1e9])
def test_engine_update_matches_torch_adamw(max_norm):
    """EngineRef (zero/stage0_ddp.py:66-88 order) vs torch.optim.AdamW +
    clip_grad_norm_ over 6 steps."""
    g = torch.Generator().manual_seed(3)
    n = 1000
    p0 = 0.02 * torch.randn(n, generator=g, dtype=torch.float64)
    eng = OE.EngineRef(p0, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    tp = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([tp], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for _ in range(6):
        grad = 1e-2 * torch.randn(n, generator=g, dtype=torch.float64)
        norm = eng.step(grad, max_grad_norm=max_norm)
        opt.zero_grad()
        tp.grad = grad.clone()
        tn = float(torch.nn.utils.clip_grad_norm_([tp], max_norm)) if max_norm > 0 else float(grad.norm())
        opt.step()
        assert abs(norm - tn) < 1e-12
    torch.testing.assert_close(eng.master, tp.detach(), atol=1e-12, rtol=1e-9)
    assert eng.step_count == 6


def test_train_reference_low_precision_state():
    """The train.py leg with the reference's bf16 optimizer state
    (low_precision_state): after training, every parameter is a bf16 value
    (no fp32 master behind it), the parameters moved, and they differ from
    the fp32-master leg run on the same stream; a fp32 param_dtype is
    refused."""
    cfg = OM.Cfg(vocab_size=256, dim=64, n_layers=1, n_heads=4, n_kv_heads=2, ffn_dim=128, rope_theta=10_000.0,
                 rope_angle_dtype=torch.bfloat16)
    torch.manual_seed(0)
    P0 = OM.init_params(cfg)
    out = {}
    for low in (True, False):
        P = {k: v.clone() for k, v in P0.items()}
        OE.train_reference(cfg, P, OD.uniform_chunks(32, 256, 2, seed=1), steps=3, grad_accum_steps=1, lr=1e-2,
                           param_dtype=torch.bfloat16, low_precision_state=low)
        out[low] = P
    for k, v in out[True].items():
        assert torch.equal(v, v.to(torch.bfloat16).float()), k
    assert any(not torch.equal(v, v.to(torch.bfloat16).float()) for v in out[False].values())
    assert all(not torch.equal(out[True][k], P0[k].to(torch.bfloat16).float()) for k in P0 if P0[k].dim() == 2)
    assert any(not torch.equal(out[True][k], out[False][k].to(torch.bfloat16).float()) for k in P0)
    with pytest.raises(ValueError):
        OE.train_reference(cfg, dict(P0), OD.uniform_chunks(32, 256, 2, seed=1), steps=1, grad_accum_steps=1,
                           low_precision_state=True)


BASELINE_COUNTS = {
    # (dim, layers, heads, kv, ffn) -> tied parameter count (BASELINE workloads)
    (256, 4, 8, 4, 688): 11_094_272,
    (768, 12, 12, 4, 2048): 100_092_672,
    (2048, 16, 16, 8, 5632): 820_578_304,
    (4096, 32, 32, 8, 11008): 5_802_037_248,
}


@pytest.mark.parametrize("shape,count", list(BASELINE_COUNTS.items()))
def test_parameter_counts_closed_form(shape, count):
    d, L, H, KV, f = shape
    cfg = OM.Cfg(vocab_size=32000, dim=d, n_layers=L, n_heads=H, n_kv_heads=KV, ffn_dim=f)
    assert OM.num_parameters(cfg) == count
    _, numels, total = OF.flat_layout([s for _, s in OM.param_specs(cfg)])
    assert total == count
    untied = OM.Cfg(vocab_size=32000, dim=d, n_layers=L, n_heads=H, n_kv_heads=KV, ffn_dim=f, tie_word_embeddings=False)
    assert OM.num_parameters(untied) == count + 32000 * d


def test_default_ffn_dim():
    assert OM.default_ffn_dim(320) == 1024 and OM.default_ffn_dim(2048) == 5632 and OM.default_ffn_dim(64) == 256


def test_flat_layout_brute_force_and_shards():
    shapes = [(3, 4), (5,), (2, 2, 2), (1,)]
    offs, numels, total = OF.flat_layout(shapes)
    assert list(offs) == [0, 12, 17, 25] and total == 26
    for ws in (1, 2, 3, 5, 8, 27, 40):
        covered = []
        for r in range(ws):
            s = OF.shard_spec(total, r, ws)
            covered.extend(range(s["shard_start"], s["shard_end"]))
            assert s["chunk_size"] == max(1, math.ceil(total / ws))
        assert covered == list(range(total))
    buckets = OF.bucket_plan(820_578_304)
    assert buckets[0] == (0, 25_000_000) and buckets[-1][1] == 820_578_304
    assert all(a[1] == b[0] for a, b in zip(buckets, buckets[1:]))
    assert len(buckets) == 33


def test_stage3_handles_of_the_tied_model():
    cfg = tiny_cfg()
    hs = OF.stage3_handles(cfg)
    assert [h["name"] for h in hs] == ["tok_embeddings", "layers.0", "layers.1", "norm"]
    assert hs[0]["module_names"] == ["tok_embeddings", "lm_head"]
    assert len(hs[1]["params"]) == 9


def test_synthetic_streams():
    ramp = OD.ramp_chunks(seq_len=8, vocab_size=13, batch_size=2)
    first = next(ramp)
    assert first.tolist() == [[0, 1, 2, 3, 4, 5, 6, 7, 8], [9, 10, 11, 12, 0, 1, 2, 3, 4]]
    u1 = next(OD.uniform_chunks(16, 32000, 4, seed=0))
    u2 = torch.randint(0, 32000, (4, 17), generator=torch.Generator().manual_seed(0))
    assert torch.equal(u1, u2)
    inputs, labels = OD.split_chunk(first)
    assert torch.equal(inputs, labels) and inputs.shape == (2, 8)


def test_oracle_masked_attention_matches_sdpa():
    """The oracle's attn_mask branch against F.scaled_dot_product_attention
    (the call the reference makes, model/llama.py:109-117) for bool and
    additive masks, and an explicit causal mask against is_causal."""
    g = torch.Generator().manual_seed(3)
    B, H, KV, S, hd = 2, 4, 2, 12, 8
    q = torch.randn(B, H, S, hd, generator=g, dtype=torch.float64)
    k = torch.randn(B, KV, S, hd, generator=g, dtype=torch.float64)
    v = torch.randn(B, KV, S, hd, generator=g, dtype=torch.float64)
    kk, vv = k.repeat_interleave(H // KV, dim=1), v.repeat_interleave(H // KV, dim=1)
    bmask = torch.rand(B, 1, S, S, generator=g) > 0.3
    bmask[..., 0] = True
    fmask = torch.randn(S, S, generator=g, dtype=torch.float64)
    for m in (bmask, fmask):
        ref = F.scaled_dot_product_attention(q, kk, vv, attn_mask=m, is_causal=False)
        assert torch.allclose(R.causal_gqa_attention(q, k, v, attn_mask=m), ref, atol=1e-12, rtol=1e-10)
    causal = ~torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    assert torch.allclose(R.causal_gqa_attention(q, k, v, attn_mask=causal), R.causal_gqa_attention(q, k, v),
                          atol=1e-14, rtol=0)


def test_oracle_splitmix64_known_answers():
    """The dropout stream is SplitMix64 (Steele, Lea & Flood, OOPSLA 2014):
    the first five outputs of Vigna's reference splitmix64.c with state
    1234567, a published known-answer sequence; and the stream's blocks
    agree with one long draw (output i depends only on (seed, i))."""
    assert R.splitmix64(1234567, 5).tolist() == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                                 4593380528125082431, 16408922859458223821]
    full = R.splitmix64(99, 1000)
    assert np.array_equal(R.splitmix64(99, 300, start=700), full[700:])


@pytest.mark.parametrize("p", [0.0, 0.1, 0.2, 0.5, 0.9, 1.0])
def test_oracle_dropout_keep_rate(p):
    """P(keep) = 1 - p: p = 0 keeps all, p = 1 none, otherwise the kept
    fraction of 2^20 draws is within 5 binomial sigmas of 1 - p, and two keys
    give different masks."""
    n = 1 << 20
    keep = R.dropout_keep(12345, n, p)
    if p == 0.0:
        assert keep.all()
    elif p == 1.0:
        assert not keep.any()
    else:
        sigma = (p * (1 - p) / n) ** 0.5
        assert abs(keep.mean() - (1 - p)) < 5 * sigma
        assert (keep != R.dropout_keep(12346, n, p)).any()


def test_oracle_dropout_matches_torch_dropout():
    """oracle dropout(x, keep, p) reproduces F.dropout in training mode when
    given F.dropout's own keep mask (model/llama.py:146, :213), and the
    attention-probability dropout of the reference's fallback branch
    (model/llama.py:127-130: softmax, F.dropout, @ v) with its mask laid out
    [B, H, S(query), S(key)]."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 7, 33, generator=g, dtype=torch.float64)
    for p in (0.1, 0.5):
        torch.manual_seed(11)
        y = F.dropout(x, p=p, training=True)
        assert torch.equal(R.dropout(x, y != 0, p), y)
    B, H, KV, S, hd, p = 2, 4, 2, 10, 8, 0.3
    q = torch.randn(B, H, S, hd, generator=g, dtype=torch.float64)
    k = torch.randn(B, KV, S, hd, generator=g, dtype=torch.float64)
    v = torch.randn(B, KV, S, hd, generator=g, dtype=torch.float64)
    kk, vv = k.repeat_interleave(H // KV, dim=1), v.repeat_interleave(H // KV, dim=1)
    scores = (q @ kk.transpose(-2, -1)) * hd**-0.5
    scores = scores.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    torch.manual_seed(12)
    dropped = F.dropout(probs, p=p, training=True)
    ref = dropped @ vv
    keep = dropped != 0
    out = R.causal_gqa_attention(q, k, v, dropout_keep=keep, dropout_p=p)
    assert torch.allclose(out, ref, atol=1e-12, rtol=1e-12)
    # the mask changes the result (it is applied), and keep = 1 everywhere is plain attention
    assert not torch.allclose(out, R.causal_gqa_attention(q, k, v))
    ones = torch.ones(B, H, S, S, dtype=torch.bool)
    assert torch.allclose(R.causal_gqa_attention(q, k, v, dropout_keep=ones, dropout_p=0.0),
                          R.causal_gqa_attention(q, k, v), atol=1e-14, rtol=0)
