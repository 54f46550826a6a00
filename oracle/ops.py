"""Reference arithmetic of the hot-path ops, restated on the CPU.

Each function follows the reference formula it cites and computes in the dtype
of its inputs (use float64 inputs for a high-precision oracle).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """model/llama.py:20-22: x * rsqrt(mean(x^2) + eps) * w."""
    norm = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return x * norm * w


def inv_freq(hd: int, theta: float) -> torch.Tensor:
    """model/llama.py:45: 1/theta^(2i/hd), computed in fp32."""
    return 1.0 / (theta ** (torch.arange(0, hd, 2).float() / hd))


def rope_tables(seq: int, hd: int, theta: float, dtype: torch.dtype = torch.float32,
                angle_dtype: torch.dtype = torch.float32) -> Tuple[torch.Tensor, torch.Tensor]:
    """model/llama.py:42-56: emb = cat(freqs, freqs) with freqs = outer(t,
    inv_freq), cos/sin cast to `dtype`.  `angle_dtype` is the dtype of the
    inv_freq buffer at cache-build time: after Module.to(bfloat16) the
    reference's buffer is bf16, so t, freqs and cos/sin are formed in bf16.
    Returns [seq, hd] tables."""
    inv = inv_freq(hd, theta).to(angle_dtype)
    t = torch.arange(seq, dtype=angle_dtype)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """model/llama.py:25-28."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """model/llama.py:38: x*cos + rotate_half(x)*sin; x [..., S, hd], tables [S, hd]."""
    return (x * cos) + (rotate_half(x) * sin)


def causal_gqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
                         attn_mask: Optional[torch.Tensor] = None, dropout_keep: Optional[torch.Tensor] = None,
                         dropout_p: float = 0.0) -> torch.Tensor:
    """model/llama.py:88-117 with is_causal=True: q [B,H,S,hd], k/v [B,KV,S,hd];
    K/V heads repeated (repeat_interleave) to H, softmax(q k^T * scale) v with
    the upper triangle masked.  Written out explicitly (no fused kernel).
    With attn_mask (model/llama.py:109-117, is_causal=False): a bool mask
    keeps the scores where True, a float mask is added to the scaled scores
    (the reference's fallback branch, llama.py:118-129).  With dropout_keep
    ([B, H, S, S], nonzero = kept): probs * keep / (1 - dropout_p) before
    the product with v (llama.py:115 dropout_p, :129 F.dropout(probs))."""
    B, H, S, hd = q.shape
    KV = k.shape[1]
    if H != KV:
        k = k.repeat_interleave(H // KV, dim=1)
        v = v.repeat_interleave(H // KV, dim=1)
    scale = hd**-0.5 if scale is None else scale
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if attn_mask is None:
        mask = torch.triu(torch.ones(S, S, dtype=torch.bool), diagonal=1)
        scores = scores.masked_fill(mask, float("-inf"))
    elif attn_mask.dtype == torch.bool:
        scores = scores.masked_fill(~attn_mask, float("-inf"))
    else:
        scores = scores + attn_mask.to(scores.dtype)
    probs = torch.softmax(scores, dim=-1)
    if dropout_keep is not None:
        probs = dropout(probs, dropout_keep, dropout_p)
    return torch.matmul(probs, v)


def dropout(x: torch.Tensor, keep: torch.Tensor, p: float) -> torch.Tensor:
    """nn.Dropout in training mode given its keep mask (model/llama.py:146,
    :213): x * keep / (1 - p); p == 1 gives zeros."""
    if p >= 1.0:
        return x * 0.0
    return x * keep.to(x.dtype) * (1.0 / (1.0 - p))


_GAMMA = 0x9E3779B97F4A7C15


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start+n-1 of SplitMix64 with state `seed` (Steele,
    Lea & Flood, "Fast splittable pseudorandom number generators", OOPSLA
    2014; the constants of Vigna's public-domain splitmix64.c): output i is
    mix(seed + (i + 1) * 0x9E3779B97F4A7C15) with mix(z) = z ^ z >> 31 after
    z = (z ^ z >> 30) * 0xBF58476D1CE4E5B9, z = (z ^ z >> 27) *
    0x94D049BB133111EB, all modulo 2^64 (numpy uint64 wraps)."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & (2**64 - 1)) + i * np.uint64(_GAMMA)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def dropout_keep(seed: int, n: int, p: float) -> np.ndarray:
    """The keep mask of elements 0..n-1 of the dropout stream with key
    `seed`: kept when the top 24 bits of SplitMix64 output i are >= ceil(p *
    2^24), so P(keep) = 1 - p to 2^-24 (bool array)."""
    thresh = min(math.ceil(p * 16777216.0), 16777216)
    return (splitmix64(seed, n) >> np.uint64(40)) >= np.uint64(thresh)


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """model/llama.py:145: silu(g) * u, silu(g) = g * sigmoid(g)."""
    return g * torch.sigmoid(g) * u


def shifted_cross_entropy(logits: torch.Tensor, labels: torch.Tensor, clamp: bool = False,
                          ignore_index: int = -100) -> torch.Tensor:
    """model/llama.py:273-302: CE of logits[:, :-1] against labels[:, 1:].
    clamp=False: mean over valid targets (F.cross_entropy); clamp=True: sum /
    max(count, 1) (the chunked variant).  Computed with an explicit
    log-sum-exp in the dtype of `logits`."""
    lg = logits[:, :-1, :]
    tg = labels[:, 1:]
    valid = tg.ne(ignore_index)
    lse = torch.logsumexp(lg, dim=-1)
    safe = torch.where(valid, tg, torch.zeros_like(tg))
    picked = torch.gather(lg, -1, safe.unsqueeze(-1)).squeeze(-1)
    per = torch.where(valid, lse - picked, torch.zeros_like(lse))
    count = valid.sum()
    denom = count.clamp_min(1) if clamp else count
    return per.sum() / denom.to(per.dtype)


def clip_scale(grad_norm: float, max_grad_norm: float) -> float:
    """zero/stage0_ddp.py:66-71: scale applied when 0 < max < norm."""
    if max_grad_norm > 0 and grad_norm > max_grad_norm:
        return max_grad_norm / (grad_norm + 1e-6)
    return 1.0


def adamw_update(p: torch.Tensor, m: torch.Tensor, v: torch.Tensor, g: torch.Tensor, *, lr: float, beta1: float,
                 beta2: float, eps: float, weight_decay: float, step: int) -> None:
    """In place, in the operation order of zero/stage0_ddp.py:73-88 (step is the
    already-incremented 1-based count)."""
    m.mul_(beta1).add_(g, alpha=1.0 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1.0 - beta2)
    bc1 = 1.0 - beta1**step
    bc2 = 1.0 - beta2**step
    if weight_decay != 0.0:
        p.mul_(1.0 - lr * weight_decay)
    denom = v.sqrt().div_(math.sqrt(bc2)).add_(eps)
    p.addcdiv_(m, denom, value=-(lr / bc1))
