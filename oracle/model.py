"""Functional restatement of the reference LLaMA model on the CPU.

Parameters are a dict keyed like the reference state_dict
(`tok_embeddings.weight`, `layers.{i}.attn.q_proj.weight`, ...).  init_params
draws them in the reference's construction order (model/llama.py:169-192):
nn.Embedding's normal_, nn.Linear's kaiming_uniform_(a=sqrt(5)) per projection
in registration order, then apply(_init_weights)'s N(0, 0.02) re-draws in
module post-order, the tied LM head re-drawing the embedding last.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import ops


@dataclass(frozen=True)
class Cfg:
    vocab_size: int
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: int
    rope_theta: float = 500_000.0
    rms_norm_eps: float = 1e-5
    tie_word_embeddings: bool = True
    initializer_range: float = 0.02
    # dtype of the RoPE angle computation: float32, or bfloat16 for the
    # reference after Module.to(bfloat16) (its inv_freq buffer is cast too)
    rope_angle_dtype: torch.dtype = torch.float32

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads


def default_ffn_dim(dim: int) -> int:
    """model/config.py:7-15."""
    v = int((8 * dim) / 3)
    return v if v % 256 == 0 else v + 256 - (v % 256)


def num_parameters(cfg: Cfg) -> int:
    """model/config.py:129-151."""
    kv = cfg.n_kv_heads * cfg.head_dim
    per_block = cfg.dim * cfg.dim * 2 + cfg.dim * kv * 2 + cfg.dim * cfg.ffn_dim * 3 + 2 * cfg.dim
    total = cfg.vocab_size * cfg.dim + per_block * cfg.n_layers + cfg.dim
    if not cfg.tie_word_embeddings:
        total += cfg.vocab_size * cfg.dim
    return total


def param_specs(cfg: Cfg) -> List[Tuple[str, Tuple[int, ...]]]:
    """(name, shape) in model.parameters() order (the tied LM head is not a
    separate parameter)."""
    d, hd = cfg.dim, cfg.head_dim
    specs: List[Tuple[str, Tuple[int, ...]]] = [("tok_embeddings.weight", (cfg.vocab_size, d))]
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        specs += [
            (p + "input_norm.weight", (d,)),
            (p + "attn.q_proj.weight", (cfg.n_heads * hd, d)),
            (p + "attn.k_proj.weight", (cfg.n_kv_heads * hd, d)),
            (p + "attn.v_proj.weight", (cfg.n_kv_heads * hd, d)),
            (p + "attn.o_proj.weight", (d, cfg.n_heads * hd)),
            (p + "post_attn_norm.weight", (d,)),
            (p + "mlp.gate_proj.weight", (cfg.ffn_dim, d)),
            (p + "mlp.up_proj.weight", (cfg.ffn_dim, d)),
            (p + "mlp.down_proj.weight", (d, cfg.ffn_dim)),
        ]
    specs.append(("norm.weight", (d,)))
    if not cfg.tie_word_embeddings:
        specs.append(("lm_head.weight", (cfg.vocab_size, d)))
    return specs


def _kaiming(out_f: int, in_f: int) -> torch.Tensor:
    w = torch.empty(out_f, in_f)
    torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    return w


def init_params(cfg: Cfg) -> Dict[str, torch.Tensor]:
    """Draws from torch's global CPU generator in the reference order; seed it
    first (torch.manual_seed) to reproduce a reference initialisation."""
    d, hd = cfg.dim, cfg.head_dim
    P: Dict[str, torch.Tensor] = {}
    emb = torch.empty(cfg.vocab_size, d)
    torch.nn.init.normal_(emb)
    P["tok_embeddings.weight"] = emb
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        P[p + "input_norm.weight"] = torch.ones(d)
        P[p + "attn.q_proj.weight"] = _kaiming(cfg.n_heads * hd, d)
        P[p + "attn.k_proj.weight"] = _kaiming(cfg.n_kv_heads * hd, d)
        P[p + "attn.v_proj.weight"] = _kaiming(cfg.n_kv_heads * hd, d)
        P[p + "attn.o_proj.weight"] = _kaiming(d, cfg.n_heads * hd)
        P[p + "post_attn_norm.weight"] = torch.ones(d)
        P[p + "mlp.gate_proj.weight"] = _kaiming(cfg.ffn_dim, d)
        P[p + "mlp.up_proj.weight"] = _kaiming(cfg.ffn_dim, d)
        P[p + "mlp.down_proj.weight"] = _kaiming(d, cfg.ffn_dim)
    P["norm.weight"] = torch.ones(d)
    lm_head = _kaiming(cfg.vocab_size, d)
    # apply(_init_weights): post-order over modules
    std = cfg.initializer_range
    torch.nn.init.normal_(P["tok_embeddings.weight"], mean=0.0, std=std)
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        for name in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj",
                     "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            torch.nn.init.normal_(P[p + name + ".weight"], mean=0.0, std=std)
    if cfg.tie_word_embeddings:
        torch.nn.init.normal_(P["tok_embeddings.weight"], mean=0.0, std=std)
    else:
        torch.nn.init.normal_(lm_head, mean=0.0, std=std)
        P["lm_head.weight"] = lm_head
    return P


def lm_head_weight(P: Dict[str, torch.Tensor], cfg: Cfg) -> torch.Tensor:
    return P["tok_embeddings.weight"] if cfg.tie_word_embeddings else P["lm_head.weight"]


def block_forward(P: Dict[str, torch.Tensor], cfg: Cfg, i: int, x: torch.Tensor, attn_impl: str = "sdpa",
                  drop: Optional[Dict] = None) -> torch.Tensor:
    """model/llama.py:149-160 with GroupedQueryAttention (:95-133) and SwiGLU
    (:143-146).  drop (training-mode dropout given its keep masks): {"p": p,
    (i, "attn"): keep [B, H, S, S], (i, "mlp"): keep [B, S, ffn]}."""
    p = f"layers.{i}."
    B, S, d = x.shape
    H, KV, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    h = ops.rmsnorm(x, P[p + "input_norm.weight"], cfg.rms_norm_eps)
    q = (h @ P[p + "attn.q_proj.weight"].t()).view(B, S, H, hd).transpose(1, 2)
    k = (h @ P[p + "attn.k_proj.weight"].t()).view(B, S, KV, hd).transpose(1, 2)
    v = (h @ P[p + "attn.v_proj.weight"].t()).view(B, S, KV, hd).transpose(1, 2)
    cos, sin = ops.rope_tables(S, hd, cfg.rope_theta, dtype=q.dtype, angle_dtype=cfg.rope_angle_dtype)
    q = ops.apply_rope(q, cos, sin)
    k = ops.apply_rope(k, cos, sin)
    if drop is not None:
        y = ops.causal_gqa_attention(q, k, v, dropout_keep=drop[(i, "attn")], dropout_p=drop["p"])
    elif attn_impl == "sdpa":
        if H != KV:
            k = k.repeat_interleave(H // KV, dim=1)
            v = v.repeat_interleave(H // KV, dim=1)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    else:
        y = ops.causal_gqa_attention(q, k, v)
    y = y.transpose(1, 2).contiguous().view(B, S, H * hd)
    x = x + y @ P[p + "attn.o_proj.weight"].t()
    h2 = ops.rmsnorm(x, P[p + "post_attn_norm.weight"], cfg.rms_norm_eps)
    g = h2 @ P[p + "mlp.gate_proj.weight"].t()
    u = h2 @ P[p + "mlp.up_proj.weight"].t()
    m = ops.swiglu(g, u)
    if drop is not None:
        m = ops.dropout(m, drop[(i, "mlp")], drop["p"])
    return x + m @ P[p + "mlp.down_proj.weight"].t()


def hidden_states(P: Dict[str, torch.Tensor], cfg: Cfg, ids: torch.Tensor, attn_impl: str = "sdpa",
                  drop: Optional[Dict] = None) -> torch.Tensor:
    """drop: see block_forward; its "embed" entry ([B, S, dim]) is the token
    embeddings' dropout (model/llama.py:212-213)."""
    x = P["tok_embeddings.weight"][ids]
    if drop is not None:
        x = ops.dropout(x, drop["embed"], drop["p"])
    for i in range(cfg.n_layers):
        x = block_forward(P, cfg, i, x, attn_impl, drop)
    return ops.rmsnorm(x, P["norm.weight"], cfg.rms_norm_eps)


def logits(P: Dict[str, torch.Tensor], cfg: Cfg, ids: torch.Tensor, attn_impl: str = "sdpa") -> torch.Tensor:
    return hidden_states(P, cfg, ids, attn_impl) @ lm_head_weight(P, cfg).t()


def loss(P: Dict[str, torch.Tensor], cfg: Cfg, ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
         chunk_size: int = 0, attn_impl: str = "sdpa", drop: Optional[Dict] = None) -> torch.Tensor:
    """Training loss: full mean CE (chunk_size == 0, model/llama.py:273-280) or
    the chunked sum/max(count,1) computed chunk by chunk with F.cross_entropy
    (model/llama.py:282-302)."""
    labels = ids if labels is None else labels
    x = hidden_states(P, cfg, ids, attn_impl, drop)
    W = lm_head_weight(P, cfg)
    S = x.size(1)
    if chunk_size <= 0:
        lg = x @ W.t()
        if S <= 1:
            return lg.sum() * 0.0
        return F.cross_entropy(lg[:, :-1, :].transpose(1, 2), labels[:, 1:], ignore_index=-100)
    if S <= 1:
        return x.sum() * 0.0
    total = torch.zeros((), dtype=x.dtype)
    count = torch.zeros((), dtype=torch.long)
    for start in range(0, S - 1, chunk_size):
        end = min(start + chunk_size, S - 1)
        lg = x[:, start:end, :] @ W.t()
        lab = labels[:, start + 1 : end + 1]
        total = total + F.cross_entropy(lg.transpose(1, 2), lab, ignore_index=-100, reduction="sum")
        count = count + lab.ne(-100).sum()
    return total / count.clamp_min(1).to(total.dtype)
