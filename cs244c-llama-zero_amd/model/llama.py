"""LLaMA-style causal LM whose compute runs on the gfx950 HIP kernels.

Module tree, class names, attribute names, state_dict keys, constructor
signatures and the order of parameter construction follow the reference
(model/llama.py:14-335), so checkpoints, the ZeRO engines' flat layouts and the
seeded initial weights carry over.  The forward/backward math is the
reference's; it is computed by lzhip (RMSNorm, RoPE, fused QKV + flash
attention, fused gate/up + SwiGLU, GEMMs with the residual add in the
epilogue, embedding, cross entropy).  Tensors must live on a ROCm GPU; there is
no CPU compute path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional, Tuple

import torch
import torch.nn as nn
from torch.utils.checkpoint import checkpoint as activation_checkpoint

from lzhip import functional as LF
from lzhip import ops

from .config import ModelConfig


def _next_token(logits: torch.Tensor, temperature: float, top_k: Optional[int]) -> torch.Tensor:
    """One token per row of [B, V] logits (see LlamaForCausalLM.generate)."""
    if temperature <= 0:
        return logits.argmax(dim=-1)
    scaled = logits / temperature
    if top_k is not None:
        kth = torch.topk(scaled, min(top_k, scaled.size(-1))).values[:, -1:]
        scaled = scaled.masked_fill(scaled < kth, float("-inf"))
    return torch.multinomial(torch.softmax(scaled, dim=-1), num_samples=1).squeeze(-1)


class HipLinear(nn.Linear):
    """nn.Linear (same parameters, initialisation and state_dict) whose
    forward is the MFMA GEMM; bias is not supported (the model has none)."""

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.bias is not None:
            raise NotImplementedError("HipLinear has no bias path")
        return LF.linear(x, self.weight, residual)


class HipLMHead(HipLinear):
    """The LM head (nn.Linear, tied to the embedding).  Called with labels it
    returns the shifted cross-entropy loss instead of the logits, through the
    fused LM-head + loss Function, which never holds the [B*S, V] logits."""

    fused_chunk_bytes = 1 << 30  # logits buffer of the fused loss

    def forward(self, x: torch.Tensor, labels: Optional[torch.Tensor] = None, clamp: bool = False) -> torch.Tensor:
        if labels is None:
            return super().forward(x)
        if self.bias is not None:
            raise NotImplementedError("the fused LM-head loss has no bias path")
        return LF.lm_head_cross_entropy(x, self.weight, labels, clamp, self.fused_chunk_bytes)


class HipEmbedding(nn.Embedding):
    """nn.Embedding (same parameters and initialisation) with the HIP gather."""

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return LF.EmbeddingFn.apply(ids, self.weight)


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return LF.rms_norm(x, self.weight, self.eps)

    def forward_with_residual(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(norm(x), x) for a pre-norm residual block; the residual gradient is
        added inside the norm's backward kernel."""
        return LF.rms_norm_with_residual(x, self.weight, self.eps)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """cat(-x2, x1) over the last dimension (model/llama.py:25-28); a tensor
    helper kept for API compatibility, not used by the training path."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
) -> Tuple[torch.Tensor, torch.Tensor]:
    """q/k [..., S, hd] with tables [1, 1, S, hd] (model/llama.py:31-39)."""
    seq, hd = q.shape[-2], q.shape[-1]
    c2, s2 = cos.reshape(-1, hd)[:seq], sin.reshape(-1, hd)[:seq]
    return LF.RopeFn.apply(q, c2, s2), LF.RopeFn.apply(k, c2, s2)


class RotaryEmbedding(nn.Module):
    """cos/sin cache [1, 1, S, hd] in the activation dtype, rebuilt when the
    sequence grows or the device/dtype changes (model/llama.py:42-69); the
    table is computed by the lz_rope_table kernel from the inv_freq buffer.
    Like the reference's, that buffer follows Module.to(dtype), and the
    positions and angles are then formed in its dtype."""

    def __init__(self, dim: int, base: float = 500_000.0) -> None:
        super().__init__()
        self.dim = dim
        self.base = float(base)
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self.max_seq_len_cached = 0
        self.register_buffer("cos_cached", torch.empty(0), persistent=False)
        self.register_buffer("sin_cached", torch.empty(0), persistent=False)

    def _build_cache(self, seq_len: int, device: torch.device, dtype: torch.dtype) -> None:
        inv = self.inv_freq
        if inv.device != device:
            inv = inv.to(device)
        cos, sin = ops.rope_table(seq_len, self.dim, inv.contiguous(), dtype)
        self.cos_cached = cos[None, None]
        self.sin_cached = sin[None, None]
        self.max_seq_len_cached = seq_len

    def forward(self, seq_len: int, device: torch.device, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        if (
            seq_len > self.max_seq_len_cached
            or self.cos_cached.device != device
            or self.cos_cached.dtype != dtype
        ):
            self._build_cache(seq_len=seq_len, device=device, dtype=dtype)
        return self.cos_cached[:, :, :seq_len, :], self.sin_cached[:, :, :seq_len, :]

    def tables(self, seq_len: int, device: torch.device, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """[S, hd] views of the cache for the fused kernels."""
        cos, sin = self.forward(seq_len, device, dtype)
        return cos.reshape(-1, self.dim), sin.reshape(-1, self.dim)


class GroupedQueryAttention(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.n_heads = cfg.n_heads
        self.n_kv_heads = cfg.n_kv_heads
        self.head_dim = cfg.head_dim
        self.dropout = cfg.dropout
        self.scale = self.head_dim**-0.5

        self.q_proj = HipLinear(cfg.dim, cfg.n_heads * self.head_dim, bias=False)
        self.k_proj = HipLinear(cfg.dim, cfg.n_kv_heads * self.head_dim, bias=False)
        self.v_proj = HipLinear(cfg.dim, cfg.n_kv_heads * self.head_dim, bias=False)
        self.o_proj = HipLinear(cfg.n_heads * self.head_dim, cfg.dim, bias=False)

        self.rotary = RotaryEmbedding(dim=self.head_dim, base=cfg.rope_theta)

    def forward(
        self,
        x: torch.Tensor,
        attention_mask: Optional[torch.Tensor] = None,
        residual: Optional[torch.Tensor] = None,
    ) -> torch.Tensor:
        """GQA (model/llama.py:95-133): causal, or with `attention_mask` in its
        place (SDPA's attn_mask: bool keeps where True, a float mask is added
        to the scaled scores; broadcastable to [B, H, S, S]); attention
        dropout with p = cfg.dropout in training mode (model/llama.py:107);
        `residual` (optional) is added inside the o_proj GEMM."""
        ops.require_gpu(x)
        bsz, seq_len, _ = x.shape
        cos, sin = self.rotary.tables(seq_len, x.device, x.dtype)
        attn_dropout = float(self.dropout) if self.training else 0.0
        seed = ops.dropout_seed(x.device) if attn_dropout > 0.0 else 0
        y = LF.AttnProjFn.apply(
            x, self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, cos, sin,
            self.n_heads, self.n_kv_heads, float(self.scale), attention_mask, attn_dropout, seed,
        )
        return self.o_proj(y, residual)


class SwiGLU(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.gate_proj = HipLinear(cfg.dim, cfg.ffn_dim, bias=False)
        self.up_proj = HipLinear(cfg.dim, cfg.ffn_dim, bias=False)
        self.down_proj = HipLinear(cfg.ffn_dim, cfg.dim, bias=False)
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                compute_output: bool = True) -> torch.Tensor:
        """compute_output=False (the caller only takes gradients through the
        result): the down projection's product is left uncomputed."""
        ops.require_gpu(x)
        p = float(self.dropout.p) if self.training else 0.0  # nn.Dropout on the gated activations
        seed = ops.dropout_seed(x.device) if p > 0.0 else 0
        return LF.MLPFn.apply(x, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight, residual,
                              torch.is_grad_enabled(), p, seed, compute_output)


class TransformerBlock(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.input_norm = RMSNorm(cfg.dim, eps=cfg.rms_norm_eps)
        self.attn = GroupedQueryAttention(cfg)
        self.post_attn_norm = RMSNorm(cfg.dim, eps=cfg.rms_norm_eps)
        self.mlp = SwiGLU(cfg)

    def forward(self, x: torch.Tensor, attention_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        # x + attn(norm(x)); then x + mlp(norm(x)) — residual adds in the GEMM
        # epilogues, residual gradients inside the norm backward
        h, x = self.input_norm.forward_with_residual(x)
        x = self.attn(h, attention_mask=attention_mask, residual=x)
        h, x = self.post_attn_norm.forward_with_residual(x)
        # the block's output is the MLP's: under output_unused() (the ZeRO-3
        # recompute) its value is not formed
        return self.mlp(h, residual=x, compute_output=not LF.output_is_unused())


@dataclass
class CausalLMOutput:
    logits: Optional[torch.Tensor]
    loss: Optional[torch.Tensor] = None


class LlamaForCausalLM(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.cfg = cfg
        # construction order = the reference's (its RNG draws and parameter order)
        self.tok_embeddings = HipEmbedding(cfg.vocab_size, cfg.dim)
        self.dropout = nn.Dropout(cfg.dropout)
        self.layers = nn.ModuleList([TransformerBlock(cfg) for _ in range(cfg.n_layers)])
        self.norm = RMSNorm(cfg.dim, eps=cfg.rms_norm_eps)
        self.lm_head = HipLMHead(cfg.dim, cfg.vocab_size, bias=False)

        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.tok_embeddings.weight

        self.apply(self._init_weights)
        self._zero3_executor = None
        self.loss_chunk_size = 0
        self.activation_checkpointing = False
        # training loss without returned logits: LM head and cross entropy fused
        self.fused_lm_head_loss = True

    def _init_weights(self, module: nn.Module) -> None:
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=self.cfg.initializer_range)
            if isinstance(module, nn.Linear) and module.bias is not None:
                nn.init.zeros_(module.bias)

    def set_loss_chunk_size(self, chunk_size: int) -> None:
        if chunk_size < 0:
            raise ValueError(f"loss chunk size must be non-negative, got {chunk_size}")
        self.loss_chunk_size = int(chunk_size)

    def set_activation_checkpointing(self, enabled: bool) -> None:
        self.activation_checkpointing = bool(enabled)

    def forward(
        self,
        input_ids: torch.Tensor,
        labels: Optional[torch.Tensor] = None,
        attention_mask: Optional[torch.Tensor] = None,
        return_logits: bool = True,
    ) -> CausalLMOutput:
        if input_ids.ndim != 2:
            raise ValueError(f"input_ids should have shape [batch, seq], got {tuple(input_ids.shape)}")

        x = self._call_parametrized_module("tok_embeddings", self.tok_embeddings, input_ids)
        x = LF.dropout(x, float(self.dropout.p), self.training)

        for layer_idx in range(len(self.layers)):
            if self._should_checkpoint_activations(x):
                x = activation_checkpoint(
                    lambda hidden_states, _i=layer_idx, _m=attention_mask: self._call_layer(_i, hidden_states, _m),
                    x,
                    use_reentrant=False,
                )
            else:
                x = self._call_layer(layer_idx, x, attention_mask)

        x = self._call_parametrized_module("norm", self.norm, x)
        logits = None
        chunked = self._should_chunk_training_loss(input_ids)
        # fp16 takes the unfused loss: the fused one forms the logit gradient
        # for a unit loss gradient before the (loss-scaled) gradient arrives,
        # and (softmax - onehot) / count underflows fp16's range
        if labels is not None and not return_logits and self.fused_lm_head_loss and x.dtype != torch.float16:
            if labels.shape != input_ids.shape:
                raise ValueError(
                    f"labels should have same shape as input_ids; got {tuple(labels.shape)} vs {tuple(input_ids.shape)}"
                )
            # same divisor rule as the unfused paths: the chunked loss (and a
            # length-1 sequence) clamps the target count at 1
            clamp = chunked or input_ids.size(1) <= 1
            loss = self._call_parametrized_module("lm_head", self.lm_head, x, labels, clamp)
            return CausalLMOutput(logits=None, loss=loss)
        if labels is None or return_logits or not chunked:
            logits = self._call_parametrized_module("lm_head", self.lm_head, x)

        loss = None
        if labels is not None:
            if labels.shape != input_ids.shape:
                raise ValueError(
                    f"labels should have same shape as input_ids; got {tuple(labels.shape)} vs {tuple(input_ids.shape)}"
                )
            if logits is not None:
                loss = self._full_cross_entropy(logits=logits, labels=labels, internal=not return_logits)
            else:
                loss = self._chunked_cross_entropy(hidden_states=x, labels=labels)
            if not return_logits:
                logits = None

        return CausalLMOutput(logits=logits, loss=loss)

    def _call_layer(self, layer_idx: int, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor]):
        layer = self.layers[layer_idx]
        return self._call_parametrized_module(f"layers.{layer_idx}", layer, hidden_states, attention_mask)

    def _should_checkpoint_activations(self, hidden_states: torch.Tensor) -> bool:
        return (
            self.activation_checkpointing
            and self.training
            and self._zero3_executor is None
            and hidden_states.requires_grad
        )

    def _should_chunk_training_loss(self, input_ids: torch.Tensor) -> bool:
        return self.loss_chunk_size > 0 and input_ids.size(1) > 1 and self._zero3_executor is None

    def _full_cross_entropy(self, logits: torch.Tensor, labels: torch.Tensor, internal: bool = False) -> torch.Tensor:
        """Mean CE of logits[:, :-1] against labels[:, 1:], ignore_index -100
        (model/llama.py:273-280).  A length-1 sequence gives a zero loss."""
        if logits.size(1) <= 1:
            return LF.cross_entropy(logits, labels, clamp=True, inplace=False)
        return LF.cross_entropy(logits, labels, clamp=False, inplace=internal)

    def _chunked_cross_entropy(self, hidden_states: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        """Sum of per-token losses / max(#targets, 1) (model/llama.py:282-302).
        The LM head runs once over all positions; the loss kernel streams the
        logits row by row, which yields the chunked sum exactly."""
        logits = self._call_parametrized_module("lm_head", self.lm_head, hidden_states)
        return LF.cross_entropy(logits, labels, clamp=True, inplace=True)

    def _call_parametrized_module(self, module_name: str, module: nn.Module, *args: Any) -> torch.Tensor:
        executor = self._zero3_executor
        if executor is None:
            return module(*args)
        return executor.call_module(module_name, module, *args)

    @torch.no_grad()
    def generate(
        self,
        input_ids: torch.Tensor,
        max_new_tokens: int,
        temperature: float = 1.0,
        top_k: Optional[int] = None,
    ) -> torch.Tensor:
        """Autoregressive sampling with the reference's semantics
        (model/llama.py:311-335): each new token takes a full forward over the
        last max_seq_len tokens; temperature <= 0 picks the arg-max, otherwise
        the logits / temperature, cut to their top_k largest, are sampled.
        The sequence grows in one preallocated buffer."""
        self.eval()
        bsz, t0 = input_ids.shape
        seq = input_ids.new_empty((bsz, t0 + max_new_tokens))
        seq[:, :t0] = input_ids
        window = self.cfg.max_seq_len
        for t in range(t0, t0 + max_new_tokens):
            context = seq[:, max(0, t - window) : t].contiguous()
            last = self(context).logits[:, -1, :].float()
            seq[:, t] = _next_token(last, temperature, top_k)
        return seq
