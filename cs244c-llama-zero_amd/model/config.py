"""Model hyper-parameters and presets (reference: model/config.py).

ModelConfig, the ffn default, validation, the tiny/small/medium presets and
estimate_num_parameters keep the reference's names, fields and formulas so
configs, checkpoints and parameter counts carry over unchanged.  The presets
`plumbing`, `125m`, `1b` and `7b` are additions: the LLaMA shapes of the
single-GPU benchmark workloads (RoPE theta 10000, explicit ffn widths).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional


def _round_up(value: int, multiple: int) -> int:
    rem = value % multiple
    return value if rem == 0 else value + (multiple - rem)


def _default_ffn_dim(hidden_dim: int) -> int:
    # SwiGLU width ~ 8/3 * d rounded up to a multiple of 256 (model/config.py:13-15).
    return _round_up(int((8 * hidden_dim) / 3), 256)


@dataclass
class ModelConfig:
    name: str
    vocab_size: int
    max_seq_len: int
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: Optional[int] = None
    rope_theta: float = 500_000.0
    rms_norm_eps: float = 1e-5
    dropout: float = 0.0
    tie_word_embeddings: bool = True
    initializer_range: float = 0.02

    def __post_init__(self) -> None:
        if self.ffn_dim is None:
            self.ffn_dim = _default_ffn_dim(self.dim)
        # validation order and messages follow model/config.py:38-51
        if self.dim <= 0 or self.n_layers <= 0:
            raise ValueError("dim and n_layers must be positive")
        if self.n_heads <= 0 or self.n_kv_heads <= 0:
            raise ValueError("n_heads and n_kv_heads must be positive")
        if self.dim % self.n_heads != 0:
            raise ValueError("dim must be divisible by n_heads")
        if self.n_heads % self.n_kv_heads != 0:
            raise ValueError("n_heads must be divisible by n_kv_heads")
        if (self.dim // self.n_heads) % 2 != 0:
            raise ValueError("head_dim must be even for rotary embeddings")
        if self.vocab_size <= 0 or self.max_seq_len <= 0:
            raise ValueError("vocab_size and max_seq_len must be positive")
        if self.ffn_dim <= 0:
            raise ValueError("ffn_dim must be positive")

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    def with_vocab_size(self, vocab_size: int) -> "ModelConfig":
        return ModelConfig(**{**self.to_dict(), "vocab_size": vocab_size})

    def to_dict(self) -> Dict[str, object]:
        keys = (
            "name", "vocab_size", "max_seq_len", "dim", "n_layers", "n_heads", "n_kv_heads", "ffn_dim",
            "rope_theta", "rms_norm_eps", "dropout", "tie_word_embeddings", "initializer_range",
        )
        return {k: getattr(self, k) for k in keys}


def build_tiny_config(vocab_size: int = 128_256, max_seq_len: int = 2048) -> ModelConfig:
    return ModelConfig(name="tiny", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=320, n_layers=4, n_heads=10,
                       n_kv_heads=2)


def build_small_config(vocab_size: int = 128_256, max_seq_len: int = 2048) -> ModelConfig:
    return ModelConfig(name="small", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=1152, n_layers=12,
                       n_heads=18, n_kv_heads=6)


def build_medium_config(vocab_size: int = 128_256, max_seq_len: int = 2048) -> ModelConfig:
    return ModelConfig(name="medium", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=2048, n_layers=24,
                       n_heads=32, n_kv_heads=8)


def build_plumbing_config(vocab_size: int = 32_000, max_seq_len: int = 128) -> ModelConfig:
    """d256, 4 layers, 8 query / 4 KV heads (hd 32), ffn 688."""
    return ModelConfig(name="plumbing", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=256, n_layers=4,
                       n_heads=8, n_kv_heads=4, ffn_dim=688, rope_theta=10_000.0)


def build_125m_config(vocab_size: int = 32_000, max_seq_len: int = 1024) -> ModelConfig:
    """d768, 12 layers, 12 query / 4 KV heads (hd 64), ffn 2048."""
    return ModelConfig(name="125m", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=768, n_layers=12,
                       n_heads=12, n_kv_heads=4, ffn_dim=2048, rope_theta=10_000.0)


def build_1b_config(vocab_size: int = 32_000, max_seq_len: int = 2048) -> ModelConfig:
    """d2048, 16 layers, 16 query / 8 KV heads (hd 128), ffn 5632."""
    return ModelConfig(name="1b", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=2048, n_layers=16,
                       n_heads=16, n_kv_heads=8, ffn_dim=5632, rope_theta=10_000.0)


def build_7b_config(vocab_size: int = 32_000, max_seq_len: int = 2048) -> ModelConfig:
    """d4096, 32 layers, 32 query / 8 KV heads (hd 128), ffn 11008."""
    return ModelConfig(name="7b", vocab_size=vocab_size, max_seq_len=max_seq_len, dim=4096, n_layers=32,
                       n_heads=32, n_kv_heads=8, ffn_dim=11008, rope_theta=10_000.0)


_BUILDERS = {
    "tiny": build_tiny_config,
    "small": build_small_config,
    "medium": build_medium_config,
    "plumbing": build_plumbing_config,
    "125m": build_125m_config,
    "1b": build_1b_config,
    "7b": build_7b_config,
}

MODEL_SIZES = list(_BUILDERS)


def build_config(size: str, vocab_size: int = 128_256, max_seq_len: int = 2048) -> ModelConfig:
    size = size.lower().strip()
    if size not in _BUILDERS:
        raise ValueError(f"Unknown model size '{size}'. Expected one of {sorted(_BUILDERS)}")
    return _BUILDERS[size](vocab_size=vocab_size, max_seq_len=max_seq_len)


def estimate_num_parameters(cfg: ModelConfig) -> int:
    """Parameter count (model/config.py:129-151): embedding (shared with the LM
    head when tied), per block q/k/v/o + 3 MLP matrices + 2 norms, final norm."""
    kv_dim = cfg.n_kv_heads * cfg.head_dim
    per_block = 2 * cfg.dim * cfg.dim + 2 * cfg.dim * kv_dim + 3 * cfg.dim * cfg.ffn_dim + 2 * cfg.dim
    total = cfg.vocab_size * cfg.dim + cfg.n_layers * per_block + cfg.dim
    if not cfg.tie_word_embeddings:
        total += cfg.vocab_size * cfg.dim
    return total


def human_readable_count(num_params: int) -> str:
    for div, suffix in ((1_000_000_000, "B"), (1_000_000, "M"), (1_000, "K")):
        if num_params >= div:
            return f"{num_params / div:.2f}{suffix}"
    return str(num_params)
