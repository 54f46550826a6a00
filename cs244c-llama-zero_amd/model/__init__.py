from .config import (
    MODEL_SIZES,
    ModelConfig,
    build_125m_config,
    build_1b_config,
    build_7b_config,
    build_config,
    build_medium_config,
    build_plumbing_config,
    build_small_config,
    build_tiny_config,
    estimate_num_parameters,
    human_readable_count,
)
from .llama import CausalLMOutput, LlamaForCausalLM

__all__ = [
    "MODEL_SIZES",
    "ModelConfig",
    "build_config",
    "build_tiny_config",
    "build_small_config",
    "build_medium_config",
    "build_plumbing_config",
    "build_125m_config",
    "build_1b_config",
    "build_7b_config",
    "estimate_num_parameters",
    "human_readable_count",
    "CausalLMOutput",
    "LlamaForCausalLM",
]
