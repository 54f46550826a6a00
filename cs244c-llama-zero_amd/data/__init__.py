from .fineweb import (
    PackedFineWebDataset,
    RankShardIterableDataset,
    SyntheticPatternDataset,
    SyntheticUniformDataset,
    TokenizerBundle,
    load_fineweb_stream,
    load_llama_tokenizer,
)

__all__ = [
    "PackedFineWebDataset",
    "RankShardIterableDataset",
    "SyntheticPatternDataset",
    "SyntheticUniformDataset",
    "TokenizerBundle",
    "load_fineweb_stream",
    "load_llama_tokenizer",
]
