from .fineweb import (
    FineWebUnavailable,
    PackedFineWebDataset,
    RankShardIterableDataset,
    SyntheticPatternDataset,
    SyntheticUniformDataset,
    TokenizerBundle,
    TokenPacker,
    load_fineweb_stream,
    load_llama_tokenizer,
)

__all__ = [
    "FineWebUnavailable",
    "PackedFineWebDataset",
    "RankShardIterableDataset",
    "SyntheticPatternDataset",
    "SyntheticUniformDataset",
    "TokenizerBundle",
    "TokenPacker",
    "load_fineweb_stream",
    "load_llama_tokenizer",
]
