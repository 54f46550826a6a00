"""Token streams for training (reference: data/fineweb.py).

SyntheticPatternDataset, RankShardIterableDataset and PackedFineWebDataset keep
the reference's behaviour.  SyntheticUniformDataset is an addition: iid uniform
token ids over [0, vocab) from one seeded torch.Generator, drawn as [S+1]
chunks (the benchmark workloads' synthetic data).  The FineWeb loaders need
the Hugging Face hub (network); they raise with a clear message when the
libraries or the network are unavailable.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Iterator, Optional

import torch
from torch.utils.data import IterableDataset


@dataclass
class TokenizerBundle:
    tokenizer: object
    vocab_size: int
    eos_token_id: int


def load_llama_tokenizer(tokenizer_name: str) -> TokenizerBundle:
    try:
        from transformers import AutoTokenizer
    except ImportError as exc:
        raise RuntimeError("transformers is required for real-data training") from exc
    tok = AutoTokenizer.from_pretrained(tokenizer_name, use_fast=True)
    if tok.eos_token_id is None:
        raise ValueError(f"Tokenizer '{tokenizer_name}' has no eos_token_id")
    if tok.pad_token_id is None:
        tok.pad_token = tok.eos_token
    return TokenizerBundle(tokenizer=tok, vocab_size=tok.vocab_size, eos_token_id=tok.eos_token_id)


def load_fineweb_stream(subset: str, split: str = "train", shuffle_buffer: int = 10_000, seed: int = 42):
    try:
        from datasets import load_dataset
    except ImportError as exc:
        raise RuntimeError("datasets is required for FineWeb-Edu streaming") from exc
    ds = load_dataset("HuggingFaceFW/fineweb-edu", subset, split=split, streaming=True)
    return ds.shuffle(buffer_size=shuffle_buffer, seed=seed)


class PackedFineWebDataset(IterableDataset):
    """Packs a text stream into fixed [seq_len + 1] token chunks, optionally
    separating documents with EOS (data/fineweb.py:58-97)."""

    def __init__(self, text_iterable: Iterable, tokenizer, seq_len: int, eos_token_id: int, text_key: str = "text",
                 add_eos_between_samples: bool = True) -> None:
        super().__init__()
        self.text_iterable = text_iterable
        self.tokenizer = tokenizer
        self.seq_len = seq_len
        self.eos_token_id = eos_token_id
        self.text_key = text_key
        self.add_eos_between_samples = add_eos_between_samples

    def __iter__(self) -> Iterator[torch.Tensor]:
        buf: list = []
        size = self.seq_len + 1
        for row in self.text_iterable:
            text = row.get(self.text_key, "") if isinstance(row, dict) else str(row)
            if not text:
                continue
            ids = self.tokenizer.encode(text, add_special_tokens=False)
            if not ids:
                continue
            buf.extend(ids)
            if self.add_eos_between_samples:
                buf.append(self.eos_token_id)
            while len(buf) >= size:
                chunk, buf = buf[:size], buf[size:]
                yield torch.tensor(chunk, dtype=torch.long)


class SyntheticPatternDataset(IterableDataset):
    """Deterministic ramp chunks (cursor + arange(S+1)) % V, the cursor
    advancing by S+1 modulo V (data/fineweb.py:100-122)."""

    def __init__(self, seq_len: int, vocab_size: int, num_sequences: Optional[int] = None) -> None:
        super().__init__()
        self.seq_len = seq_len
        self.vocab_size = vocab_size
        self.num_sequences = num_sequences

    def __iter__(self) -> Iterator[torch.Tensor]:
        produced, cursor = 0, 0
        length = self.seq_len + 1
        while self.num_sequences is None or produced < self.num_sequences:
            yield torch.arange(cursor, cursor + length, dtype=torch.long) % self.vocab_size
            cursor = (cursor + length) % self.vocab_size
            produced += 1


class SyntheticUniformDataset(IterableDataset):
    """iid uniform token ids over [0, vocab); every iteration restarts the
    seeded stream, so a DataLoader epoch is reproducible."""

    def __init__(self, seq_len: int, vocab_size: int, seed: int = 0, num_sequences: Optional[int] = None) -> None:
        super().__init__()
        self.seq_len = seq_len
        self.vocab_size = vocab_size
        self.seed = seed
        self.num_sequences = num_sequences

    def __iter__(self) -> Iterator[torch.Tensor]:
        gen = torch.Generator().manual_seed(self.seed)
        produced = 0
        while self.num_sequences is None or produced < self.num_sequences:
            yield torch.randint(0, self.vocab_size, (self.seq_len + 1,), generator=gen, dtype=torch.long)
            produced += 1


class RankShardIterableDataset(IterableDataset):
    """Strides an iterable dataset so each rank sees a disjoint shard."""

    def __init__(self, dataset: IterableDataset, rank: int, world_size: int) -> None:
        super().__init__()
        if rank < 0 or world_size <= 0 or rank >= world_size:
            raise ValueError(f"invalid rank/world_size: rank={rank}, world_size={world_size}")
        self.dataset = dataset
        self.rank = rank
        self.world_size = world_size

    def __iter__(self):
        for idx, sample in enumerate(self.dataset):
            if idx % self.world_size == self.rank:
                yield sample
