"""Token streams for training, with the reference's names (data/fineweb.py).

- SyntheticPatternDataset reproduces the reference's ramp stream exactly
  (data/fineweb.py:100-122): chunk i is (cursor + arange(S+1)) % V with the
  cursor advancing by S+1 modulo V.  Its bytes are part of the contract.
- SyntheticUniformDataset (not in the reference): iid uniform ids over
  [0, V) from one seeded torch.Generator, one [S+1] draw per chunk; the
  benchmark workloads' synthetic data.
- PackedFineWebDataset packs any text stream with any tokenizer into
  [S+1] chunks (documents separated by EOS), through TokenPacker, a fixed
  buffer that is filled and emitted in place.
- RankShardIterableDataset strides a stream over ranks.
- The Hugging Face pieces the reference's `--data-mode fineweb` needs (the
  meta-llama tokenizer and the FineWeb-Edu stream, data/fineweb.py:17-55)
  are downloads, which this build does not do: load_llama_tokenizer and
  load_fineweb_stream raise FineWebUnavailable with what to use instead, and
  the trainers' --allow-synthetic-fallback switches to synthetic data as the
  reference's does.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass
from typing import Iterable, Iterator, List, Optional, Sequence

import torch
from torch.utils.data import IterableDataset


class FineWebUnavailable(RuntimeError):
    """The real-data pipeline needs network downloads this build does not make."""


_OFFLINE_HINT = ("use --data-mode synthetic or --data-mode synthetic-uniform, or pass "
                 "--allow-synthetic-fallback; PackedFineWebDataset also packs any local text "
                 "iterable with a tokenizer object you supply")


@dataclass
class TokenizerBundle:
    tokenizer: object
    vocab_size: int
    eos_token_id: int


def load_llama_tokenizer(tokenizer_name: str) -> TokenizerBundle:
    raise FineWebUnavailable(f"tokenizer '{tokenizer_name}' would be downloaded from the Hugging Face hub; "
                             + _OFFLINE_HINT)


def load_fineweb_stream(subset: str, split: str = "train", shuffle_buffer: int = 10_000, seed: int = 42):
    raise FineWebUnavailable(f"FineWeb-Edu '{subset}/{split}' would be streamed from the Hugging Face hub; "
                             + _OFFLINE_HINT)


class TokenPacker:
    """Concatenates token id sequences into fixed chunks of `chunk_len`
    ids.  Ids are written into one preallocated int64 buffer at a cursor;
    whenever the buffer is full it is emitted (as a copy) and the cursor
    restarts, so a long document fills several chunks and its tail starts
    the next one."""

    def __init__(self, chunk_len: int) -> None:
        if chunk_len <= 0:
            raise ValueError("chunk_len must be positive")
        self.chunk_len = chunk_len
        self._buf = torch.empty(chunk_len, dtype=torch.long)
        self._fill = 0

    def push(self, ids: Sequence[int]) -> List[torch.Tensor]:
        out: List[torch.Tensor] = []
        src = torch.as_tensor(ids, dtype=torch.long).reshape(-1)
        pos = 0
        while pos < src.numel():
            take = min(self.chunk_len - self._fill, src.numel() - pos)
            self._buf[self._fill:self._fill + take] = src[pos:pos + take]
            self._fill += take
            pos += take
            if self._fill == self.chunk_len:
                out.append(self._buf.clone())
                self._fill = 0
        return out


class PackedFineWebDataset(IterableDataset):
    """Packs rows of a text stream (dicts holding `text_key`, or strings) into
    [seq_len + 1] token chunks with `tokenizer.encode(text,
    add_special_tokens=False)`, appending `eos_token_id` after each
    non-empty document when add_eos_between_samples is set."""

    def __init__(self, text_iterable: Iterable, tokenizer, seq_len: int, eos_token_id: int, text_key: str = "text",
                 add_eos_between_samples: bool = True) -> None:
        super().__init__()
        self.text_iterable = text_iterable
        self.tokenizer = tokenizer
        self.seq_len = seq_len
        self.eos_token_id = eos_token_id
        self.text_key = text_key
        self.add_eos_between_samples = add_eos_between_samples

    def _texts(self) -> Iterator[str]:
        for row in self.text_iterable:
            text = row.get(self.text_key, "") if isinstance(row, dict) else str(row)
            if text:
                yield text

    def __iter__(self) -> Iterator[torch.Tensor]:
        packer = TokenPacker(self.seq_len + 1)
        eos = [self.eos_token_id] if self.add_eos_between_samples else []
        for text in self._texts():
            ids = list(self.tokenizer.encode(text, add_special_tokens=False))
            if ids:
                yield from packer.push(ids + eos)


class SyntheticPatternDataset(IterableDataset):
    """Deterministic ramp chunks (cursor + arange(S+1)) % V, the cursor
    advancing by S+1 modulo V (data/fineweb.py:100-122)."""

    def __init__(self, seq_len: int, vocab_size: int, num_sequences: Optional[int] = None) -> None:
        super().__init__()
        self.seq_len = seq_len
        self.vocab_size = vocab_size
        self.num_sequences = num_sequences

    def __iter__(self) -> Iterator[torch.Tensor]:
        length = self.seq_len + 1
        counter = itertools.count() if self.num_sequences is None else range(self.num_sequences)
        for i in counter:
            start = (i * length) % self.vocab_size
            yield torch.arange(start, start + length, dtype=torch.long) % self.vocab_size


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
        counter = itertools.count() if self.num_sequences is None else range(self.num_sequences)
        for _ in counter:
            yield torch.randint(0, self.vocab_size, (self.seq_len + 1,), generator=gen, dtype=torch.long)


class RankShardIterableDataset(IterableDataset):
    """Rank r of world_size sees items r, r + world_size, ... of the stream."""

    def __init__(self, dataset: IterableDataset, rank: int, world_size: int) -> None:
        super().__init__()
        if world_size <= 0 or not 0 <= rank < world_size:
            raise ValueError(f"invalid rank/world_size: rank={rank}, world_size={world_size}")
        self.dataset = dataset
        self.rank = rank
        self.world_size = world_size

    def __iter__(self):
        return itertools.islice(iter(self.dataset), self.rank, None, self.world_size)
