"""Synthetic token streams (data/fineweb.py:100-139, train.py:139-145).

  ramp_chunks     SyntheticPatternDataset: (cursor + arange(S+1)) % V, the
                  cursor advancing by S+1 modulo V.
  uniform_chunks  iid uniform ids over [0, V) from one torch.Generator seeded
                  once, one [B, S+1] draw per micro-batch (the benchmark
                  workloads' "synthetic uniform token ids").
  split_chunk     inputs = chunk[:, :-1]; labels = inputs (the shift is inside
                  the loss).
"""
from __future__ import annotations

from typing import Iterator, Tuple

import torch


def ramp_chunks(seq_len: int, vocab_size: int, batch_size: int) -> Iterator[torch.Tensor]:
    cursor = 0
    while True:
        rows = []
        for _ in range(batch_size):
            length = seq_len + 1
            rows.append(torch.arange(cursor, cursor + length, dtype=torch.long) % vocab_size)
            cursor = (cursor + length) % vocab_size
        yield torch.stack(rows, 0)


def uniform_chunks(seq_len: int, vocab_size: int, batch_size: int, seed: int) -> Iterator[torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    while True:
        yield torch.randint(0, vocab_size, (batch_size, seq_len + 1), generator=gen, dtype=torch.long)


def split_chunk(chunk: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    inputs = chunk[:, :-1].contiguous()
    return inputs, inputs.clone()
