"""Integer index maps of the ZeRO flat layouts (bit-exact), restated in numpy.

  flat_layout     zero/common.py:59-96  (dedupe by identity, prefix offsets)
  shard_spec      zero/common.py:99-111 (chunk = max(1, ceil(P/ws)))
  stage3_handles  zero/stage3_optimizer.py:313-349 (one handle per module,
                  tied LM head reusing the embedding's handle)
  bucket_plan     25M-element gradient buckets whose concatenation is the flat
                  layout (the bucketing has no reference counterpart; it is
                  pinned to the reference's per-handle layout by concatenation)
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import numpy as np

from .model import Cfg, param_specs


def flat_layout(shapes: Sequence[Tuple[int, ...]]) -> Tuple[np.ndarray, np.ndarray, int]:
    """offsets (int64), numels (int64), total for parameters in order."""
    numels = np.array([int(np.prod(s, dtype=np.int64)) for s in shapes], dtype=np.int64)
    offsets = np.zeros(len(shapes), dtype=np.int64)
    if len(shapes) > 1:
        offsets[1:] = np.cumsum(numels[:-1])
    return offsets, numels, int(numels.sum())


def shard_spec(total: int, rank: int, world_size: int) -> Dict[str, int]:
    chunk = max(1, math.ceil(total / world_size))
    start = rank * chunk
    end = min(start + chunk, total)
    return {
        "rank": rank,
        "world_size": world_size,
        "shard_start": start,
        "shard_end": end,
        "shard_numel": max(0, end - start),
        "chunk_size": chunk,
    }


def model_param_names(cfg: Cfg) -> List[str]:
    return [n for n, _ in param_specs(cfg)]


def stage3_handles(cfg: Cfg) -> List[Dict[str, object]]:
    """Handles in creation order: name, module_names, param names (flat order)."""
    handles: List[Dict[str, object]] = []
    emb = {"name": "tok_embeddings", "module_names": ["tok_embeddings"], "params": ["tok_embeddings.weight"]}
    handles.append(emb)
    specs = param_specs(cfg)
    for i in range(cfg.n_layers):
        names = [n for n, _ in specs if n.startswith(f"layers.{i}.")]
        handles.append({"name": f"layers.{i}", "module_names": [f"layers.{i}"], "params": names})
    handles.append({"name": "norm", "module_names": ["norm"], "params": ["norm.weight"]})
    if cfg.tie_word_embeddings:
        emb["module_names"].append("lm_head")
    else:
        handles.append({"name": "lm_head", "module_names": ["lm_head"], "params": ["lm_head.weight"]})
    return handles


def bucket_plan(total: int, bucket_numel: int = 25_000_000) -> List[Tuple[int, int]]:
    if bucket_numel <= 0:
        raise ValueError("bucket_numel must be positive")
    return [(s, min(s + bucket_numel, total)) for s in range(0, total, bucket_numel)]
