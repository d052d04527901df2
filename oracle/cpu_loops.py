"""ORACLE — test infrastructure, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

The reference's CPU pooling, restated with torch CPU operators:
  baseline_loop       baseline/infer.py:253-266: per field, clamp the ids to [0, V-1], look the
                      rows up (F.embedding), torch.segment_reduce(sum, initial=0) over the bag
                      offsets, then concatenate the fields along dim 1 (mean divides by the bag
                      length, empty bag -> 0)
  embedding_bag_loop  the same per-field loop with F.embedding_bag(mode=sum|mean,
                      include_last_offset=True), the "PyTorch embedding_bag loop"
Inputs are the global layout: values [nnz], offsets [F*B+1], and F CPU tables.
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as Fn


def _field(values, offsets, f, batch):
    s = int(offsets[f * batch])
    e = int(offsets[(f + 1) * batch])
    local = offsets[f * batch:(f + 1) * batch + 1] - s
    return values[s:e], local


def baseline_loop(values: torch.Tensor, offsets: torch.Tensor, tables: Sequence[torch.Tensor], pooling: str = "sum",
                  batch: int = None) -> torch.Tensor:
    F = len(tables)
    batch = (offsets.numel() - 1) // F if batch is None else batch
    pooled = []
    for f, w in enumerate(tables):
        v, local = _field(values, offsets, f, batch)
        v = v.clamp(0, w.shape[0] - 1)
        emb = Fn.embedding(v, w)
        res = torch.segment_reduce(emb, reduce="sum", offsets=local, initial=0)
        if pooling == "mean":
            L = (local[1:] - local[:-1]).to(res.dtype).clamp(min=1)
            res = res / L[:, None]
        pooled.append(res)
    return torch.cat(pooled, dim=1)


def embedding_bag_loop(values: torch.Tensor, offsets: torch.Tensor, tables: Sequence[torch.Tensor],
                       pooling: str = "sum", batch: int = None) -> torch.Tensor:
    F = len(tables)
    batch = (offsets.numel() - 1) // F if batch is None else batch
    pooled = []
    for f, w in enumerate(tables):
        v, local = _field(values, offsets, f, batch)
        v = v.clamp(0, w.shape[0] - 1)
        pooled.append(Fn.embedding_bag(v, w, local, mode=pooling, include_last_offset=True))
    return torch.cat(pooled, dim=1)
