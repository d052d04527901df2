"""Seeded synthetic workloads of the fused embedding-bag path (no dataset ships with the path).

Six shapes, all with 28 fields in the flat field-major layout (values + global offsets):

  small-fp32   fp32 tables 10,000 x 64, B=256, Poisson(3) lengths clipped to [0, 32] plus
               ~10% empty bags, uniform ids, sum
  fp32-1m      fp32 tables 1,000,000 x 128, B=4096, geometric lengths (mean 8) clipped to
               [0, 256], Zipf(1.1) ids, sum
  bf16-2m      bf16 tables 2,000,000 x 128, B=4096, lengths and ids as fp32-1m, mean pooling,
               bf16 output [4096, 28*128] (the headline shape)
  hetero-bf16  bf16 tables with widths cycling 32/64/128 and log-uniform vocabularies in
               [1e3, 5e6], B=8192; 20 short fields Poisson(2) and 8 long fields with
               lognormal lengths (median 64) clipped to [1, 2048]; 5% empty bags; sum
  lazy-32k     bf16 tables 4,000,000 x 128, B=32768 = 8 sub-batches of 4096 with Poisson
               lengths of mean 1, 4 or 16, concatenated field by field; Zipf(0.8) ids; mean
  reference-5m the reference's own shape: one shared bf16 table 5,000,000 x 512 (5.12 GB) for
               all 28 slots, B=4096, lengths and ids as bf16-2m, sum

Five shapes come from the path's benchmark configurations; reference-5m is the reference's own.

Choices the shape descriptions leave open: rows ~ N(0, 0.01); lengths "geometric(mean 8)" are
Geometric(p=1/9) - 1 on {0, 1, ...}; the small config forces each bag empty with q = 0.0528 on
top of Poisson(3) (about 10% empty in total); bounded Zipf draws rank r in [0, V) with
P(r) ~ (r+1)^-s by inverse CDF and maps it to row (a*r + c) mod V with gcd(a, V) = 1, so hot
rows are scattered; per-field random streams come from numpy SeedSequence(seed).spawn(28).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from functools import lru_cache
from typing import List, Optional

import numpy as np
import torch

NUM_FIELDS = 28


@dataclass
class Workload:
    name: str
    batch: int
    dims: List[int]
    vocab: List[int]
    table_dtype: torch.dtype
    out_dtype: torch.dtype
    pooling: str
    values: np.ndarray            # int64 [nnz]
    offsets: np.ndarray           # int64 [F*B+1]
    seed: int
    sub_batches: Optional[list] = field(default=None)  # lazy-32k: per sub-batch flat layouts

    @property
    def num_fields(self) -> int:
        return len(self.dims)

    @property
    def nnz(self) -> int:
        return int(self.values.shape[0])

    @property
    def num_bags(self) -> int:
        return self.batch * self.num_fields

    def lengths(self) -> np.ndarray:
        return np.diff(self.offsets)

    def bytes_algorithmic(self, int8: bool = False, index_bytes: int = 0) -> int:
        """Each lookup's row once, plus indices, offsets and the output (logical bytes).
        With ``int8`` the rows are int8 row-quantised: 1 byte per element + a 4-byte scale.
        ``index_bytes``: bytes per id as the kernel reads them (0: the generated int64)."""
        tb = 1 if int8 else torch.tensor([], dtype=self.table_dtype).element_size()
        extra = 4 if int8 else 0
        ob = torch.tensor([], dtype=self.out_dtype).element_size()
        L = self.lengths().reshape(self.num_fields, self.batch).sum(axis=1)
        rows = int(sum(int(L[f]) * (self.dims[f] * tb + extra) for f in range(self.num_fields)))
        ib = index_bytes or self.values.itemsize
        return rows + self.nnz * ib + self.offsets.size * 8 + self.batch * sum(self.dims) * ob

    def bytes_compulsory(self, int8: bool = False, index_bytes: int = 0) -> int:
        """As bytes_algorithmic, but each distinct (field, row) read once."""
        tb = 1 if int8 else torch.tensor([], dtype=self.table_dtype).element_size()
        extra = 4 if int8 else 0
        ob = torch.tensor([], dtype=self.out_dtype).element_size()
        total = 0
        for f in range(self.num_fields):
            s, e = int(self.offsets[f * self.batch]), int(self.offsets[(f + 1) * self.batch])
            rows = np.clip(self.values[s:e], 0, self.vocab[f] - 1)
            total += np.unique(rows).size * (self.dims[f] * tb + extra)
        ib = index_bytes or self.values.itemsize
        return total + self.nnz * ib + self.offsets.size * 8 + self.batch * sum(self.dims) * ob


@lru_cache(maxsize=4)
def _zipf_cdf(vocab: int, s: float) -> np.ndarray:
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    c = np.cumsum(w)
    c /= c[-1]
    return c


def row_permutation(rng: np.random.Generator, vocab: int):
    """(a, c) with gcd(a, vocab) = 1: rank r -> row (a*r + c) mod vocab is a bijection."""
    while True:
        a = int(rng.integers(1, vocab)) if vocab > 1 else 1
        if math.gcd(a, vocab) == 1:
            break
    return a, int(rng.integers(0, vocab))


def zipf_rows(rng: np.random.Generator, n: int, vocab: int, s: float, perm) -> np.ndarray:
    """n bounded Zipf(s) ranks over [0, vocab) mapped to rows through the permutation `perm`."""
    cdf = _zipf_cdf(vocab, s)
    r = np.searchsorted(cdf, rng.random(n), side="right").astype(np.int64)
    np.minimum(r, vocab - 1, out=r)
    a, c = perm
    return (a * r + c) % vocab


def _finish(name, batch, dims, vocab, tdt, odt, pooling, lengths, ids, seed, sub=None) -> Workload:
    L = np.concatenate(lengths).astype(np.int64)
    offsets = np.zeros(L.size + 1, dtype=np.int64)
    np.cumsum(L, out=offsets[1:])
    values = np.concatenate(ids).astype(np.int64) if ids else np.zeros(0, np.int64)
    return Workload(name, batch, list(dims), list(vocab), tdt, odt, pooling, values, offsets, seed, sub)


def _streams(seed: int) -> List[np.random.Generator]:
    return [np.random.default_rng(s) for s in np.random.SeedSequence(seed).spawn(NUM_FIELDS)]


def small_fp32(seed: int = 0, batch: int = 256) -> Workload:
    V, D = 10_000, 64
    lengths, ids = [], []
    for rng in _streams(seed):
        L = np.clip(rng.poisson(3.0, batch), 0, 32)
        L[rng.random(batch) < 0.0528] = 0
        lengths.append(L)
        ids.append(rng.integers(0, V, int(L.sum())))
    return _finish("small-fp32", batch, [D] * NUM_FIELDS, [V] * NUM_FIELDS, torch.float32, torch.float32,
                   "sum", lengths, ids, seed)


def _geometric_zipf(name, seed, batch, V, D, tdt, odt, pooling, s=1.1) -> Workload:
    lengths, ids = [], []
    for rng in _streams(seed):
        perm = row_permutation(rng, V)
        L = np.clip(rng.geometric(1.0 / 9.0, batch) - 1, 0, 256)
        lengths.append(L)
        ids.append(zipf_rows(rng, int(L.sum()), V, s, perm))
    return _finish(name, batch, [D] * NUM_FIELDS, [V] * NUM_FIELDS, tdt, odt, pooling, lengths, ids, seed)


def fp32_1m(seed: int = 0, batch: int = 4096, vocab: int = 1_000_000) -> Workload:
    return _geometric_zipf("fp32-1m", seed, batch, vocab, 128, torch.float32, torch.float32, "sum")


def bf16_2m(seed: int = 0, batch: int = 4096, vocab: int = 2_000_000) -> Workload:
    return _geometric_zipf("bf16-2m", seed, batch, vocab, 128, torch.bfloat16, torch.bfloat16, "mean")


def reference_5m(seed: int = 0, batch: int = 4096, vocab: int = 5_000_000) -> Workload:
    """The reference's own table shape: 28 slots over one shared bf16 nn.Embedding(5,000,000,
    512) (online_best/infer.py:948, :2757-2771), summed (:819-827); lengths and Zipf(1.1) ids as
    bf16-2m, each slot with its own popularity order over the shared rows."""
    return _geometric_zipf("reference-5m", seed, batch, vocab, 512, torch.bfloat16, torch.bfloat16, "sum")


def hetero_bf16(seed: int = 0, batch: int = 8192, vocab_max: int = 5_000_000) -> Workload:
    lengths, ids, dims, vocab = [], [], [], []
    for f, rng in enumerate(_streams(seed)):
        V = int(round(math.exp(rng.uniform(math.log(1e3), math.log(vocab_max)))))
        D = (32, 64, 128)[f % 3]
        if f < 20:
            L = rng.poisson(2.0, batch)
        else:
            L = np.clip(np.rint(rng.lognormal(math.log(64.0), 1.0, batch)), 1, 2048).astype(np.int64)
        L[rng.random(batch) < 0.05] = 0
        lengths.append(L)
        ids.append(rng.integers(0, V, int(L.sum())))
        dims.append(D)
        vocab.append(V)
    return _finish("hetero-bf16", batch, dims, vocab, torch.bfloat16, torch.bfloat16, "sum", lengths, ids, seed)


def lazy_32k(seed: int = 0, sub_batch: int = 4096, num_sub: int = 8, vocab: int = 4_000_000) -> Workload:
    """8 sub-batches (own length distributions) merged field by field in sub-batch order."""
    lams = [(1.0, 4.0, 16.0)[k % 3] for k in range(num_sub)]
    streams = _streams(seed)
    per_field_len = [[] for _ in range(NUM_FIELDS)]
    per_field_ids = [[] for _ in range(NUM_FIELDS)]
    for f, rng in enumerate(streams):
        perm = row_permutation(rng, vocab)  # one popularity order per field, shared by sub-batches
        for k in range(num_sub):
            L = np.clip(rng.poisson(lams[k], sub_batch), 0, 2048)
            per_field_len[f].append(L)
            per_field_ids[f].append(zipf_rows(rng, int(L.sum()), vocab, 0.8, perm))
    # sub-batch k: flat layout (field-major) of its own bags
    subs = []
    for k in range(num_sub):
        lens = [per_field_len[f][k] for f in range(NUM_FIELDS)]
        ids = [per_field_ids[f][k] for f in range(NUM_FIELDS)]
        subs.append(_finish(f"lazy-32k[{k}]", sub_batch, [128] * NUM_FIELDS, [vocab] * NUM_FIELDS,
                            torch.bfloat16, torch.bfloat16, "mean", lens, ids, seed))
    merged_len = [np.concatenate(per_field_len[f]) for f in range(NUM_FIELDS)]
    merged_ids = [np.concatenate(per_field_ids[f]) for f in range(NUM_FIELDS)]
    return _finish("lazy-32k", sub_batch * num_sub, [128] * NUM_FIELDS, [vocab] * NUM_FIELDS, torch.bfloat16,
                   torch.bfloat16, "mean", merged_len, merged_ids, seed, subs)


CONFIGS = {
    "small-fp32": small_fp32,
    "fp32-1m": fp32_1m,
    "bf16-2m": bf16_2m,
    "hetero-bf16": hetero_bf16,
    "lazy-32k": lazy_32k,
    "reference-5m": reference_5m,
}


def make(name: str, seed: int = 0, **kw) -> Workload:
    return CONFIGS[name](seed=seed, **kw)


def make_tables(wl: Workload, device, seed: int = 0) -> List[torch.Tensor]:
    """One table per field, rows ~ N(0, 0.01), in the workload's table dtype (reference-5m: one
    table shared by all fields).

    The small config draws its rows on the host (numpy, seed) so that the same tables can be
    rebuilt anywhere; the large ones are drawn on the device (torch generator, seed + field).
    """
    device = torch.device(device)
    tables = []
    if wl.name == "reference-5m":  # one table shared by every slot, as the reference's nn.Embedding
        g = torch.Generator(device=device)
        g.manual_seed(seed * 1000)
        t = torch.empty((wl.vocab[0], wl.dims[0]), dtype=wl.table_dtype, device=device)
        t.normal_(0.0, 0.01, generator=g)
        return [t] * wl.num_fields
    if wl.name == "small-fp32":
        rng = np.random.default_rng(seed)
        for f in range(wl.num_fields):
            t = rng.normal(0.0, 0.01, size=(wl.vocab[f], wl.dims[f])).astype(np.float32)
            tables.append(torch.from_numpy(t).to(device=device, dtype=wl.table_dtype))
        return tables
    for f in range(wl.num_fields):
        g = torch.Generator(device=device)
        g.manual_seed(seed * 1000 + f)
        t = torch.empty((wl.vocab[f], wl.dims[f]), dtype=wl.table_dtype, device=device)
        t.normal_(0.0, 0.01, generator=g)
        tables.append(t)
    return tables


def to_device(wl: Workload, device, index_dtype=torch.int64):
    """(values, offsets) of the workload as device tensors."""
    v = torch.from_numpy(wl.values).to(device=device, dtype=index_dtype)
    o = torch.from_numpy(wl.offsets).to(device=device)
    return v, o
