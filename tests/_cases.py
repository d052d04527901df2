"""Seeded random pooling cases shared by the CPU and GPU tests."""
from __future__ import annotations

import numpy as np

from oracle import ebag_oracle as orc

I64_MAX = np.iinfo(np.int64).max
I64_MIN = np.iinfo(np.int64).min


def make_lengths(rng, F, B, max_len, empty_frac=0.1, long_every=0, long_len=0):
    L = rng.integers(0, max_len + 1, size=(F, B))
    L[rng.random((F, B)) < empty_frac] = 0
    if long_every and B:
        L[:, ::long_every] = long_len
    return L


def make_ids(rng, n, V, clamp_frac=0.05):
    ids = rng.integers(0, V, size=n).astype(np.int64)
    if n and clamp_frac:
        m = rng.random(n) < clamp_frac
        k = int(m.sum())
        ids[m] = rng.choice(np.array([-1, V, V + 7, -(2 ** 40), I64_MAX, I64_MIN], dtype=np.int64), size=k)
    return ids


def make_table(rng, V, D, dt, kind="normal"):
    if kind == "normal":
        x = rng.normal(0.0, 1.0, size=(V, D)).astype(np.float32)
    elif kind == "int":
        x = rng.integers(-32, 33, size=(V, D)).astype(np.float32)
    elif kind == "tern":
        x = rng.integers(-1, 2, size=(V, D)).astype(np.float32)
    else:
        raise ValueError(kind)
    return orc.encode(x, dt)


class Case:
    """A global-layout case: values, offsets[F*B+1], per-field tables (encoded)."""

    def __init__(self, values, lengths, tables, tdt):
        self.values = values
        self.lengths = lengths  # [F, B]
        F, B = lengths.shape
        self.F, self.B = F, B
        self.offsets = np.zeros(F * B + 1, dtype=np.int64)
        np.cumsum(lengths.reshape(-1), out=self.offsets[1:])
        self.tables = tables
        self.tdt = tdt

    def reference_layout(self):
        """(row_offsets[F*(B+1)], val_offsets[F]) of the same bags."""
        F, B = self.F, self.B
        ro = np.zeros((F, B + 1), dtype=np.int64)
        np.cumsum(self.lengths, axis=1, out=ro[:, 1:])
        vo = np.concatenate([[0], np.cumsum(self.lengths.sum(axis=1))[:-1]]).astype(np.int64)
        return ro.reshape(-1), vo


def random_case(seed, F=4, B=33, dims=(64,), V=(500,), max_len=20, tdt="f32", kind="normal",
                empty_frac=0.1, clamp_frac=0.05, long_every=0, long_len=0):
    rng = np.random.default_rng(seed)
    dims = [dims[f % len(dims)] for f in range(F)]
    vocab = [V[f % len(V)] for f in range(F)]
    L = make_lengths(rng, F, B, max_len, empty_frac, long_every, long_len)
    ids = np.concatenate([make_ids(rng, int(L[f].sum()), vocab[f], clamp_frac) for f in range(F)]) \
        if L.sum() else np.zeros(0, np.int64)
    tables = [make_table(rng, vocab[f], dims[f], tdt, kind) for f in range(F)]
    return Case(ids.astype(np.int64), L, tables, tdt)
