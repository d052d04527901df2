"""Write the golden fixtures of the pooling path (run from the repository root:
``python tests/golden/make_golden.py``).

Each fixture's expected output comes from the oracle's C restatement and is cross-checked here,
before it is written, against torch's library routines in this container
(torch.segment_reduce after F.embedding, the loop of baseline/infer.py:256-263, and
F.embedding_bag): exactly for integer-valued and row-id tables, within the fp32 reassociation
bound otherwise. The reference repository ships no fixtures or golden vectors of its own.
"""
import os
import sys

import numpy as np
import torch
import torch.nn.functional as Fn

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from golden import fixture_io  # noqa: E402
from oracle import ebag_oracle as orc  # noqa: E402

I64_MAX = np.iinfo(np.int64).max
I64_MIN = np.iinfo(np.int64).min


def _offsets(lengths):
    o = np.zeros(lengths.size + 1, np.int64)
    np.cumsum(lengths.reshape(-1), out=o[1:])
    return o


def _torch_check(values, offsets, tables, tdt, pooling, batch):
    """fp64 segment_reduce pooling, its fp32 reassociation bound L * 2^-24 * sum|x| (per mean
    divided by L), and a check of fp32 F.embedding_bag against the two."""
    F = len(tables)
    got, bounds = [], []
    for f in range(F):
        s, e = int(offsets[f * batch]), int(offsets[(f + 1) * batch])
        w = torch.from_numpy(orc.decode(tables[f], tdt).astype(np.float64))
        v = torch.from_numpy(values[s:e]).clamp(0, w.shape[0] - 1)
        local = torch.from_numpy(offsets[f * batch:(f + 1) * batch + 1] - s)
        L = (local[1:] - local[:-1]).double()
        r = torch.segment_reduce(Fn.embedding(v, w), reduce="sum", offsets=local, initial=0)
        bound = torch.segment_reduce(Fn.embedding(v, w).abs(), reduce="sum", offsets=local, initial=0)
        bound = bound * L[:, None] * 2.0 ** -24
        if pooling == "mean":
            r = torch.where(L[:, None] > 0, r / L.clamp(min=1)[:, None], torch.zeros_like(r))
            bound = bound / L.clamp(min=1)[:, None]
        eb = Fn.embedding_bag(v, w.float(), local, mode=pooling, include_last_offset=True).double()
        assert torch.all((r - eb).abs() <= bound + 1e-30)
        got.append(r)
        bounds.append(bound)
    return torch.cat(got, dim=1).numpy(), torch.cat(bounds, dim=1).numpy()


def _touched_only(values, goff, tables, batch, shared):
    """Zero the rows no bag reads, so a fixture stores only the rows that matter."""
    out = []
    for f, t in enumerate(tables):
        if shared:
            used = np.clip(values, 0, t.shape[0] - 1)
        else:
            s, e = int(goff[f * batch]), int(goff[(f + 1) * batch])
            used = np.clip(values[s:e], 0, t.shape[0] - 1)
        keep = np.zeros(t.shape[0], bool)
        keep[used] = True
        out.append(np.where(keep[:, None], t, np.zeros_like(t)))
        if shared:
            return out * len(tables)
    return out


def _write(name, values, offsets, batch, tables, tdt, odt, pooling, exact=False, val_base=None, shared=False):
    values = np.asarray(values, np.int64)
    goff = offsets if val_base is None else orc.to_global_offsets(val_base, offsets, batch, len(values))
    tables = _touched_only(values, goff, tables, batch, shared)
    if val_base is not None:
        exp = orc.pool_c(values, offsets, tables, tdt, pooling, odt, batch=batch, val_base=val_base)
        goff = orc.to_global_offsets(val_base, offsets, batch, len(values))
    else:
        exp = orc.pool_c(values, offsets, tables, tdt, pooling, odt)
        goff = offsets
    ref64, bound = _torch_check(values, goff, tables, tdt, pooling, batch)
    got = orc.decode(exp, odt).astype(np.float64)
    if exact:
        assert np.array_equal(got, ref64), name
    else:
        # fp32 result: within the reassociation bound; 16-bit result: plus half an ulp of rounding
        tol = bound + (np.abs(ref64) * 2.0 ** -8 if odt == "bf16" else np.abs(ref64) * 2.0 ** -11 if odt == "f16"
                       else 0.0) + 1e-30
        assert np.all(np.abs(got - ref64) <= tol), name
    fixture_io.save(os.path.join(HERE, name + ".npz"), values, offsets, batch, tables, tdt, odt, pooling, exp,
                    val_base=val_base, shared=shared)


def edge_lengths(rng, F, B):
    L = rng.integers(0, 9, size=(F, B))
    L[:, -1] = 0                 # last bag of every field empty
    L[0, 0] = 0
    L[1, 1] = 256
    L[1, 2] = 2048
    L[2, 3] = 1
    return L


def edge_ids(rng, L, vocab):
    ids = []
    for f in range(L.shape[0]):
        n = int(L[f].sum())
        x = rng.integers(0, vocab[f], size=n)
        if n >= 8:
            x[:8] = [-1, vocab[f], I64_MAX, I64_MIN, 0, vocab[f] - 1, 3, 3]  # clamps and duplicates
        ids.append(x)
    return np.concatenate(ids).astype(np.int64)


def main():
    rng = np.random.default_rng(2024)
    # 1-2: mixed widths, clamp cases, empty/last-empty bags, a 256 and a 2048 bag
    dims, vocab, B = (32, 64, 128, 512), (7, 300, 1000, 50), 9
    L = edge_lengths(rng, 4, B)
    ids = edge_ids(rng, L, vocab)
    t32 = [rng.normal(0, 1, (vocab[f], dims[f])).astype(np.float32) for f in range(4)]
    _write("edge_mix_f32_sum", ids, _offsets(L), B, t32, "f32", "f32", "sum")
    tb = [orc.f32_to_bf16(t) for t in t32]
    _write("edge_mix_bf16_mean", ids, _offsets(L), B, tb, "bf16", "bf16", "mean")
    # 3: a field with no ids at all, fp16 tables, fp32 output
    L = rng.integers(0, 5, size=(3, 5))
    L[1] = 0
    ids = np.concatenate([rng.integers(0, 40, int(L[f].sum())) for f in range(3)])
    t16 = [orc.f32_to_f16(rng.normal(0, 1, (40, 64)).astype(np.float32)) for _ in range(3)]
    _write("all_empty_field_f16", ids, _offsets(L), 5, t16, "f16", "f32", "sum")
    # 4: a single sample, 28 fields
    L = rng.integers(0, 6, size=(28, 1))
    ids = np.concatenate([rng.integers(0, 500, int(L[f].sum())) for f in range(28)])
    t = [rng.normal(0, 0.01, (500, 64)).astype(np.float32) for _ in range(28)]
    _write("single_sample_f32", ids, _offsets(L), 1, t, "f32", "f32", "sum")
    # 5: a slice of the small fp32 shape: B=16, 28 fields, V=10000, D=64, Poisson(3) lengths
    L = np.clip(rng.poisson(3.0, size=(28, 16)), 0, 32)
    L[rng.random((28, 16)) < 0.0528] = 0
    ids = np.concatenate([rng.integers(0, 10_000, int(L[f].sum())) for f in range(28)])
    t = []
    for f in range(28):
        tf = np.zeros((10_000, 64), np.float32)
        s, e = int(L[:f].sum()), int(L[:f + 1].sum())
        rows = np.unique(ids[s:e])
        tf[rows] = rng.normal(0, 0.01, (rows.size, 64)).astype(np.float32)
        t.append(tf)
    _write("small_fp32_slice", ids, _offsets(L), 16, t, "f32", "f32", "sum")
    # 6: the reference layout with one shared bf16 table (online_best/infer.py:446-474, :805-827)
    S, B, V, D = 28, 6, 3000, 128
    L = rng.integers(0, 8, size=(S, B))
    ids = np.concatenate([rng.integers(-2, V + 2, int(L[s].sum())) for s in range(S)])
    w = np.zeros((V, D), np.float32)
    rows = np.unique(np.clip(ids, 0, V - 1))
    w[rows] = rng.normal(0, 0.05, (rows.size, D)).astype(np.float32)
    wb = orc.f32_to_bf16(w)
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    _write("reference_layout_bf16", ids, ro.reshape(-1), B, [wb] * S, "bf16", "bf16", "sum", val_base=vo,
           shared=True)
    # 7: integer-valued rows: every partial sum exact, so the check is bitwise
    L = rng.integers(0, 40, size=(3, 8))
    L[0, 0] = 2048
    ids = np.concatenate([rng.integers(0, 100, int(L[f].sum())) for f in range(3)])
    ti = [rng.integers(-32, 33, (100, 128)).astype(np.float32) for _ in range(3)]
    _write("int_exact_f32", ids, _offsets(L), 8, ti, "f32", "f32", "sum", exact=True)
    # 8: row-id table: bit j of the row id in column j; length-1 bags, clamps included
    V = 4096
    r = np.arange(V, dtype=np.int64)
    tr = ((r[:, None] >> np.arange(16)) & 1).astype(np.float32)
    ids = np.concatenate([rng.integers(0, V, 60), [-1, V, I64_MAX, I64_MIN]]).astype(np.int64)
    L = np.ones((1, ids.size), np.int64)
    _write("rowid_f32", ids, _offsets(L), ids.size, [tr], "f32", "f32", "sum", exact=True)
    # 9: one id repeated (duplicate rows), ternary bf16 rows (exact), fp32 output
    L = np.array([[50, 3, 0, 17]])
    ids = np.full(int(L.sum()), 5, np.int64)
    tt = [orc.f32_to_bf16(rng.integers(-1, 2, (10, 128)).astype(np.float32))]
    _write("duplicates_bf16", ids, _offsets(L), 4, tt, "bf16", "f32", "sum", exact=True)
    total = sum(os.path.getsize(os.path.join(HERE, f)) for f in os.listdir(HERE) if f.endswith(".npz"))
    print(f"fixtures written, {total / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
