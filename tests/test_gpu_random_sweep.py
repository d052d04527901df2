"""Seeded random sweep of the pooling entry points against the oracle, on the GPU.

Each case draws the slot count, batch, per-slot widths and vocabularies (including one-row
tables), the table and output dtypes, the pooling, the index type, a mix of bag lengths with
long bags, and one of the execution paths (no split, the per-shape default, every bag split,
the length-binning pass with random thresholds). Tables hold small integers (int8 tables: small
integers times a power-of-two scale), so every partial sum is exact and every path, split or
not, must equal the oracle's result bit for bit. A second pass with N(0, 1) tables holds the
unsplit path to bit equality and the split paths to the fp32 reassociation bound.
"""
import numpy as np
import pytest
import torch

from _cases import make_ids
from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
NO_SPLIT = 2 ** 31 - 1
WIDTHS = [1, 3, 4, 8, 16, 24, 32, 48, 64, 100, 128, 256, 512, 1024]


def draw(seed):
    rng = np.random.default_rng(seed)
    F = int(rng.choice([1, 2, 3, 7, 28, 40]))
    B = int(rng.choice([1, 2, 7, 64, 257, 600]))
    if rng.random() < 0.5:
        dims = [int(rng.choice(WIDTHS))] * F
    else:
        dims = [int(rng.choice(WIDTHS)) for _ in range(F)]
    while sum(dims) * B > 4_000_000:  # keep each case small
        dims = [max(1, d // 2) for d in dims]
    vocab = [int(rng.choice([1, 2, 17, 300, 5000])) for _ in range(F)]
    vocab = [max(1, min(V, 262_144 // D)) for V, D in zip(vocab, dims)]  # <= 1 MiB of fp32 per table
    tdt = str(rng.choice(["f32", "bf16", "f16", "i8"]))
    odt = str(rng.choice(["f32", "bf16", "f16"])) if tdt != "i8" else str(rng.choice(["f32", "bf16"]))
    pooling = str(rng.choice(["sum", "mean"]))
    kind = str(rng.choice(["geometric", "uniform", "fixed", "heavy"]))
    if kind == "geometric":
        L = np.clip(rng.geometric(1 / 9, (F, B)) - 1, 0, 256)
    elif kind == "uniform":
        L = rng.integers(0, 40, (F, B))
    elif kind == "fixed":
        L = np.full((F, B), int(rng.integers(0, 12)))
    else:  # mostly short, a few very long
        L = rng.integers(0, 6, (F, B))
        L[rng.random((F, B)) < 0.02] = int(rng.integers(200, 3000))
    path = str(rng.choice(["nosplit", "default", "allsplit", "bins"]))
    idx = str(rng.choice(["i64", "i32"]))
    return dict(rng=rng, F=F, B=B, dims=dims, vocab=vocab, tdt=tdt, odt=odt, pooling=pooling, L=L, path=path,
                idx=idx, kind=kind)


def tables_for(rng, c, integer):
    out = []
    for V, D in zip(c["vocab"], c["dims"]):
        if c["tdt"] == "i8":
            q = rng.integers(-127, 128, (V, D)).astype(np.int8)
            # powers of two in [2^-7, 2^-4]: products and sums of up to 3000 rows fit 24 bits exactly
            scale = (2.0 ** rng.integers(-7, -3, V)).astype(np.float32)
            if not integer:
                scale = (scale * (1 + rng.random(V))).astype(np.float32)
            out.append((q, scale))
        else:
            x = rng.integers(-16, 17, (V, D)).astype(np.float32) if integer else \
                rng.standard_normal((V, D)).astype(np.float32)
            out.append(orc.encode(x, c["tdt"]))
    return out


def run(pkg, dev, c, values, offsets, tables):
    v = torch.from_numpy(values).to(dev, torch.int32 if c["idx"] == "i32" else torch.int64)
    o = torch.from_numpy(offsets).to(dev)
    if c["tdt"] == "i8":
        tt = [(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)) for q, s in tables]
    else:
        tt = []
        for t in tables:
            x = torch.from_numpy(np.ascontiguousarray(t))
            tt.append((x if c["tdt"] == "f32" else x.view(torch.int16).view(TORCH_DT[c["tdt"]])).to(dev))
    kw = {"nosplit": dict(long_threshold=NO_SPLIT), "default": {}, "allsplit": dict(long_threshold=-1),
          "bins": dict(use_bins=True, block_threshold=int(c["rng"].choice([0, 8, 40, 100])),
                       split_threshold=int(c["rng"].choice([0, 50, 300])))}[c["path"]]
    out = pkg.embedding_bag_pooled(v, o, tt, pooling=c["pooling"], out_dtype=TORCH_DT[c["odt"]], **kw)
    torch.cuda.synchronize()
    out = out.cpu()
    return out.numpy() if c["odt"] == "f32" else out.view(torch.int16).numpy().view(np.uint16)


def case_arrays(c):
    rng, F, B, L = c["rng"], c["F"], c["B"], c["L"]
    ids = [make_ids(rng, int(L[f].sum()), c["vocab"][f]) for f in range(F)]
    values = np.concatenate(ids) if L.sum() else np.zeros(0, np.int64)
    offsets = np.zeros(F * B + 1, np.int64)
    np.cumsum(L.reshape(-1), out=offsets[1:])
    if c["idx"] == "i32":
        values = np.clip(values, -2 ** 31, 2 ** 31 - 1).astype(np.int32)  # saturating, as the stager narrows
    return values, offsets


def f64_bound(values, offsets, tables, c):
    """fp64 pooling of the decoded rows and the fp32 reassociation bound of each element."""
    F, B = c["F"], c["B"]
    outs, bounds = [], []
    for f in range(F):
        if c["tdt"] == "i8":
            q, s = tables[f]
            w = q.astype(np.float64) * s.astype(np.float64)[:, None]
        else:
            w = orc.decode(tables[f], c["tdt"]).astype(np.float64)
        acc = np.zeros((B, w.shape[1]))
        bnd = np.zeros_like(acc)
        for b in range(B):
            s0, e0 = offsets[f * B + b], offsets[f * B + b + 1]
            if e0 > s0:
                rows = w[np.clip(values[s0:e0].astype(np.int64), 0, w.shape[0] - 1)]
                acc[b] = rows.sum(axis=0)
                bnd[b] = np.abs(rows).sum(axis=0) * (e0 - s0) * 2.0 ** -24
                if c["pooling"] == "mean":
                    acc[b] /= (e0 - s0)
                    bnd[b] /= (e0 - s0)
        outs.append(acc)
        bounds.append(bnd)
    return np.concatenate(outs, axis=1), np.concatenate(bounds, axis=1)


@pytest.mark.parametrize("seed", range(160))
def test_random_case_integer_tables_bitwise(pkg, dev, seed):
    c = draw(seed)
    print(f"sweep seed={seed} F={c['F']} B={c['B']} dims={sorted(set(c['dims']))} tdt={c['tdt']} odt={c['odt']} "
          f"{c['pooling']} {c['kind']} path={c['path']} idx={c['idx']}", flush=True)
    values, offsets = case_arrays(c)
    tables = tables_for(c["rng"], c, integer=True)
    want = orc.pool_c(values, offsets, tables, c["tdt"], c["pooling"], c["odt"])
    got = run(pkg, dev, c, values, offsets, tables)
    assert np.array_equal(got, want), f"{(got != want).sum()} of {got.size} elements differ"


@pytest.mark.parametrize("seed", range(1000, 1064))
def test_random_case_normal_tables(pkg, dev, seed):
    c = draw(seed)
    print(f"sweep seed={seed} F={c['F']} B={c['B']} dims={sorted(set(c['dims']))} tdt={c['tdt']} odt={c['odt']} "
          f"{c['pooling']} {c['kind']} path={c['path']} idx={c['idx']}", flush=True)
    values, offsets = case_arrays(c)
    tables = tables_for(c["rng"], c, integer=False)
    got = run(pkg, dev, c, values, offsets, tables)
    if c["path"] == "nosplit":
        want = orc.pool_c(values, offsets, tables, c["tdt"], c["pooling"], c["odt"])
        assert np.array_equal(got, want), f"{(got != want).sum()} of {got.size} elements differ"
        return
    ref64, bound = f64_bound(values, offsets, tables, c)
    g = orc.decode(got, c["odt"]).astype(np.float64)
    rnd = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}[c["odt"]]
    tol = bound * (1 + rnd) + np.abs(ref64) * rnd + 1e-30
    if c["odt"] == "f16":
        tol = tol + 2.0 ** -25  # fp16 subnormal spacing
    if c["tdt"] == "i8":
        # one fma per element: the oracle's products are rounded once inside the fma, the fp64
        # reference is exact; each product contributes at most half an fp32 ulp more
        tol = tol + bound
    bad = np.abs(g - ref64) > tol
    assert not bad.any(), f"{bad.sum()} elements outside the bound; worst {np.abs(g - ref64)[bad].max():.3e}"


def _ref_layout(L):
    F, B = L.shape
    ro = np.zeros((F, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    return ro.reshape(-1), vo


@pytest.mark.parametrize("seed", range(2000, 2048))
def test_random_reference_layout_and_fused_layernorm(pkg, dev, seed):
    """The reference-layout entry points on one shared table: the pooled block bit for bit
    (integer table), int64 or int32 ids and offsets; where the fused LayerNorm covers the shape,
    LayerNorm(pooled) within the LayerNorm tolerance of the oracle's."""
    c = draw(seed)
    rng = c["rng"]
    tdt = c["tdt"] if c["tdt"] != "i8" else "bf16"
    D, V, F, B, L = c["dims"][0], c["vocab"][0], c["F"], c["B"], c["L"]
    print(f"sweep seed={seed} F={F} B={B} D={D} V={V} tdt={tdt} {c['kind']} idx={c['idx']}", flush=True)
    ids = make_ids(rng, int(L.sum()), V)
    ro, vo = _ref_layout(L)
    w = orc.encode(rng.integers(-16, 17, (V, D)).astype(np.float32), tdt)
    want = orc.pool_c(ids, ro, [w] * F, tdt, "sum", tdt, batch=B, val_base=vo)
    wt = torch.from_numpy(np.ascontiguousarray(w))
    wt = (wt if tdt == "f32" else wt.view(torch.int16).view(TORCH_DT[tdt])).to(dev)
    it = torch.int32 if c["idx"] == "i32" else torch.int64
    v = torch.from_numpy(np.clip(ids, -2 ** 31, 2 ** 31 - 1) if it == torch.int32 else ids).to(dev, it)
    vo_t, ro_t = torch.from_numpy(vo).to(dev, it), torch.from_numpy(ro).to(dev, it)
    out = torch.empty((B, F * D), dtype=wt.dtype, device=dev)
    pkg.fused_all_slots_embedding(v, vo_t, ro_t, wt, out, B, D, V - 1)
    torch.cuda.synchronize()
    got = out.cpu()
    got = got.numpy() if tdt == "f32" else got.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    if tdt == "f16":
        return  # the fused LayerNorm covers fp32 / bf16 tables
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(F * D)).astype(np.float32)).to(dev)
    bb = torch.from_numpy((0.1 * rng.standard_normal(F * D)).astype(np.float32)).to(dev)
    norm = torch.empty_like(out)
    pkg.fused_all_slots_embedding_layernorm(v, vo_t, ro_t, wt, norm, B, D, V - 1, g, bb, 1e-5)
    torch.cuda.synchronize()
    y, _, _ = orc.layer_norm_np(orc.decode(want, tdt), g.cpu().numpy(), bb.cpu().numpy(), 1e-5)
    gotn = norm.float().cpu().numpy()
    tol = 2e-5 + np.abs(y) * (1e-5 if tdt == "f32" else 2.0 ** -8)
    assert (np.abs(gotn - y) <= tol).all(), np.abs(gotn - y).max()
