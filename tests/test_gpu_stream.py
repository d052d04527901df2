"""Streamed tiles on the GPU: 256-byte rows (bf16 / fp16 D = 128, fp32 D = 64) and 128-byte int8 rows
(D = 128, each row's scale read beside it) without binning and with the default short-bag limit,
where a wavefront walks a tile's rows in order across bag boundaries.

Bar: every bag, whatever its length, equals the oracle's sequential fp32 sum bit for bit (sum and
mean, every output type, int32 and int64 ids, with and without a dispatch order); malformed
offsets (decreasing, negative, past nnz), whose bags are not one contiguous run, pool exactly as
the oracle clamps them, in the global and the reference layout; an explicit short-bag limit
takes the length-ranked tiles instead.
"""
import numpy as np
import pytest
import torch

from _cases import make_ids, make_table, random_case
from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
SHAPES = [("bf16", 128), ("f16", 128), ("f32", 64)]


def to_dev(arr, tdt, dev):
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if tdt != "f32":
        t = t.view(torch.int16).view(TORCH_DT[tdt])
    return t.to(dev)


def to_np(t, odt):
    t = t.cpu()
    return t.numpy() if odt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def pooled(pkg, dev, values, offsets, tables, tdt, pooling, odt, idx=torch.int64, **kw):
    v = torch.from_numpy(np.ascontiguousarray(values)).to(dev, idx)
    o = torch.from_numpy(np.ascontiguousarray(offsets)).to(dev)
    out = pkg.embedding_bag_pooled(v, o, [to_dev(t, tdt, dev) for t in tables], pooling=pooling,
                                   out_dtype=TORCH_DT[odt], **kw)
    torch.cuda.synchronize()
    return to_np(out, odt)


@pytest.mark.parametrize("tdt,D", SHAPES)
@pytest.mark.parametrize("odt", ["same", "f32"])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
def test_every_length_bitwise(pkg, dev, tdt, D, odt, pooling, idx):
    odt = tdt if odt == "same" else odt
    print(f"stream {tdt} D={D} out={odt} {pooling} {idx}", flush=True)
    # lengths 0..60 with every fifth bag 300 rows: walks of many 64-row id chunks, bags ending
    # anywhere inside a 16-row step, runs of empty bags, and a short last tile (B = 37)
    case = random_case(D + len(tdt) + len(pooling), F=5, B=37, dims=(D,), V=(900,), max_len=60, tdt=tdt,
                       long_every=5, long_len=300)
    values = case.values if idx == torch.int64 else np.clip(case.values, -2 ** 31, 2 ** 31 - 1).astype(np.int32)
    want = orc.pool_c(values, case.offsets, case.tables, tdt, pooling, odt)
    got = pooled(pkg, dev, values, case.offsets, case.tables, tdt, pooling, odt, idx=idx)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("tdt,D", SHAPES)
def test_long_runs_and_empty_tiles(pkg, dev, tdt, D):
    """One bag of 5,000 rows among empty ones, tiles with no rows at all, and a single sample."""
    rng = np.random.default_rng(7)
    F, B, V = 3, 19, 4000
    L = np.zeros((F, B), np.int64)
    L[0, 9] = 5000
    L[1, :] = rng.integers(0, 3, B)
    L[2, 17:] = [64, 65]
    ids = make_ids(rng, int(L.sum()), V)
    offsets = np.concatenate([[0], np.cumsum(L.reshape(-1))]).astype(np.int64)
    tables = [make_table(rng, V, D, tdt) for _ in range(F)]
    for pooling in ("sum", "mean"):
        want = orc.pool_c(ids, offsets, tables, tdt, pooling, tdt)
        assert np.array_equal(pooled(pkg, dev, ids, offsets, tables, tdt, pooling, tdt), want), pooling
    one = np.array([0, 70], np.int64)
    want = orc.pool_c(ids[:70], one, tables[:1], tdt, "sum", tdt)
    assert np.array_equal(pooled(pkg, dev, ids[:70], one, tables[:1], tdt, "sum", tdt), want)


def _malformed(offsets, nnz, rng):
    """Offsets that step back, go negative and run past nnz in places (each bag is then what the
    clamps make of it: start in [0, nnz], end in [start, nnz])."""
    o = offsets.copy()
    n = o.size
    for k in rng.choice(np.arange(1, n - 1), size=max(1, n // 6), replace=False):
        o[k] = o[k] - int(rng.integers(1, 40))  # a decrease (possibly below zero)
    o[rng.integers(1, n - 1)] = -5
    o[rng.integers(1, n - 1)] = nnz + 9
    return o


@pytest.mark.parametrize("tdt,D,kind", [("bf16", 128, "normal"), ("f32", 64, "normal"), ("bf16", 256, "int")])
def test_malformed_global_offsets_match_oracle(pkg, dev, tdt, D, kind):
    # 256-wide bf16 rows take the ranked tiles, which split the long bags the bad offsets make:
    # integer rows keep those sums exact
    print(f"malformed global {tdt} D={D}", flush=True)
    rng = np.random.default_rng(D + 1)
    case = random_case(D + 2, F=4, B=45, dims=(D,), V=(700,), max_len=20, tdt=tdt, kind=kind)
    bad = _malformed(case.offsets, case.values.size, rng)
    for pooling in ("sum", "mean"):
        want = orc.pool_c(case.values, bad, case.tables, tdt, pooling, tdt)
        got = pooled(pkg, dev, case.values, bad, case.tables, tdt, pooling, tdt)
        assert np.array_equal(got, want), pooling


def test_malformed_reference_layout_matches_oracle(pkg, dev):
    rng = np.random.default_rng(3)
    S, B, V, D = 6, 30, 800, 128
    case = random_case(11, F=S, B=B, dims=(D,), V=(V,), max_len=20, tdt="bf16")
    ro, vo = case.reference_layout()
    ro = _malformed(ro, case.values.size, rng)
    w = torch.from_numpy(case.tables[0].view(np.int16)).view(torch.bfloat16).to(dev)
    out = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding(torch.from_numpy(case.values).to(dev), torch.from_numpy(vo).to(dev),
                                  torch.from_numpy(ro).to(dev), w, out, B, D, V - 1)
    torch.cuda.synchronize()
    want = orc.pool_c(case.values, ro, [case.tables[0]] * S, "bf16", "sum", "bf16", batch=B, val_base=vo)
    assert np.array_equal(to_np(out, "bf16"), want)


def test_explicit_short_bag_limit_takes_the_ranked_tiles(pkg, dev):
    """With a short-bag limit of the caller's, bags above it are split over the wavefront's lane
    groups (sums within the reassociation bound, not the sequential sum); the default streams."""
    case = random_case(5, F=3, B=40, dims=(128,), V=(600,), max_len=10, tdt="bf16", long_every=4, long_len=200)
    args = (case.values, case.offsets, case.tables, "bf16", "sum", "f32")
    want = orc.pool_c(*args)
    assert np.array_equal(pooled(pkg, dev, *args), want)
    split = pooled(pkg, dev, *args, long_threshold=-1)
    assert not np.array_equal(split, want)  # the split sums round differently somewhere
    np.testing.assert_allclose(split, want, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("tdt,D", [("bf16", 128), ("f32", 64)])
@pytest.mark.parametrize("odt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_special_values_streamed(pkg, dev, tdt, D, odt, pooling):
    """Inf, NaN, overflow, subnormals, signed zeros and bf16 / fp16 rounding ties in bags of one,
    two and three rows, through the streamed walk: finite and infinite results bit for bit, NaN
    where the oracle has NaN."""
    from test_gpu_parity import _special_rows
    table32 = _special_rows(D)
    table = orc.encode(table32, tdt)
    n = len(table32)
    bags = [[i] for i in range(n)] + [[i, j] for i in range(n) for j in range(n)] + \
           [[i, j, k] for i in range(0, n, 3) for j in range(1, n, 4) for k in range(2, n, 5)]
    np.random.default_rng(6).shuffle(bags)
    lens = np.array([len(x) for x in bags])
    values = np.concatenate([np.array(x, np.int64) for x in bags])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    got = pooled(pkg, dev, values, offsets, [table], tdt, pooling, odt)
    ref = orc.pool_c(values, offsets, [table], tdt, pooling, odt)
    g, r = orc.decode(got, odt), orc.decode(ref, odt)
    assert np.array_equal(np.isnan(g), np.isnan(r))
    fin = ~np.isnan(r)
    assert np.array_equal(got[fin], ref[fin])


def test_walks_ending_at_step_and_chunk_edges(pkg, dev):
    """Tiles (8 consecutive bags) whose rows number exactly a multiple of the 16-row step or of the
    64-row id chunk, one more or one less, with the rows in one bag or spread over all eight, and
    bags ending on the last row of a step."""
    rng = np.random.default_rng(21)
    V, D = 3000, 128
    tiles = []
    for T in (1, 15, 16, 17, 31, 32, 48, 63, 64, 65, 80, 127, 128, 129, 192, 256):
        tiles.append([T] + [0] * 7)                      # one bag holds the walk
        tiles.append([0] * 7 + [T])                      # the last bag holds it, after seven empty ones
        cuts = np.sort(rng.integers(0, T + 1, 7))
        tiles.append(list(np.diff(np.concatenate([[0], cuts, [T]]))))  # spread over all eight
    tiles.append([16] * 8)                               # every bag ends on a step's last row
    tiles.append([64, 0, 64, 0, 1, 63, 0, 0])
    L = np.array([x for t in tiles for x in t], np.int64)
    B = L.size  # one field, tiles in order
    ids = make_ids(rng, int(L.sum()), V)
    offsets = np.concatenate([[0], np.cumsum(L)]).astype(np.int64)
    table = make_table(rng, V, D, "bf16")
    for pooling in ("sum", "mean"):
        want = orc.pool_c(ids, offsets, [table], "bf16", pooling, "f32")
        assert np.array_equal(pooled(pkg, dev, ids, offsets, [table], "bf16", pooling, "f32"), want), pooling
        narrow = np.clip(ids, -2 ** 31, 2 ** 31 - 1).astype(np.int32)
        want32 = orc.pool_c(narrow, offsets, [table], "bf16", pooling, "f32")
        got32 = pooled(pkg, dev, narrow, offsets, [table], "bf16", pooling, "f32", idx=torch.int32)
        assert np.array_equal(got32, want32), pooling


# int8 tables of 128-byte rows (D = 128): 2 bytes of every row per lane and the row's scale read
# with it; each element accumulates fma(q, scale, acc) in row order, as the oracle's int8 loop.
def _int8_case(seed, F, B, V, long_every=0, long_len=0, max_len=60):
    rng = np.random.default_rng(seed)
    L = rng.integers(0, max_len + 1, size=(F, B))
    L[rng.random((F, B)) < 0.1] = 0
    if long_every:
        L[:, ::long_every] = long_len
    ids = np.concatenate([make_ids(rng, int(L[f].sum()), V) for f in range(F)])
    offsets = np.concatenate([[0], np.cumsum(L.reshape(-1))]).astype(np.int64)
    tables = [(rng.integers(-128, 128, (V, 128)).astype(np.int8),
               (rng.random(V) * 0.02 + 1e-4).astype(np.float32)) for _ in range(F)]
    return ids, offsets, tables


def _int8_pooled(pkg, dev, values, offsets, tables, pooling, odt, idx=torch.int64):
    v = torch.from_numpy(np.ascontiguousarray(values)).to(dev, idx)
    o = torch.from_numpy(np.ascontiguousarray(offsets)).to(dev)
    t = [(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)) for q, s in tables]
    out = pkg.embedding_bag_pooled(v, o, t, pooling=pooling, out_dtype=TORCH_DT[odt])
    torch.cuda.synchronize()
    return to_np(out, odt)


@pytest.mark.parametrize("odt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
def test_int8_every_length_bitwise(pkg, dev, odt, pooling, idx):
    """Lengths 0..60 with every fifth bag 300 rows; fp32 / fp16 outputs take the reference's bf16
    rounding of each result first."""
    print(f"stream int8 out={odt} {pooling} {idx}", flush=True)
    ids, offsets, tables = _int8_case(len(odt) + len(pooling), F=4, B=37, V=900, long_every=5, long_len=300)
    values = ids if idx == torch.int64 else np.clip(ids, -2 ** 31, 2 ** 31 - 1).astype(np.int32)
    want = orc.pool_c(values, offsets, tables, "i8", pooling, odt)
    assert np.array_equal(_int8_pooled(pkg, dev, values, offsets, tables, pooling, odt, idx=idx), want)


def test_int8_malformed_offsets_match_oracle(pkg, dev):
    rng = np.random.default_rng(17)
    ids, offsets, tables = _int8_case(18, F=4, B=45, V=700, max_len=20)
    bad = _malformed(offsets, ids.size, rng)
    for pooling in ("sum", "mean"):
        want = orc.pool_c(ids, bad, tables, "i8", pooling, "bf16")
        assert np.array_equal(_int8_pooled(pkg, dev, ids, bad, tables, pooling, "bf16"), want), pooling


@pytest.mark.parametrize("tdt,D,stride", [("bf16", 128, 136), ("f32", 64, 72)])
def test_padded_table_takes_the_ranked_tiles(pkg, dev, tdt, D, stride):
    """A table whose row stride in bytes is not a power of two cannot be read by buffer loads, so
    its 256-byte rows take the length-ranked tiles: bags of up to 24 rows are still sequential
    sums (bit for bit), longer bags are split and meet the fp32 reassociation bound; the padding
    columns are never read (they hold NaN)."""
    case = random_case(D + stride, F=4, B=45, dims=(D,), V=(700,), max_len=60, tdt=tdt, long_every=3,
                       long_len=200)
    B = 45
    padded = []
    for t in case.tables:
        p = np.zeros((t.shape[0], stride), dtype=t.dtype)
        p[:, :D] = t
        p[:, D:] = np.float32("nan") if tdt == "f32" else 0x7FC0
        padded.append(to_dev(p, tdt, dev)[:, :D])
    v = torch.from_numpy(case.values).to(dev)
    o = torch.from_numpy(case.offsets).to(dev)
    out = pkg.embedding_bag_pooled(v, o, padded, pooling="sum", out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    want = orc.pool_c(case.values, case.offsets, case.tables, tdt, "sum", "f32")
    lens = np.diff(case.offsets).reshape(4, B).T  # [B, F]
    assert (lens > 24).sum() > 10
    for f in range(4):
        cols = slice(f * D, (f + 1) * D)
        short = lens[:, f] <= 24
        assert np.array_equal(got[short, cols], want[short, cols].astype(np.float64))
        w = orc.decode(case.tables[f], tdt).astype(np.float64)
        for b in np.nonzero(~short)[0]:
            s, e = case.offsets[f * B + b], case.offsets[f * B + b + 1]
            rows = w[np.clip(case.values[s:e], 0, w.shape[0] - 1)]
            ref = rows.sum(axis=0)
            bound = np.abs(rows).sum(axis=0) * (e - s) * 2.0 ** -24
            assert np.all(np.abs(got[b, cols] - ref) <= bound * (1 + 2.0 ** -24) + np.abs(ref) * 2.0 ** -24 + 1e-30)
