"""Parity of the HIP path (through the C ABI) with the oracle, on the GPU.

Bar: bags pooled by one lane group (every bag when splitting is disabled) match the oracle's
sequential fp32 sum bit for bit; bags split across wavefronts match the fp64 pooling of the
same rows within the fp32 reassociation bound L * 2^-24 * sum|x| plus the output rounding;
on the configuration-sized workloads (rows ~ N(0, 0.01)) fp32 tables are within max-abs 1e-5
of the oracle and bf16 tables within 1e-2 relative (plus the reassociation bound) of the fp64
pooling. Index, offset and segment handling is checked bit for bit with integer-valued tables.
"""
import glob
import os

import numpy as np
import pytest
import torch

from _cases import random_case
from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

NO_SPLIT = 2 ** 31 - 1
ALL_SPLIT = -1
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def to_dev(arr, tdt, dev):
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if tdt != "f32":
        t = t.view(torch.int16).view(TORCH_DT[tdt])
    return t.to(dev)


def to_np(t, odt):
    t = t.cpu()
    if odt == "f32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def gpu_pool(pkg, dev, values, offsets, tables, tdt, pooling, odt, long_threshold=0, idx=torch.int64,
             use_bins=False, block_threshold=0, split_threshold=0):
    v = torch.from_numpy(np.ascontiguousarray(values)).to(dev, idx)
    o = torch.from_numpy(np.ascontiguousarray(offsets)).to(dev)
    tt = [to_dev(t, tdt, dev) for t in tables]
    out = pkg.embedding_bag_pooled(v, o, tt, pooling=pooling, out_dtype=TORCH_DT[odt], long_threshold=long_threshold,
                                   use_bins=use_bins, block_threshold=block_threshold,
                                   split_threshold=split_threshold)
    torch.cuda.synchronize()
    return to_np(out, odt)


def f64_pool(values, offsets, tables, tdt, pooling, batch):
    """fp64 pooling of the decoded rows and the fp32 reassociation bound of each element."""
    F = len(tables)
    outs, bounds = [], []
    for f in range(F):
        w = orc.decode(tables[f], tdt).astype(np.float64)
        acc = np.zeros((batch, w.shape[1]))
        bnd = np.zeros_like(acc)
        for b in range(batch):
            s, e = offsets[f * batch + b], offsets[f * batch + b + 1]
            if e > s:
                rows = w[np.clip(values[s:e], 0, w.shape[0] - 1)]
                acc[b] = rows.sum(axis=0)
                bnd[b] = np.abs(rows).sum(axis=0) * (e - s) * 2.0 ** -24
                if pooling == "mean":
                    acc[b] /= (e - s)
                    bnd[b] /= (e - s)
        outs.append(acc)
        bounds.append(bnd)
    return np.concatenate(outs, axis=1), np.concatenate(bounds, axis=1)


def assert_within_bound(got_enc, odt, ref64, bound):
    got = orc.decode(got_enc, odt).astype(np.float64)
    rnd = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}[odt]
    tol = bound * (1 + rnd) + np.abs(ref64) * rnd + 1e-30
    if odt == "f16":
        tol = tol + 2.0 ** -25  # fp16 subnormal spacing
    bad = np.abs(got - ref64) > tol
    assert not bad.any(), f"{bad.sum()} elements outside the bound; worst {np.abs(got - ref64)[bad].max():.3e}"


# ---- golden fixtures ---------------------------------------------------------------------------
def _fixtures():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


@pytest.mark.parametrize("path", _fixtures(), ids=lambda p: os.path.basename(p)[:-4])
def test_fixture_bitwise_without_split(pkg, dev, path):
    from golden import fixture_io

    fx = fixture_io.load(path)
    if fx["val_base"] is not None:
        S, B = len(fx["val_base"]), fx["batch"]
        w = to_dev(fx["tables"][0], fx["table_dtype"], dev)
        out = torch.empty(B, S * w.shape[1], dtype=w.dtype, device=dev)
        pkg.fused_all_slots_embedding(torch.from_numpy(fx["values"]).to(dev), torch.from_numpy(fx["val_base"]).to(dev),
                                      torch.from_numpy(fx["offsets"]).to(dev), w, out, B, w.shape[1], w.shape[0] - 1)
        torch.cuda.synchronize()
        got = to_np(out, fx["out_dtype"])
    else:
        got = gpu_pool(pkg, dev, fx["values"], fx["offsets"], fx["tables"], fx["table_dtype"], fx["pooling"],
                       fx["out_dtype"], long_threshold=NO_SPLIT)
    assert np.array_equal(got, fx["expected"])


@pytest.mark.parametrize("path", [p for p in _fixtures() if "reference" not in p], ids=lambda p: os.path.basename(p)[:-4])
def test_fixture_all_split_within_bound(pkg, dev, path):
    from golden import fixture_io

    fx = fixture_io.load(path)
    got = gpu_pool(pkg, dev, fx["values"], fx["offsets"], fx["tables"], fx["table_dtype"], fx["pooling"],
                   fx["out_dtype"], long_threshold=ALL_SPLIT)
    ref64, bound = f64_pool(fx["values"], fx["offsets"], fx["tables"], fx["table_dtype"], fx["pooling"], fx["batch"])
    assert_within_bound(got, fx["out_dtype"], ref64, bound)
    if "int_exact" in path or "rowid" in path or "duplicates" in path:
        assert np.array_equal(got, fx["expected"])  # integer partial sums are exact in any order


# ---- every kernel variant ----------------------------------------------------------------------
VARIANTS = [
    # (dims, tdt, odt)
    ((4,), "f32", "f32"), ((8,), "bf16", "bf16"), ((8,), "f32", "f32"), ((16,), "bf16", "f32"),
    ((32,), "bf16", "bf16"), ((32,), "f32", "bf16"), ((64,), "f32", "f32"), ((64,), "f16", "f16"),
    ((128,), "bf16", "bf16"), ((128,), "f32", "f32"), ((128,), "f16", "f32"), ((256,), "bf16", "bf16"),
    ((512,), "bf16", "bf16"), ((512,), "f32", "f32"), ((1024,), "bf16", "f32"), ((1024,), "f32", "f32"),
    ((2048,), "bf16", "bf16"), ((100,), "bf16", "bf16"), ((7,), "f32", "f32"), ((3, 64), "bf16", "bf16"),
    ((32, 64, 128), "bf16", "bf16"),
]


@pytest.mark.parametrize("dims,tdt,odt", VARIANTS, ids=lambda x: str(x))
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_variant_bitwise_without_split(pkg, dev, dims, tdt, odt, pooling):
    case = random_case(VARIANTS.index((dims, tdt, odt)), F=4, B=37, dims=dims, V=(300, 41), tdt=tdt, max_len=24,
                       long_every=9, long_len=150)
    want = orc.pool_c(case.values, case.offsets, case.tables, tdt, pooling, odt)
    got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, tdt, pooling, odt, long_threshold=NO_SPLIT)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dims,tdt,odt", VARIANTS, ids=lambda x: str(x))
def test_variant_split_within_bound(pkg, dev, dims, tdt, odt):
    case = random_case(500 + VARIANTS.index((dims, tdt, odt)), F=3, B=29, dims=dims, V=(500,), tdt=tdt, max_len=40,
                       long_every=5, long_len=700)
    ref64, bound = f64_pool(case.values, case.offsets, case.tables, tdt, "sum", case.B)
    for thr in (ALL_SPLIT, 0):
        got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, tdt, "sum", odt, long_threshold=thr)
        assert_within_bound(got, odt, ref64, bound)


@pytest.mark.parametrize("dims,tdt,odt", VARIANTS, ids=lambda x: str(x))
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_variant_binned_long_kernel_within_bound(pkg, dev, dims, tdt, odt, pooling):
    # bags longer than 40 are listed by the binning pass: those up to split_threshold are pooled by
    # one wavefront each, longer ones split across 8 (or 4) wavefronts
    case = random_case(900 + VARIANTS.index((dims, tdt, odt)), F=3, B=41, dims=dims, V=(500,), tdt=tdt,
                       max_len=60, long_every=4, long_len=900)
    ref64, bound = f64_pool(case.values, case.offsets, case.tables, tdt, pooling, case.B)
    for thr, split in ((0, 0), (8, 0), (0, 50), (0, 100000)):
        got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, tdt, pooling, odt, long_threshold=thr,
                       use_bins=True, block_threshold=40, split_threshold=split)
        assert_within_bound(got, odt, ref64, bound)
    # the short bags never reach a split path: bit for bit with the oracle
    want = orc.pool_c(case.values, case.offsets, case.tables, tdt, pooling, odt)
    got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, tdt, pooling, odt, long_threshold=NO_SPLIT - 1,
                   use_bins=True, block_threshold=40)
    L = case.lengths.reshape(-1)
    short_rows = np.ones(case.B, bool)
    for f in range(case.F):
        short_rows &= case.lengths[f] <= 40
    assert np.array_equal(got[short_rows], want[short_rows])


def test_integer_tables_bitwise_in_every_path(pkg, dev):
    case = random_case(21, F=5, B=64, dims=(32, 128, 512), V=(1000,), tdt="bf16", kind="int", max_len=80,
                       long_every=3, long_len=1500)
    want = orc.pool_c(case.values, case.offsets, case.tables, "bf16", "sum", "f32")
    for thr in (NO_SPLIT, ALL_SPLIT, 0, 40):
        got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, "bf16", "sum", "f32", long_threshold=thr)
        assert np.array_equal(got, want), thr
    for bt, split in ((0, 0), (1, 0), (100, 0), (1, 60), (20, 1000), (20, 2000)):
        got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, "bf16", "sum", "f32", use_bins=True,
                       block_threshold=bt, split_threshold=split)
        assert np.array_equal(got, want), (bt, split)


def test_binning_workspace_is_left_zeroed(pkg, dev):
    case = random_case(77, F=4, B=300, dims=(128,), V=(900,), tdt="bf16", max_len=30, long_every=7, long_len=600)
    tt = [to_dev(t, "bf16", dev) for t in case.tables]
    plan = pkg.PooledEmbedding(tt, pooling="sum", use_bins=True, block_threshold=50, max_batch=case.B,
                               split_threshold=300)
    v = torch.from_numpy(case.values).to(dev)
    o = torch.from_numpy(case.offsets).to(dev)
    first = plan(v, o).clone()
    for _ in range(3):
        again = plan(v, o)
    torch.cuda.synchronize()
    # the two list counters (bytes 0-3 and 8-11) are back at zero; bytes 4-7 and 12-15 hold the
    # list lengths the last call handed to the list kernel
    assert torch.count_nonzero(plan._ws[0:4]).item() == 0 and torch.count_nonzero(plan._ws[8:12]).item() == 0
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    ref64, bound = f64_pool(case.values, case.offsets, case.tables, "bf16", "sum", case.B)
    assert_within_bound(to_np(again, "bf16"), "bf16", ref64, bound)


def test_int32_indices_match_int64(pkg, dev):
    case = random_case(5, F=6, B=50, dims=(128,), V=(4000,), tdt="bf16", clamp_frac=0)
    a = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, "bf16", "mean", "bf16")
    b = gpu_pool(pkg, dev, case.values.astype(np.int32), case.offsets, case.tables, "bf16", "mean", "bf16",
                 idx=torch.int32)
    assert np.array_equal(a, b)


def test_clamp_equivalence(pkg, dev):
    case = random_case(9, F=4, B=40, dims=(64,), V=(77,), tdt="f32", clamp_frac=0.4)
    clamped = case.values.copy()
    for f in range(case.F):
        s, e = case.offsets[f * case.B], case.offsets[(f + 1) * case.B]
        clamped[s:e] = np.clip(clamped[s:e], 0, case.tables[f].shape[0] - 1)
    a = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, "f32", "sum", "f32")
    b = gpu_pool(pkg, dev, clamped, case.offsets, case.tables, "f32", "sum", "f32")
    assert np.array_equal(a, b)


def test_edge_shapes(pkg, dev):
    # one sample; all bags empty (nnz = 0); many fields (several launches of 64 fields)
    for kw in (dict(F=28, B=1), dict(F=3, B=10, max_len=0), dict(F=70, B=5, dims=(128,))):
        case = random_case(3, tdt="bf16", **kw)
        want = orc.pool_c(case.values, case.offsets, case.tables, "bf16", "sum", "bf16")
        got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, "bf16", "sum", "bf16")
        assert np.array_equal(got, want), kw


@pytest.mark.parametrize("path", [dict(), dict(use_bins=True), dict(use_bins=True, split_threshold=100000000),
                                  dict(long_threshold=-1)])
def test_one_bag_of_five_million_rows(pkg, dev, path):
    # the longest bags the layout allows: 5,000,000 rows in one bag beside an empty and a short
    # one, pooled by one wavefront (no binning, or binned below the split length), by the 8
    # wavefronts of a list workgroup (binned and split), or with every bag split. Rows in
    # {-1, 0, 1}: every fp32 partial sum stays below 2^24 and is exact, so all paths equal the
    # int64 sums bit for bit.
    rng = np.random.default_rng(77)
    V, D, lens = 3000, 64, np.array([0, 5_000_000, 7])
    rows = rng.integers(-1, 2, (V, D)).astype(np.float32)
    ids = rng.integers(-5, V + 5, int(lens.sum()))
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    want = np.zeros((3, D), np.int64)
    clamped = np.clip(ids, 0, V - 1)
    for b in range(3):  # row counts times rows: the int64 sum of the bag's rows
        want[b] = np.bincount(clamped[offsets[b]:offsets[b + 1]], minlength=V) @ rows.astype(np.int64)
    got = gpu_pool(pkg, dev, ids, offsets, [orc.encode(rows, "bf16")], "bf16", "sum", "f32", **path)
    assert np.array_equal(got, want.astype(np.float32))


# ---- reference layout (drop-in entry point) and the RepEncoder caller --------------------------
def _reference_batch(seed, S=28, B=64, V=5000, D=128, dt="bf16", max_len=12):
    case = random_case(seed, F=S, B=B, dims=(D,), V=(V,), tdt=dt, max_len=max_len)
    ro, vo = case.reference_layout()
    return case, ro, vo, case.tables[0]


def _special_rows(D):
    """Rows that exercise the fp32 sum and the output rounding at their edges."""
    f32max = np.finfo(np.float32).max
    tiny = np.float32(1e-40)  # fp32 subnormal
    vals = [np.inf, -np.inf, np.nan, f32max, -f32max, 3.3961e38, tiny, -tiny, -0.0, 0.0,
            1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -11, 65504.0, 65520.0, 6e-8, 1e-45, 1.0]
    rows = [np.full(D, v, np.float32) for v in vals]
    rows.append(np.linspace(-3, 3, D).astype(np.float32))
    return np.stack(rows)


@pytest.mark.parametrize("tdt", ["f32", "bf16"])
@pytest.mark.parametrize("odt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_special_values_match_oracle(pkg, dev, tdt, odt, pooling):
    # bags of every pair, triple and single of the special rows (Inf, NaN, overflow, subnormals,
    # rounding ties of bf16 / fp16, signed zeros); finite and infinite results bit for bit, NaN
    # where the oracle has NaN
    D = 128
    table32 = _special_rows(D)
    table = orc.encode(table32, tdt)
    n = len(table32)
    bags = [[i] for i in range(n)] + [[i, j] for i in range(n) for j in range(n)] + \
           [[i, j, k] for i in range(0, n, 3) for j in range(1, n, 4) for k in range(2, n, 5)]
    rng = np.random.default_rng(5)
    rng.shuffle(bags)
    B = len(bags)
    lens = np.array([len(x) for x in bags])
    values = np.concatenate([np.array(x, np.int64) for x in bags])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    got = gpu_pool(pkg, dev, values, offsets, [table], tdt, pooling, odt, long_threshold=NO_SPLIT)
    ref = orc.pool_c(values, offsets, [table], tdt, pooling, odt)
    g, r = orc.decode(got, odt), orc.decode(ref, odt)
    assert np.array_equal(np.isnan(g), np.isnan(r))
    fin = ~np.isnan(r)
    assert np.array_equal(got[fin], ref[fin])


@pytest.mark.parametrize("long_threshold", [NO_SPLIT, 0])
def test_mean_of_subnormal_midpoints(pkg, dev, long_threshold):
    # bags whose fp32 mean is exactly halfway between two subnormals: (L - 1) rows of 2^-149 and
    # one row of (m - L + 1) * 2^-149 sum to m * 2^-149, and m / L = (2k+1) / 2 (ties to even)
    D = 64
    cases = [(98, 147), (150, 2175), (154, 2233), (182, 1183), (186, 1209), (2, 3), (6, 9)]
    rows = [np.full(D, 2.0 ** -149, np.float32)]
    values, lens = [], []
    for L, m in cases:
        rows.append(np.full(D, (m - L + 1) * 2.0 ** -149, np.float32))
        values += [0] * (L - 1) + [len(rows) - 1]
        lens.append(L)
    table = np.stack(rows)
    values = np.array(values, np.int64)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    for odt in ("f32", "bf16", "f16"):
        # sums of integer multiples of 2^-149 are exact in any order, so split bags
        # (long_threshold 0) must match bit for bit as well
        got = gpu_pool(pkg, dev, values, offsets, [table], "f32", "mean", odt, long_threshold=long_threshold)
        ref = orc.pool_c(values, offsets, [table], "f32", "mean", odt)
        assert np.array_equal(got, ref), odt


@pytest.mark.parametrize("dt", ["bf16", "f32", "f16"])
def test_fused_all_slots_matches_oracle(pkg, dev, dt):
    case, ro, vo, w = _reference_batch(31, dt=dt)
    wd = to_dev(w, dt, dev)
    out = torch.empty(case.B, case.F * 128, dtype=TORCH_DT[dt], device=dev)
    ret = pkg.fused_all_slots_embedding(torch.from_numpy(case.values).to(dev), torch.from_numpy(vo).to(dev),
                                        torch.from_numpy(ro).to(dev), wd, out, case.B, 128, w.shape[0] - 1)
    assert ret is out
    torch.cuda.synchronize()
    want = orc.pool_c(case.values, ro, [w] * case.F, dt, "sum", dt, batch=case.B, val_base=vo)
    assert np.array_equal(to_np(out, dt), want)


def test_rep_encoder_drop_in(pkg, dev):
    case, ro, vo, _ = _reference_batch(41, V=3000, D=64, dt="f32")
    enc = pkg.RepEncoder(vocab_size=3000, emb_dim=64, padding_idx=0, slot_num=28, d_model=32).to(dev)
    with torch.no_grad():
        enc.emb.weight.normal_(0, 0.1)
    w = enc.emb.weight.detach().cpu().numpy()
    batch = {"_flat_values": torch.from_numpy(case.values).to(dev), "_flat_row_offsets": torch.from_numpy(ro).to(dev),
             "_val_offsets": torch.from_numpy(vo).to(dev)}
    pooled = enc.pooled(batch)
    want = orc.pool_c(case.values, ro, [w] * 28, "f32", "sum", "f32", batch=case.B, val_base=vo)
    assert np.array_equal(pooled.cpu().numpy(), want)
    # int-keyed per-slot batch: packed on the GPU first (online_best/infer.py:960-974)
    slots = {}
    for s in range(28):
        a, b = int(vo[s]), int(vo[s]) + int(ro[s * (case.B + 1) + case.B])
        slots[s + 1] = (torch.from_numpy(case.values[a:b]).to(dev), torch.from_numpy(ro[s * (case.B + 1):(s + 1) * (case.B + 1)]).to(dev))
    assert torch.equal(enc.pooled(slots), pooled)
    # input LayerNorm on the HIP path (online_best/infer.py:1061-1076), then torch's Linear
    g = enc.input_norm.weight.detach().cpu().numpy()
    bta = enc.input_norm.bias.detach().cpu().numpy()
    norm_ref, _, _ = orc.layer_norm_np(want, g, bta, enc.input_norm.eps)
    np.testing.assert_allclose(enc.normalized(batch).cpu().numpy(), norm_ref, rtol=1e-5, atol=1e-5)
    y = enc(batch)
    ref = enc.linear(enc.input_norm(torch.from_numpy(want).to(dev)))
    assert y.shape == (case.B, 32)
    torch.testing.assert_close(y, ref, rtol=1e-4, atol=1e-4)


# ---- device layout builders --------------------------------------------------------------------
def test_pack_slots_matches_restatement(pkg, dev):
    case, ro, vo, _ = _reference_batch(51, S=28, B=33)
    slots = []
    for s in range(28):
        a = int(vo[s])
        b = a + int(ro[s * (case.B + 1) + case.B])
        slots.append((case.values[a:b], ro[s * (case.B + 1):(s + 1) * (case.B + 1)]))
    fv, fro, fvo = orc.prebuild_layout(slots)
    got = pkg.pack_slots([(torch.from_numpy(v).to(dev), torch.from_numpy(o).to(dev)) for v, o in slots],
                         with_global_offsets=True)
    torch.cuda.synchronize()
    assert np.array_equal(got["_flat_values"].cpu().numpy(), fv)
    assert np.array_equal(got["_flat_row_offsets"].cpu().numpy(), fro)
    assert np.array_equal(got["_val_offsets"].cpu().numpy(), fvo)
    assert np.array_equal(got["offsets"].cpu().numpy(), orc.to_global_offsets(fvo, fro, case.B, len(fv)))
    # non-contiguous slot tensors are packed from a contiguous copy
    strided = [(torch.from_numpy(np.repeat(v, 2)).to(dev)[::2], torch.from_numpy(o).to(dev)) for v, o in slots]
    assert any(not t.is_contiguous() for t, _ in strided)
    again = pkg.pack_slots(strided)
    assert np.array_equal(again["_flat_values"].cpu().numpy(), fv)


def test_pack_slots_rejects_bad_slots(pkg, dev):
    v, o = torch.arange(3, device=dev), torch.tensor([0, 1, 3], device=dev)
    with pytest.raises(ValueError, match="same GPU"):
        pkg.pack_slots([(v, o), (v.cpu(), o)])
    with pytest.raises(ValueError, match="same GPU"):
        pkg.pack_slots([(v.cpu(), o.cpu())])
    with pytest.raises(TypeError, match="int64"):
        pkg.pack_slots([(v, o), (v.int(), o)])
    with pytest.raises(ValueError, match="entries"):
        pkg.pack_slots([(v, o), (v, o[:2])])


def test_merge_batches_matches_restatement_and_pooling_commutes(pkg, dev):
    S = 28
    subs = [random_case(60 + k, F=S, B=B, dims=(128,), V=(2000,), tdt="bf16") for k, B in enumerate((40, 7, 1, 64, 13))]
    lays = []
    dev_batches = []
    for c in subs:
        ro, vo = c.reference_layout()
        lays.append((c.values, ro, vo))
        dev_batches.append({"_flat_values": torch.from_numpy(c.values).to(dev),
                            "_flat_row_offsets": torch.from_numpy(ro).to(dev),
                            "_val_offsets": torch.from_numpy(vo).to(dev)})
    v, ro, vo = orc.merge_layouts(lays, S)
    got = pkg.merge_batches(dev_batches, S, with_global_offsets=True)
    torch.cuda.synchronize()
    assert np.array_equal(got["_flat_values"].cpu().numpy(), v)
    assert np.array_equal(got["_flat_row_offsets"].cpu().numpy(), ro)
    assert np.array_equal(got["_val_offsets"].cpu().numpy(), vo)
    B = sum(c.B for c in subs)
    assert np.array_equal(got["offsets"].cpu().numpy(), orc.to_global_offsets(vo, ro, B, len(v)))
    w = to_dev(subs[0].tables[0], "bf16", dev)
    merged = pkg.fused_embedding(got, w, S)
    parts = [pkg.fused_embedding(b, w, S) for b in dev_batches]
    assert torch.equal(merged, torch.cat(parts, dim=0))


def test_pair_merge_int32_round_trip(pkg, dev):
    """merge_batches(int32_round_trip=True) is the pair merge (online_best/infer.py:2977-3037): the
    merged values pass through int32, so ids of 2^31 or more wrap there (and nowhere else), and the
    pooled result is the pooling of the wrapped ids. Slot offsets of 2^31 or more would wrap the
    same way; they need batches of 2^31 ids, so only the values' wrap is exercised here."""
    S = 28
    subs = [random_case(90 + k, F=S, B=B, dims=(128,), V=(2000,), tdt="bf16") for k, B in enumerate((33, 5, 60))]
    rng = np.random.default_rng(5)
    lays, dev_batches = [], []
    for c in subs:
        m = rng.random(c.values.size) < 0.1
        c.values[m] = rng.integers(2 ** 31, 2 ** 33, int(m.sum())) * rng.choice([-1, 1], int(m.sum()))
        ro, vo = c.reference_layout()
        lays.append((c.values, ro, vo))
        dev_batches.append({"_flat_values": torch.from_numpy(c.values).to(dev),
                            "_flat_row_offsets": torch.from_numpy(ro).to(dev),
                            "_val_offsets": torch.from_numpy(vo).to(dev)})
    v, ro, vo = orc.merge_pair_layouts(lays, S)
    v_lazy, _, _ = orc.merge_layouts(lays, S)
    assert not np.array_equal(v, v_lazy)  # the wrap is visible in this batch
    got = pkg.merge_batches(dev_batches, S, with_global_offsets=True, int32_round_trip=True)
    plain = pkg.merge_batches(dev_batches, S)
    torch.cuda.synchronize()
    assert np.array_equal(got["_flat_values"].cpu().numpy(), v)
    assert np.array_equal(got["_flat_row_offsets"].cpu().numpy(), ro)
    assert np.array_equal(got["_val_offsets"].cpu().numpy(), vo)
    assert np.array_equal(plain["_flat_values"].cpu().numpy(), v_lazy)
    B = sum(c.B for c in subs)
    assert np.array_equal(got["offsets"].cpu().numpy(), orc.to_global_offsets(vo, ro, B, len(v)))
    w = to_dev(subs[0].tables[0], "bf16", dev)
    pooled = pkg.fused_embedding(got, w, S)
    torch.cuda.synchronize()
    want = orc.pool_c(v, ro, [subs[0].tables[0]] * S, "bf16", "sum", batch=B, val_base=vo)
    assert np.array_equal(to_np(pooled, "bf16"), want)


# ---- configuration-sized workloads -------------------------------------------------------------
def _sampled_check(pkg, wl, tables, out, rng, n_sample=400, bag_filter=None):
    """Compare sampled bags (plus every empty, clamped-free longest bag per field) with the oracle
    fed only the rows those bags read."""
    tdt = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[wl.table_dtype]
    odt = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[wl.out_dtype]
    B = wl.batch
    L = wl.lengths().reshape(wl.num_fields, B)
    col = 0
    out_np = to_np(out, odt)
    for f in range(wl.num_fields):
        bags = set(rng.choice(B, size=min(n_sample // wl.num_fields + 1, B), replace=False).tolist())
        bags.add(int(np.argmax(L[f])))
        if (L[f] == 0).any():
            bags.add(int(np.argmax(L[f] == 0)))
        bags = sorted(bags)
        ids = [np.clip(wl.values[wl.offsets[f * B + b]:wl.offsets[f * B + b + 1]], 0, wl.vocab[f] - 1) for b in bags]
        allids = np.concatenate(ids) if ids else np.zeros(0, np.int64)
        uniq, inv = np.unique(allids, return_inverse=True)
        rows = tables[f].index_select(0, torch.from_numpy(uniq).to(tables[f].device)).cpu()
        rows = rows.numpy() if tdt == "f32" else rows.view(torch.int16).numpy().view(np.uint16)
        lens = np.array([len(x) for x in ids], np.int64)
        offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        want = orc.pool_c(inv.astype(np.int64), offs, [rows], tdt, wl.pooling, odt)
        got = out_np[bags, col:col + wl.dims[f]]
        ref64, bound = f64_pool(inv.astype(np.int64), offs, [rows], tdt, wl.pooling, len(bags))
        if tdt == "f32":
            assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() <= 1e-5
        else:
            g = orc.decode(got, odt).astype(np.float64)
            assert np.all(np.abs(g - ref64) <= 1e-2 * np.abs(ref64) + bound + 1e-30)
        short = lens <= 16
        assert np.array_equal(got[short], want[short]), f"field {f}: short bags differ from the oracle"
        col += wl.dims[f]


@pytest.mark.parametrize("name", ["small-fp32", "fp32-1m", "bf16-2m", "hetero-bf16"])
def test_workload_parity_and_properties(pkg, dev, name):
    W = pkg.workloads
    wl = W.make(name, seed=0)
    print(f"[{name}] B={wl.batch} nnz={wl.nnz}", flush=True)
    tables = W.make_tables(wl, dev, seed=0)
    v, o = W.to_device(wl, dev)
    out = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=wl.out_dtype)
    torch.cuda.synchronize()
    if name == "small-fp32":
        tn = [t.cpu().numpy() for t in tables]
        assert np.array_equal(out.cpu().numpy(), orc.pool_c(wl.values, wl.offsets, tn, "f32", "sum", "f32"))
    else:
        _sampled_check(pkg, wl, tables, out, np.random.default_rng(0))
    # determinism: a second call is bitwise identical
    out2 = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=wl.out_dtype)
    assert torch.equal(out.view(torch.int16) if out.dtype != torch.float32 else out,
                       out2.view(torch.int16) if out2.dtype != torch.float32 else out2)
    # scaling every table by 2 (exact) scales every pooled value by 2 (exact)
    for t in tables:
        t.mul_(2)
    out3 = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=wl.out_dtype)
    for t in tables:
        t.div_(2)
    assert torch.equal(out3, out * 2)
    del tables
    torch.cuda.empty_cache()


def test_lazy_grouped_workload(pkg, dev):
    W = pkg.workloads
    wl = W.make("lazy-32k", seed=0)
    print(f"[lazy-32k] B={wl.batch} nnz={wl.nnz}", flush=True)
    tables = W.make_tables(wl, dev, seed=0)
    # sub-batches merged on the device == the workload's merged layout
    batches = []
    for sb in wl.sub_batches:
        ro = np.concatenate([np.concatenate([[0], np.cumsum(sb.lengths()[f * sb.batch:(f + 1) * sb.batch])])
                             for f in range(28)]).astype(np.int64)
        vo = sb.offsets[::sb.batch][:28].astype(np.int64)
        batches.append({"_flat_values": torch.from_numpy(sb.values).to(dev),
                        "_flat_row_offsets": torch.from_numpy(ro).to(dev), "_val_offsets": torch.from_numpy(vo).to(dev)})
    merged = pkg.merge_batches(batches, 28, with_global_offsets=True)
    torch.cuda.synchronize()
    assert np.array_equal(merged["_flat_values"].cpu().numpy(), wl.values)
    assert np.array_equal(merged["offsets"].cpu().numpy(), wl.offsets)
    out = pkg.embedding_bag_pooled(merged["_flat_values"], merged["offsets"], tables, pooling="mean",
                                   out_dtype=torch.bfloat16)
    parts = []
    for sb in wl.sub_batches:
        v, o = W.to_device(sb, dev)
        parts.append(pkg.embedding_bag_pooled(v, o, tables, pooling="mean", out_dtype=torch.bfloat16))
    assert torch.equal(out.view(torch.int16), torch.cat(parts, dim=0).view(torch.int16))
    _sampled_check(pkg, wl, tables, out, np.random.default_rng(1))
    del tables
    torch.cuda.empty_cache()


# The binned path hetero-bf16 is measured with: binning pass, mixed-width main kernel, list kernel
# with bags of 33..192 rows on one wavefront each and longer bags split over a workgroup.
HETERO_BINS = dict(use_bins=True, block_threshold=32, split_threshold=192)


def test_hetero_binned_full_size(pkg, dev):
    """hetero-bf16 at full size (B = 8192) through the binned launch sequence its timings come
    from: sampled bags (more of them, so the split list is hit) against the oracle, short bags bit
    for bit, and the same output as the unbinned launch within the reassociation bound."""
    W = pkg.workloads
    wl = W.make("hetero-bf16", seed=0)
    L = wl.lengths().reshape(wl.num_fields, wl.batch)
    print(f"[hetero-bf16 binned] B={wl.batch} nnz={wl.nnz} bags>192: {(L > 192).sum()} bags 33..192: "
          f"{((L > 32) & (L <= 192)).sum()}", flush=True)
    assert (L > 192).sum() > 1000 and ((L > 32) & (L <= 192)).sum() > 1000
    tables = W.make_tables(wl, dev, seed=0)
    v, o = W.to_device(wl, dev)
    out = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=wl.out_dtype, **HETERO_BINS)
    torch.cuda.synchronize()
    _sampled_check(pkg, wl, tables, out, np.random.default_rng(7), n_sample=4000)
    out2 = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=wl.out_dtype, **HETERO_BINS)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))  # deterministic
    del tables
    torch.cuda.empty_cache()


def test_hetero_binned_full_size_integer_tables_bitwise(pkg, dev):
    """The same binned launch on integer-valued bf16 tables in [-32, 32]: every partial sum is
    exact in fp32 (|sum| <= 2048 * 32 < 2^24), so each output is the bf16 rounding of the exact
    sum whatever the order, and the whole [8192, 2048] output must equal the oracle bit for bit
    (index, offset, segment and list handling of every bag)."""
    W = pkg.workloads
    wl = W.make("hetero-bf16", seed=0)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    tables = [torch.randint(-32, 33, (wl.vocab[f], wl.dims[f]), generator=g, device=dev).to(torch.bfloat16)
              for f in range(wl.num_fields)]
    v, o = W.to_device(wl, dev)
    out = pkg.embedding_bag_pooled(v, o, tables, pooling=wl.pooling, out_dtype=torch.bfloat16, **HETERO_BINS)
    torch.cuda.synchronize()
    got = to_np(out, "bf16")
    B = wl.batch
    col = 0
    for f in range(wl.num_fields):
        s, e = int(wl.offsets[f * B]), int(wl.offsets[(f + 1) * B])
        ids = np.clip(wl.values[s:e], 0, wl.vocab[f] - 1)
        uniq, inv = np.unique(ids, return_inverse=True)
        rows = tables[f].index_select(0, torch.from_numpy(uniq).to(dev)).cpu().view(torch.int16).numpy().view(np.uint16)
        offs = (wl.offsets[f * B:(f + 1) * B + 1] - s).astype(np.int64)
        want = orc.pool_c(inv.astype(np.int64), offs, [rows], "bf16", "sum", "bf16")
        assert np.array_equal(got[:, col:col + wl.dims[f]], want), f"field {f} (D={wl.dims[f]})"
        col += wl.dims[f]
    del tables
    torch.cuda.empty_cache()


@pytest.mark.parametrize("tdt,D", [("bf16", 512), ("f32", 256)])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_one_lane_group_rows_are_sequential(pkg, dev, tdt, D, pooling):
    """1 KiB rows fill a wavefront with one lane group, so a bag above the short-bag limit is
    still walked in element order by that group: every bag, up to 300 rows, equals the oracle's
    sequential sum bit for bit (the reference's own [5M, 512] table has these rows)."""
    case = random_case(D + len(pooling), F=3, B=21, dims=(D,), V=(800,), max_len=40, tdt=tdt,
                       long_every=4, long_len=300)
    want = orc.pool_c(case.values, case.offsets, case.tables, tdt, pooling, tdt)
    got = gpu_pool(pkg, dev, case.values, case.offsets, case.tables, tdt, pooling, tdt)
    assert np.array_equal(got, want)
