"""The timed configurations checked over their whole output, through exactly the calls the
benchmark times.

The oracle (`pool_c`, the sequential fp32 restatement of online_best/infer.py:805-827 and
baseline/infer.py:256-263) pools, field by field, a compact copy of the rows the batch touches
(gathered from the device tables), with the ids renumbered to it; so every bag of the batch is
checked, not a sample.

- bf16-2m and lazy-32k take the streamed tiles (256-byte rows): every bag is one sequential fp32
  sum, so the whole output must equal the oracle bit for bit, with and without the dispatch order
  that the benchmark ships with each batch (the ordered launch must also equal the plain one).
- fp32-1m (512-byte rows, two lane groups per wavefront): bags of up to 24 rows are pooled by one
  lane group in element order (bit for bit); longer ones by the whole wavefront, within max-abs
  1e-5 of the oracle (the stated fp32 tolerance) and within the fp32 reassociation bound.
- The reference's own shape (one shared bf16 [5,000,000, 512] table, 28 slots, B = 4096): 1 KiB
  rows fill a wavefront with one lane group, so every bag is sequential: bit for bit, through the
  drop-in launch, with and without the host-made order.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

DT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _bits(t, odt):
    t = t.cpu()
    return t.numpy() if odt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def _field_oracle(wl, table, f, odt):
    """Oracle pooling of field f over every bag: (output [B, D] encoded, lengths, fp64 pooling,
    reassociation bound)."""
    B = wl.batch
    tdt = DT[wl.table_dtype]
    s, e = int(wl.offsets[f * B]), int(wl.offsets[(f + 1) * B])
    ids = np.clip(wl.values[s:e], 0, wl.vocab[f] - 1)
    uniq, inv = np.unique(ids, return_inverse=True)
    rows = table.index_select(0, torch.from_numpy(uniq).to(table.device)).cpu()
    rows = rows.numpy() if tdt == "f32" else rows.view(torch.int16).numpy().view(np.uint16)
    offs = (wl.offsets[f * B:(f + 1) * B + 1] - s).astype(np.int64)
    want = orc.pool_c(inv.astype(np.int64), offs, [rows], tdt, wl.pooling, odt)
    return want, np.diff(offs), rows, inv, offs


def _f64_bound(rows, tdt, inv, offs, pooling):
    """fp64 pooling of the decoded rows and the fp32 reassociation bound L * 2^-24 * sum|x|,
    from per-bag sums of the gathered rows (np.add.reduceat over non-empty bags)."""
    w = orc.decode(rows, tdt).astype(np.float64)
    x = w[inv]
    lens = np.diff(offs)
    ref = np.zeros((lens.size, w.shape[1]))
    absum = np.zeros_like(ref)
    nz = lens > 0
    if nz.any():
        starts = offs[:-1][nz]
        ref[nz] = np.add.reduceat(x, starts, axis=0)
        absum[nz] = np.add.reduceat(np.abs(x), starts, axis=0)
    bound = absum * lens[:, None] * 2.0 ** -24
    if pooling == "mean":
        ref[nz] /= lens[nz, None]
        bound[nz] /= lens[nz, None]
    return ref, bound


def _tile_orders(pkg, wl, dev):
    return pkg.make_tile_order(torch.from_numpy(wl.offsets), wl.batch, wl.num_fields, wl.table_dtype,
                               wl.dims[0]).to(dev)


def _bench_calls(pkg, wl, tables, dev, ordered):
    """The output of the benchmark's step for this batch: plain, and with the host-made order."""
    W = pkg.workloads
    v, o = W.to_device(wl, dev)
    plan = pkg.PooledEmbedding(tables, pooling=wl.pooling, out_dtype=wl.out_dtype, max_batch=wl.batch)
    out = torch.empty((wl.batch, sum(wl.dims)), dtype=wl.out_dtype, device=dev)
    plan(v, o, out)
    outs = {"plain": out}
    if ordered:
        out_o = torch.empty_like(out)
        plan(v, o, out_o, tile_order=_tile_orders(pkg, wl, dev))
        outs["host order"] = out_o
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("name,seed,ordered", [("bf16-2m", 1, True), ("bf16-2m", 5, True), ("lazy-32k", 1, False)])
def test_streamed_workload_whole_output_bitwise(pkg, dev, name, seed, ordered):
    W = pkg.workloads
    wl = W.make(name, seed=seed)
    print(f"[{name} seed {seed}] B={wl.batch} nnz={wl.nnz} longest bag {wl.lengths().max()}", flush=True)
    tables = W.make_tables(wl, dev, seed=0)
    outs = _bench_calls(pkg, wl, tables, dev, ordered)
    odt = DT[wl.out_dtype]
    got = {k: _bits(v, odt) for k, v in outs.items()}
    D = wl.dims[0]
    for f in range(wl.num_fields):
        want, lens, _, _, _ = _field_oracle(wl, tables[f], f, odt)
        for k, g in got.items():
            assert np.array_equal(g[:, f * D:(f + 1) * D], want), f"{name} field {f} ({k}) differs from the oracle"
    if ordered:
        assert np.array_equal(got["plain"], got["host order"])
    del tables, outs
    torch.cuda.empty_cache()


def test_fp32_1m_whole_output(pkg, dev):
    W = pkg.workloads
    wl = W.make("fp32-1m", seed=1)
    print(f"[fp32-1m] B={wl.batch} nnz={wl.nnz} longest bag {wl.lengths().max()}", flush=True)
    tables = W.make_tables(wl, dev, seed=0)
    outs = _bench_calls(pkg, wl, tables, dev, ordered=True)
    got = {k: v.cpu().numpy() for k, v in outs.items()}
    assert np.array_equal(got["plain"], got["host order"])
    D = wl.dims[0]
    n_split = 0
    for f in range(wl.num_fields):
        want, lens, rows, inv, offs = _field_oracle(wl, tables[f], f, "f32")
        g = got["plain"][:, f * D:(f + 1) * D]
        short = lens <= 24
        assert np.array_equal(g[short], want[short]), f"field {f}: bags of <= 24 rows differ from the oracle"
        assert np.abs(g.astype(np.float64) - want.astype(np.float64)).max() <= 1e-5, f"field {f}"
        ref, bound = _f64_bound(rows, "f32", inv, offs, "sum")
        assert np.all(np.abs(g.astype(np.float64) - ref) <= bound * (1 + 2.0 ** -24) + np.abs(ref) * 2.0 ** -24
                      + 1e-30), f"field {f}: outside the reassociation bound"
        n_split += int((~short).sum())
    assert n_split > 1000  # the whole-wavefront path is exercised
    del tables, outs
    torch.cuda.empty_cache()


def test_reference_shape_whole_output_bitwise(pkg, dev):
    """B = 4096 over the shared [5M, 512] bf16 table (5.12 GB: rows past 4 GiB take 64-bit
    addresses), the reference layout and the drop-in launch (online_best/infer.py:1050-1059)."""
    W = pkg.workloads
    wl = W.make("reference-5m", seed=1)
    F, B, D, V = wl.num_fields, wl.batch, wl.dims[0], wl.vocab[0]
    print(f"[reference-5m] B={B} nnz={wl.nnz} longest bag {wl.lengths().max()}", flush=True)
    weight = W.make_tables(wl, dev, seed=0)[0]
    vo = wl.offsets[::B][:F].astype(np.int64)
    ro = np.concatenate([wl.offsets[f * B:(f + 1) * B + 1] - wl.offsets[f * B] for f in range(F)]).astype(np.int64)
    v_d, vo_d, ro_d = (torch.from_numpy(x).to(dev) for x in (wl.values, vo, ro))
    out = torch.empty((B, F * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding(v_d, vo_d, ro_d, weight, out, B, D, V - 1)
    out_o = torch.empty_like(out)
    order = pkg.make_tile_order(torch.from_numpy(ro), B, F, weight.dtype, D).to(dev)
    pkg.fused_all_slots_embedding(v_d, vo_d, ro_d, weight, out_o, B, D, V - 1, tile_order=order)
    torch.cuda.synchronize()
    got, got_o = _bits(out, "bf16"), _bits(out_o, "bf16")
    assert np.array_equal(got, got_o)
    # the oracle over the touched rows of the one shared table, all slots at once
    rows = np.clip(wl.values, 0, V - 1)
    uniq, inv = np.unique(rows, return_inverse=True)
    sub = weight.index_select(0, torch.from_numpy(uniq).to(dev)).cpu().view(torch.int16).numpy().view(np.uint16)
    want = orc.pool_c(inv.astype(np.int64), ro, [sub] * F, "bf16", "sum", batch=B, val_base=vo)
    assert np.array_equal(got, want)
    del weight
    torch.cuda.empty_cache()
