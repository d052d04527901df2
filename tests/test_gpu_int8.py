"""int8 row-quantised tables on the GPU (online_best/infer.py:893-942), through the C ABI.

Bar: the quantiser is bit-identical to torch's own device evaluation of the reference expression
and to the oracle; bags pooled by one lane group match the oracle's sequential fused
multiply-add bit for bit (fp32 / bf16 / fp16 output); bags split across lane groups or
wavefronts stay within the fp32 reassociation bound of the fp64 pooling of q * scale.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

NO_SPLIT = 2 ** 31 - 1
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def to_np(t, odt):
    t = t.cpu()
    if odt == "f32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def reference_quantize(weight):
    """online_best/infer.py:896-901, evaluated by torch on the tensor's device."""
    row_max = weight.abs().max(dim=1).values.float()
    scale = row_max / 127.0
    scale = torch.clamp(scale, min=1e-8)
    weight_int8 = (weight.float() / scale.unsqueeze(1)).round().clamp(-128, 127).to(torch.int8)
    return weight_int8, scale.float()


def int8_tables(rng, F, V, D):
    out = []
    for f in range(F):
        q = rng.integers(-128, 128, (V[f % len(V)], D[f % len(D)])).astype(np.int8)
        sc = (rng.random(q.shape[0]) * 0.02 + 1e-4).astype(np.float32)
        out.append((q, sc))
    return out


def lengths_offsets(rng, F, B, max_len, empty_frac=0.1):
    L = rng.integers(0, max_len + 1, (F, B))
    L[rng.random((F, B)) < empty_frac] = 0
    offsets = np.zeros(F * B + 1, np.int64)
    np.cumsum(L.reshape(-1), out=offsets[1:])
    return L, offsets


def ids_for(rng, L, V):
    F = L.shape[0]
    parts = []
    for f in range(F):
        n = int(L[f].sum())
        v = rng.integers(0, V[f % len(V)], n).astype(np.int64)
        m = rng.random(n) < 0.05
        v[m] = rng.choice(np.array([-1, -(2 ** 40), 10 ** 9, np.iinfo(np.int64).max], np.int64), int(m.sum()))
        parts.append(v)
    return np.concatenate(parts) if parts else np.zeros(0, np.int64)


def dev_tables(tables, dev):
    return [(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)) for q, s in tables]


def f64_int8_pool(values, offsets, tables, pooling, batch):
    outs, bounds = [], []
    for f, (q, s) in enumerate(tables):
        w = q.astype(np.float64) * s.astype(np.float64)[:, None]
        acc = np.zeros((batch, w.shape[1]))
        bnd = np.zeros_like(acc)
        for b in range(batch):
            st, en = offsets[f * batch + b], offsets[f * batch + b + 1]
            if en > st:
                rows = w[np.clip(values[st:en], 0, w.shape[0] - 1)]
                acc[b] = rows.sum(axis=0)
                bnd[b] = np.abs(rows).sum(axis=0) * (en - st) * 2.0 ** -23
                if pooling == "mean":
                    acc[b] /= en - st
                    bnd[b] /= en - st
        outs.append(acc)
        bounds.append(bnd)
    return np.concatenate(outs, axis=1), np.concatenate(bounds, axis=1)


# ------------------------------------------------------------------------------------------------
# quantiser
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,dim", [(1, 16), (7, 40), (1000, 128), (4099, 200), (3, 1000)])
def test_quantizer_matches_torch_on_device(pkg, dev, dt, rows, dim):
    print(f"quantize dt={dt} rows={rows} dim={dim}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows * 31 + dim)
    w = (torch.randn(rows, dim, generator=g) * torch.exp2(torch.randint(-10, 4, (rows, 1), generator=g).float()))
    w[rows // 2] = 0.0
    w = w.to(TORCH_DT[dt]).to(dev)
    q, s = pkg.quantize_embedding_int8(w)
    qr, sr = reference_quantize(w)
    torch.cuda.synchronize()
    assert torch.equal(s.view(torch.int32), sr.view(torch.int32))
    assert torch.equal(q, qr)
    qo, so = orc.quantize_int8_np(w.float().cpu().numpy())
    assert np.array_equal(so.view(np.uint32), s.cpu().numpy().view(np.uint32))
    assert np.array_equal(qo, q.cpu().numpy())


def test_quantizer_strided_rows(pkg, dev):
    g = torch.Generator(device="cpu").manual_seed(4)
    base = torch.randn(300, 160, generator=g).to(torch.bfloat16).to(dev)
    w = base[:, :128]  # row stride 160
    q, s = pkg.quantize_embedding_int8(w)
    qr, sr = reference_quantize(w.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(q, qr) and torch.equal(s, sr)


# ------------------------------------------------------------------------------------------------
# pooling
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("odt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256, 512, 1024, 2048, 4096])
def test_int8_pool_bitwise_short_bags(pkg, dev, D, odt):
    print(f"int8 pool D={D} odt={odt}", flush=True)
    rng = np.random.default_rng(D + len(odt))
    F, B = 5, 67 if D <= 512 else 9
    tables = int8_tables(rng, F, [300, 41], [D])
    L, offsets = lengths_offsets(rng, F, B, 24)
    values = ids_for(rng, L, [300, 41])
    v = torch.from_numpy(values).to(dev)
    o = torch.from_numpy(offsets).to(dev)
    for pooling in ("sum", "mean"):
        out = pkg.embedding_bag_pooled(v, o, dev_tables(tables, dev), pooling=pooling, out_dtype=TORCH_DT[odt],
                                       long_threshold=NO_SPLIT)
        torch.cuda.synchronize()
        want = orc.pool_c(values, offsets, tables, "i8", pooling, odt)
        got = to_np(out, odt)
        assert np.array_equal(got.view(np.uint32 if odt == "f32" else np.uint16),
                              want.view(np.uint32 if odt == "f32" else np.uint16)), pooling


@pytest.mark.parametrize("D", [16, 128, 512])
@pytest.mark.parametrize("mode", ["split", "bins"])
def test_int8_pool_split_bags_within_bound(pkg, dev, D, mode):
    print(f"int8 split D={D} mode={mode}", flush=True)
    rng = np.random.default_rng(D * 3 + len(mode))
    F, B = 3, 40
    tables = int8_tables(rng, F, [500], [D])
    L, offsets = lengths_offsets(rng, F, B, 40)
    L[:, ::7] = 700
    offsets = np.zeros(F * B + 1, np.int64)
    np.cumsum(L.reshape(-1), out=offsets[1:])
    values = ids_for(rng, L, [500])
    v = torch.from_numpy(values).to(dev)
    o = torch.from_numpy(offsets).to(dev)
    kw = dict(long_threshold=-1) if mode == "split" else dict(use_bins=True, block_threshold=256)
    for pooling in ("sum", "mean"):
        out = pkg.embedding_bag_pooled(v, o, dev_tables(tables, dev), pooling=pooling, out_dtype=torch.float32, **kw)
        torch.cuda.synchronize()
        ref, bnd = f64_int8_pool(values, offsets, tables, pooling, B)
        err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
        assert (err <= bnd + np.abs(ref) * 2.0 ** -24 + 1e-30).all(), (pooling, err.max())


def test_int8_fused_all_slots_reference_layout(pkg, dev):
    """The drop-in for the reference's int8 launch: 28 slots, D = 128, bf16 output, flat layout."""
    rng = np.random.default_rng(28)
    S, B, V, D = 28, 129, 5000, 128
    q = rng.integers(-128, 128, (V, D)).astype(np.int8)
    sc = (rng.random(V) * 0.01 + 1e-5).astype(np.float32)
    L = rng.integers(0, 12, (S, B))
    L[:, 3] = 0
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    values = rng.integers(-3, V + 3, int(L.sum())).astype(np.int64)
    want = orc.pool_c(values, ro.reshape(-1), [(q, sc)] * S, "i8", "sum", "bf16", batch=B, val_base=vo)
    out = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding_int8(torch.from_numpy(values).to(dev), torch.from_numpy(vo).to(dev),
                                       torch.from_numpy(ro.reshape(-1)).to(dev), torch.from_numpy(q).to(dev),
                                       torch.from_numpy(sc).to(dev), out, B, D, V - 1)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(out, "bf16"), want)


@pytest.mark.parametrize("odt", ["f32", "f16"])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
def test_int8_reference_layout_rounds_through_bf16(pkg, dev, odt, idx):
    """The reference's int8 kernel stores acc.to(tl.bfloat16) into an output of the table's dtype
    (online_best/infer.py:941, :989-996): with an fp32 / fp16 output the drop-in must hold the
    bf16-rounded sum, widened (fp32) or converted again (fp16)."""
    rng = np.random.default_rng(41)
    S, B, V, D = 28, 65, 3000, 128
    q = rng.integers(-128, 128, (V, D)).astype(np.int8)
    sc = (rng.random(V) * 0.01 + 1e-5).astype(np.float32)
    L = rng.integers(0, 12, (S, B))
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    values = rng.integers(-3, V + 3, int(L.sum())).astype(np.int64)
    bf = orc.decode(orc.pool_c(values, ro.reshape(-1), [(q, sc)] * S, "i8", "sum", "bf16", batch=B, val_base=vo),
                    "bf16")
    single = orc.pool_c(values, ro.reshape(-1), [(q, sc)] * S, "i8", "sum", "f32", batch=B, val_base=vo)
    want = bf.astype(np.float32) if odt == "f32" else bf.astype(np.float16)
    assert not np.array_equal(single, bf)  # the bf16 rounding is visible
    out = torch.empty((B, S * D), dtype=TORCH_DT[odt], device=dev)
    pkg.fused_all_slots_embedding_int8(torch.from_numpy(values).to(dev, idx), torch.from_numpy(vo).to(dev),
                                       torch.from_numpy(ro.reshape(-1)).to(dev), torch.from_numpy(q).to(dev),
                                       torch.from_numpy(sc).to(dev), out, B, D, V - 1)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32 if odt == "f32" else np.uint16),
                          want.view(np.uint32 if odt == "f32" else np.uint16))


def _unfused_int8_pool(values, offsets, tables, batch):
    """Sum pooling of int8 rows with the multiply rounded before the add, acc = RN(acc + RN(q * s)),
    in element order: the form the reference's `acc += int8_row * scale_val` (online_best/infer.py:
    934-936) takes if its compiler does not fuse the multiply into the add."""
    outs = []
    for f, (q, s) in enumerate(tables):
        acc = np.zeros((batch, q.shape[1]), np.float32)
        for b in range(batch):
            st, en = offsets[f * batch + b], offsets[f * batch + b + 1]
            for i in range(st, en):
                r = min(max(int(values[i]), 0), q.shape[0] - 1)
                acc[b] = (acc[b] + (q[r].astype(np.float32) * s[r]).astype(np.float32)).astype(np.float32)
        outs.append(acc)
    return np.concatenate(outs, axis=1)


def test_int8_within_bound_of_the_unfused_accumulation(pkg, dev):
    """The int8 pooling equals the fused multiply-add oracle bit for bit (other tests); whether the
    reference's Triton build fuses `acc += q * s` cannot be observed here, so the output is also
    checked against the unfused accumulation: within the two forms' rounding difference, at most
    one fp32 rounding of the running sum per row, L * 2^-24 * sum|q * s|, plus the output's."""
    rng = np.random.default_rng(31)
    F, B = 3, 40
    tables = int8_tables(rng, F, [500], [128])
    L, offsets = lengths_offsets(rng, F, B, 40)
    values = ids_for(rng, L, [500])
    out = pkg.embedding_bag_pooled(torch.from_numpy(values).to(dev), torch.from_numpy(offsets).to(dev),
                                   dev_tables(tables, dev), pooling="sum", out_dtype=torch.float32,
                                   long_threshold=NO_SPLIT)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    unfused = _unfused_int8_pool(values, offsets, tables, B).astype(np.float64)
    ref64, bound = f64_int8_pool(values, offsets, tables, "sum", B)
    assert (np.abs(got - unfused) <= 2 * bound + np.abs(ref64) * 2.0 ** -23 + 1e-30).all()
    assert not np.array_equal(got, unfused)  # the data does tell the two forms apart


def test_int8_matches_dequantised_float_tables_within_rounding(pkg, dev):
    """Quantise a bf16 table on the device, pool both; the int8 result tracks the bf16 one within
    the quantisation error (half a step per element, summed over the bag)."""
    rng = np.random.default_rng(8)
    V, D, F, B = 2000, 128, 4, 64
    w = torch.from_numpy((rng.standard_normal((V, D)) * 0.01).astype(np.float32)).to(torch.bfloat16).to(dev)
    q, s = pkg.quantize_embedding_int8(w)
    L, offsets = lengths_offsets(rng, F, B, 10)
    values = torch.from_numpy(ids_for(rng, L, [V])).to(dev)
    o = torch.from_numpy(offsets).to(dev)
    a = pkg.embedding_bag_pooled(values, o, [w] * F, out_dtype=torch.float32, long_threshold=NO_SPLIT)
    b = pkg.embedding_bag_pooled(values, o, [(q, s)] * F, out_dtype=torch.float32, long_threshold=NO_SPLIT)
    torch.cuda.synchronize()
    step = s.max().item()
    Lmax = int(L.max())
    assert (a - b).abs().max().item() <= 0.5 * step * Lmax * 1.01 + 1e-6


def test_int8_plan_and_encoder(pkg, dev):
    rng = np.random.default_rng(12)
    tables = int8_tables(rng, 3, [100], [64])
    L, offsets = lengths_offsets(rng, 3, 20, 8)
    values = ids_for(rng, L, [100])
    plan = pkg.PooledEmbedding(dev_tables(tables, dev), pooling="mean")
    out = plan(torch.from_numpy(values).to(dev), torch.from_numpy(offsets).to(dev))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    assert np.array_equal(to_np(out, "bf16"), orc.pool_c(values, offsets, tables, "i8", "mean", "bf16"))


@pytest.mark.parametrize("D", [1, 3, 8, 24, 100, 136, 4096])
def test_int8_any_width(pkg, dev, D):
    """Widths that are not whole lane vectors (or too wide for the vector kernels) take the
    element-wise kernel; results are still the oracle's bit for bit (one wavefront per bag)."""
    print(f"int8 width D={D}", flush=True)
    rng = np.random.default_rng(D)
    tables = int8_tables(rng, 3, [77], [D])
    L, offsets = lengths_offsets(rng, 3, 21, 30)
    values = ids_for(rng, L, [77])
    v = torch.from_numpy(values).to(dev)
    o = torch.from_numpy(offsets).to(dev)
    for pooling in ("sum", "mean"):
        out = pkg.embedding_bag_pooled(v, o, dev_tables(tables, dev), pooling=pooling, out_dtype=torch.float32,
                                       long_threshold=NO_SPLIT)
        torch.cuda.synchronize()
        want = orc.pool_c(values, offsets, tables, "i8", pooling, "f32")
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), pooling


def test_int8_strided_rows_and_unaligned_output(pkg, dev):
    """Row stride wider than the row and an output block that starts off the vector alignment."""
    rng = np.random.default_rng(77)
    q_full = torch.from_numpy(rng.integers(-128, 128, (90, 80)).astype(np.int8)).to(dev)
    s = torch.from_numpy((rng.random(90) * 0.01).astype(np.float32)).to(dev)
    q = q_full[:, :64]
    L, offsets = lengths_offsets(rng, 2, 17, 12)
    values = ids_for(rng, L, [90])
    v = torch.from_numpy(values).to(dev)
    o = torch.from_numpy(offsets).to(dev)
    out = pkg.embedding_bag_pooled(v, o, [(q, s), (q, s)], out_dtype=torch.bfloat16, long_threshold=NO_SPLIT)
    torch.cuda.synchronize()
    qn = q.cpu().numpy()
    sn = s.cpu().numpy()
    want = orc.pool_c(values, offsets, [(qn, sn), (qn, sn)], "i8", "sum", "bf16")
    assert np.array_equal(to_np(out, "bf16"), want)


def test_encoder_int8_switch(pkg, dev):
    torch.manual_seed(0)
    enc = pkg.RepEncoder(3000, 128, 0, 28, 64).to(dev).to(torch.bfloat16)
    rng = np.random.default_rng(3)
    S, B = 28, 33
    L = rng.integers(0, 6, (S, B))
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    values = rng.integers(0, 3000, int(L.sum())).astype(np.int64)
    batch = {"_flat_values": torch.from_numpy(values).to(dev), "_val_offsets": torch.from_numpy(vo).to(dev),
             "_flat_row_offsets": torch.from_numpy(ro.reshape(-1)).to(dev)}
    enc.quantize_int8_()
    pooled = enc.pooled(batch)
    q, s = reference_quantize(enc.emb.weight.detach())
    torch.cuda.synchronize()
    want = orc.pool_c(values, ro.reshape(-1), [(q.cpu().numpy(), s.cpu().numpy())] * S, "i8", "sum", "bf16",
                      batch=B, val_base=vo)
    assert np.array_equal(to_np(pooled, "bf16"), want)
    enc.dequantize_()
    assert enc._int8_weight is None
