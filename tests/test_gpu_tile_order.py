"""Dispatch order of the main pooling kernel (cti_ebag_tile_order, opts->tile_order).

An order only changes which workgroup pools which tile, and when: every output row still has one
writer and every bag is pooled by the same code in the same element order, so pooling with any
order must equal pooling without one bit for bit (the reference semantics, online_best/infer.py:
805-827, are pinned against the oracle by the other GPU tests). The order itself is checked on the
host: for each XCD's range of dispatch positions, a permutation of that range's tiles, most rows
per bag first. Orders made for another batch or another shape, and corrupt orders, must leave the
result unchanged (the kernel checks an order's header and the range of every entry).
"""
import numpy as np
import pytest
import torch

from _cases import random_case
from test_gpu_parity import to_dev

pytestmark = pytest.mark.gpu

MAGIC = 0x4F524452
# (table dtype, width, bags per tile of that row shape: 2 rounds x 64 / lanes per row)
SHAPES = [("bf16", 128, 8), ("f32", 128, 4), ("bf16", 32, 32), ("bf16", 512, 2), ("f16", 64, 16)]


def _plan_case(pkg, dev, seed, tdt, dim, F=6, B=300, pooling="sum", **kw):
    case = random_case(seed, F=F, B=B, dims=(dim,), V=(700,), tdt=tdt, max_len=40, long_every=23, long_len=150)
    tables = [to_dev(t, tdt, dev) for t in case.tables]
    plan = pkg.PooledEmbedding(tables, pooling=pooling, max_batch=B, **kw)
    v = torch.from_numpy(case.values).to(dev)
    o = torch.from_numpy(case.offsets).to(dev)
    return case, plan, v, o


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("tdt,dim,nb", SHAPES)
@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("bins", [False, True])
def test_ordered_pooling_is_bitwise_the_same(pkg, dev, tdt, dim, nb, pooling, bins):
    kw = dict(use_bins=True, block_threshold=60, split_threshold=120) if bins else {}
    case, plan, v, o = _plan_case(pkg, dev, 500 + dim + (7 if bins else 0), tdt, dim, pooling=pooling, **kw)
    order = plan.tile_order(v, o)
    got = plan(v, o, tile_order=order)
    want = plan(v, o)
    torch.cuda.synchronize()
    assert _same(got, want)


def test_ordered_int8_pooling_is_bitwise_the_same(pkg, dev):
    case = random_case(541, F=5, B=257, dims=(128,), V=(900,), tdt="bf16", max_len=40)
    tables = [pkg.quantize_embedding_int8(to_dev(t, "bf16", dev)) for t in case.tables]
    plan = pkg.PooledEmbedding(tables, pooling="mean")
    v, o = torch.from_numpy(case.values).to(dev), torch.from_numpy(case.offsets).to(dev)
    order = plan.tile_order(v, o)
    got, want = plan(v, o, tile_order=order), plan(v, o)
    torch.cuda.synchronize()
    assert _same(got, want)


@pytest.mark.parametrize("tdt,dim,nb", SHAPES)
def test_order_sorts_each_xcd_range_by_rows_per_bag(pkg, dev, tdt, dim, nb):
    F, B = 5, 777
    case, plan, v, o = _plan_case(pkg, dev, 600 + dim, tdt, dim, F=F, B=B)
    order = plan.tile_order(v, o).cpu().numpy()
    tpf = -(-B // nb)
    n = F * tpf
    assert order[0] == n and order[1] == MAGIC
    L = np.zeros((F, tpf * nb), np.int64)
    L[:, :B] = case.lengths
    key = np.minimum(L.reshape(F, tpf, nb).sum(axis=2) // nb, 63).reshape(-1)
    q, r = divmod(n, 8)
    lo = 0
    for x in range(8):
        cnt = q + (1 if x < r else 0)
        seg = order[4 + lo:4 + lo + cnt]
        assert sorted(seg.tolist()) == list(range(lo, lo + cnt)), x  # the range keeps its own tiles
        assert (np.diff(key[seg]) <= 0).all(), x                      # most rows per bag first
        lo += cnt


def test_orders_of_other_batches_or_shapes_change_nothing(pkg, dev):
    caseA, plan, vA, oA = _plan_case(pkg, dev, 701, "bf16", 128, B=400)
    caseB = random_case(702, F=6, B=400, dims=(128,), V=(700,), tdt="bf16", max_len=40)
    vB, oB = torch.from_numpy(caseB.values).to(dev), torch.from_numpy(caseB.offsets).to(dev)
    caseC = random_case(703, F=6, B=150, dims=(128,), V=(700,), tdt="bf16", max_len=40)
    vC, oC = torch.from_numpy(caseC.values).to(dev), torch.from_numpy(caseC.offsets).to(dev)
    want = plan(vB, oB).clone()
    stale = plan.tile_order(vA, oA)   # same shape, another batch: a valid order, only less apt
    other = plan.tile_order(vC, oC)   # 150 samples: made for fewer tiles, so it is ignored
    assert _same(plan(vB, oB, tile_order=stale), want)
    assert _same(plan(vB, oB, tile_order=other), want)
    torch.cuda.synchronize()


def test_corrupt_order_entries_fall_back_to_the_tile_order(pkg, dev):
    # a header that matches the launch with entries outside its tiles: every workgroup takes its
    # own position, so the result is the plain one (and nothing is read out of bounds)
    F, B, nb = 6, 300, 8
    case, plan, v, o = _plan_case(pkg, dev, 801, "bf16", 128, F=F, B=B)
    n = F * (-(-B // nb))
    want = plan(v, o).clone()
    for fill in (-1, n, 2 ** 31 - 1, -(2 ** 31)):
        bad = torch.full((plan.order_elements(B),), fill, dtype=torch.int32)
        bad[0], bad[1] = n, MAGIC
        assert _same(plan(v, o, tile_order=bad.to(dev)), want), fill
    torch.cuda.synchronize()


def test_short_order_buffer_is_rejected_on_the_host(pkg, dev):
    case, plan, v, o = _plan_case(pkg, dev, 802, "bf16", 128)
    with pytest.raises(pkg.EbagError, match="tile order"):
        plan(v, o, tile_order=torch.zeros(3, dtype=torch.int32, device=dev))


def test_mixed_width_plans_take_no_order(pkg, dev):
    case = random_case(803, F=6, B=200, dims=(128, 32), V=(500,), tdt="bf16", max_len=30)
    tables = [to_dev(t, "bf16", dev) for t in case.tables]
    plan = pkg.PooledEmbedding(tables, pooling="sum")
    v, o = torch.from_numpy(case.values).to(dev), torch.from_numpy(case.offsets).to(dev)
    with pytest.raises(pkg.EbagError, match="one row shape"):
        plan.tile_order(v, o)
    junk = torch.full((plan.order_elements(case.B),), 7, dtype=torch.int32, device=dev)
    assert _same(plan(v, o, tile_order=junk), plan(v, o))  # ignored by the mixed-width launch
    torch.cuda.synchronize()
