"""Pooling with a dispatch order made one batch ahead (PooledEmbedding(dispatch_order=True); the
C ABI's cti_ebag_options.tile_order / next_order / next_offsets).

Each call pools its batch and, in eight extra workgroups, sorts the next batch's tiles, most rows
per bag first within each XCD's share; the next call follows that order. Only the sequence in
which tiles start changes, so every output must equal the unordered call bit for bit: along a
stream of batches, when the batch that comes is not the one the order was made for, when the
order was made for another tile count (not followed), and when a buffer's entries are all out of
range. The order itself is checked on the host: its header, then each XCD range a permutation of
itself, sorted by rows per bag in chunks of 2048 tiles. Bags of at most SHORT rows are pooled by
one lane group in element order, so batches without longer bags also match the oracle bit for bit.
"""
import ctypes

import numpy as np
import pytest
import torch

from _cases import make_ids, make_table
from oracle import ebag_oracle as orc
from test_gpu_parity import to_dev, to_np

pytestmark = pytest.mark.gpu

MAGIC = 0x4F524452
CHUNK = 2048
SHORT = 24  # the tile kernels' default short-bag limit
V = 3000

# (table dtype, dim, fields, batch, max short-bag length, int8 tables, bags per tile)
SHAPES = [
    ("bf16", 128, 28, 512, 24, False, 8),   # the bf16 [*, 128] shape of the headline, smaller batch
    ("f32", 64, 5, 333, 40, False, 8),      # batch not a multiple of the tile
    ("bf16", 512, 3, 100, 30, False, 2),    # 64 lanes x 1 vector
    ("f32", 1024, 2, 50, 20, False, 2),     # 64 lanes x 4 vectors
    ("bf16", 128, 4, 200, 30, True, 8),     # int8 row-quantised tables
    ("bf16", 128, 1, 5, 48, False, 8),      # one tile: seven XCD ranges are empty
]


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


def _batches(seed, F, B, max_len, n=4):
    """n batches of one shape: short bags; some long bags; mostly empty; short bags again."""
    rng = np.random.default_rng(seed)
    out = []
    for k in range(n):
        L = rng.integers(0, max_len + 1, size=(F, B))
        if k == 1:
            L[:, ::7] = rng.integers(100, 250, size=L[:, ::7].shape)
        if k == 2:
            L[rng.random((F, B)) < 0.7] = 0
        off = np.zeros(F * B + 1, np.int64)
        np.cumsum(L.reshape(-1), out=off[1:])
        out.append((make_ids(rng, int(L.sum()), V), off, int(L.max(initial=0)) <= SHORT))
    return out


def _setup(pkg, dev, shape, seed):
    tdt, D, F, B, max_len, int8, _ = SHAPES[shape]
    rng = np.random.default_rng(seed)
    host = [make_table(rng, V, D, tdt) for _ in range(F)]
    tables = [to_dev(t, tdt, dev) for t in host]
    if int8:
        tables = [pkg.quantize_embedding_int8(t) for t in tables]
    odt = torch.float32 if tdt == "f32" else torch.bfloat16
    plain = pkg.PooledEmbedding(tables, out_dtype=odt)
    ordered = pkg.PooledEmbedding(tables, out_dtype=odt, dispatch_order=True)
    batches = _batches(seed + 1, F, B, max_len)
    dev_batches = [(torch.from_numpy(i).to(dev), torch.from_numpy(o).to(dev)) for i, o, _ in batches]
    return host, plain, ordered, batches, dev_batches


def _check_order(order, off, F, B, NB):
    """The order buffer made from offsets `off`: header, XCD ranges permuted, chunks sorted."""
    n = int(order[0])
    assert order[1] == MAGIC and order[2] == 0 and order[3] == 0
    tpf = -(-B // NB)
    assert n == F * tpf
    t = np.arange(n)
    fi = t // tpf
    b0 = (t - fi * tpf) * NB
    b1 = np.minimum(b0 + NB, B)
    per_bag = np.clip((off[fi * B + b1] - off[fi * B + b0]) // NB, 0, 63)
    body = order[4:4 + n]
    q, r = divmod(n, 8)
    for x in range(8):
        lo = x * (q + 1) if x < r else r * (q + 1) + (x - r) * q
        cnt = q + (1 if x < r else 0)
        for c0 in range(0, cnt, CHUNK):
            part = body[lo + c0:lo + min(cnt, c0 + CHUNK)]
            assert np.array_equal(np.sort(part), np.arange(lo + c0, lo + c0 + len(part))), (x, c0)
            assert (np.diff(per_bag[part]) <= 0).all(), (x, c0)


@pytest.mark.parametrize("shape", range(len(SHAPES)))
def test_ordered_stream_equals_unordered(pkg, dev, shape):
    tdt, D, F, B, _, int8, NB = SHAPES[shape]
    host, plain, ordered, batches, dev_batches = _setup(pkg, dev, shape, 700 + 10 * shape)
    n = len(dev_batches)
    for rep in range(2):
        for k, (v, o) in enumerate(dev_batches):
            # first pass: the batch that comes next; second pass: another one (a wrong guess)
            nk = k + 1 if rep == 0 else (k + 2) % n
            nxt = dev_batches[nk][1] if k + 1 < n else None
            got = ordered(v, o, next_offsets=nxt)
            if nxt is not None:
                _check_order(ordered._orders[ordered._cur].cpu().numpy(), batches[nk][1], F, B, NB)
            want = plain(v, o)
            torch.cuda.synchronize()
            assert torch.equal(_bits(got), _bits(want)), (rep, k)
            if rep == 0 and not int8 and batches[k][2]:
                odt = "f32" if tdt == "f32" else "bf16"
                ref = orc.pool_c(batches[k][0], batches[k][1], host, tdt, "sum", odt)
                assert np.array_equal(to_np(got, odt), ref), k


@pytest.mark.parametrize("F,D,B,NB", [(28, 128, 4096, 8), (64, 512, 4096, 2)])
def test_order_of_full_size_batches(pkg, dev, F, D, B, NB):
    # 28 x 4096 bags of bf16 [*, 128] rows: 14,336 tiles, one chunk per XCD range;
    # 64 x 4096 bags of bf16 [*, 512] rows: 131,072 tiles, eight chunks per XCD range
    rng = np.random.default_rng(F + D)
    tables = [to_dev(make_table(rng, 500, D, "bf16"), "bf16", dev) for _ in range(F)]
    plain = pkg.PooledEmbedding(tables)
    ordered = pkg.PooledEmbedding(tables, dispatch_order=True)
    batches = []
    for _ in range(3):
        L = np.minimum(rng.geometric(1 / 9, size=(F, B)) - 1, 256)
        off = np.zeros(F * B + 1, np.int64)
        np.cumsum(L.reshape(-1), out=off[1:])
        ids = make_ids(rng, int(off[-1]), 500)
        batches.append((off, torch.from_numpy(ids).to(dev), torch.from_numpy(off).to(dev)))
    for k in range(3):
        _, v, o = batches[k]
        nxt = batches[k + 1] if k + 1 < 3 else None
        got = ordered(v, o, next_offsets=nxt[2] if nxt else None)
        if nxt:
            _check_order(ordered._orders[ordered._cur].cpu().numpy(), nxt[0], F, B, NB)
        want = plain(v, o)
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(want)), k


def _forward(pkg, plan, v, o, out, tile_order=None, next_order=None, next_offsets=None, order_bytes=0):
    c = pkg._capi
    opts = c.Options()
    opts.tile_order, opts.next_order, opts.next_offsets, opts.order_bytes = tile_order, next_order, next_offsets, \
        order_bytes
    batch = (o.numel() - 1) // plan.num_fields
    return c.lib().cti_ebag_forward(v.data_ptr(), c.I64, v.numel(), o.data_ptr(), batch, plan.num_fields, plan._descs,
                                    plan._tdt, plan._pool, out.data_ptr(), plan._odt, plan.width, None, 0,
                                    ctypes.byref(opts), torch.cuda.current_stream().cuda_stream)


def test_orders_for_other_launches_are_not_followed(pkg, dev):
    c = pkg._capi
    F, D, V_ = 6, 128, 400
    rng = np.random.default_rng(77)
    tables = [to_dev(make_table(rng, V_, D, "bf16"), "bf16", dev) for _ in range(F)]
    plain = pkg.PooledEmbedding(tables)

    def batch(B):
        L = rng.integers(0, 40, size=(F, B))
        L[:, ::5] = 200
        off = np.zeros(F * B + 1, np.int64)
        np.cumsum(L.reshape(-1), out=off[1:])
        return torch.from_numpy(make_ids(rng, int(off[-1]), V_)).to(dev), torch.from_numpy(off).to(dev)

    small, big = batch(150), batch(300)
    nbytes = c.lib().cti_ebag_order_bytes(300, F)
    bufs = [torch.zeros(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(2)]
    out = torch.empty((300, F * D), dtype=torch.bfloat16, device=dev)
    want_small, want_big = plain(*small), plain(*big)
    # the small batch makes an order for a small batch (19 tiles per field) ...
    out_s = torch.empty((150, F * D), dtype=torch.bfloat16, device=dev)
    assert _forward(pkg, plain, *small, out_s, None, bufs[0].data_ptr(), small[1].data_ptr(), nbytes) == c.OK
    torch.cuda.synchronize()
    assert torch.equal(_bits(out_s), _bits(want_small))
    assert bufs[0][0].item() == F * 19 and bufs[0][1].item() == MAGIC
    # ... which the big batch (38 tiles per field) does not follow
    assert _forward(pkg, plain, *big, out, bufs[0].data_ptr(), None, None, nbytes) == c.OK
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(want_big))
    # a zeroed buffer, and one with the right header but every entry out of range
    for fill in (0, -1):
        bufs[1].fill_(fill)
        if fill:
            bufs[1][0], bufs[1][1] = F * 38, MAGIC
        out.zero_()
        assert _forward(pkg, plain, *big, out, bufs[1].data_ptr(), None, None, nbytes) == c.OK
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(want_big)), fill


def test_python_plan_rejects_what_it_cannot_order(pkg, dev):
    rng = np.random.default_rng(5)
    t128 = to_dev(make_table(rng, 100, 128, "bf16"), "bf16", dev)
    t64 = to_dev(make_table(rng, 100, 64, "bf16"), "bf16", dev)
    with pytest.raises(ValueError, match="use_bins"):
        pkg.PooledEmbedding([t128], dispatch_order=True, use_bins=True, max_batch=8)
    off = torch.arange(9, dtype=torch.int64, device=dev)
    ids = torch.zeros(8, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError, match="dispatch_order"):
        pkg.PooledEmbedding([t128])(ids, off, next_offsets=off)
    plan = pkg.PooledEmbedding([t128], dispatch_order=True)
    with pytest.raises(ValueError, match="next_offsets"):
        plan(ids, off, next_offsets=off[:5])
    # fields of two widths take the mixed-width launch, which has no dispatch order
    mixed = pkg.PooledEmbedding([t128, t64], dispatch_order=True)
    off2 = torch.arange(17, dtype=torch.int64, device=dev)
    ids2 = torch.zeros(16, dtype=torch.int64, device=dev)
    with pytest.raises(pkg._capi.EbagError):
        mixed(ids2, off2, next_offsets=off2)


@pytest.mark.parametrize("seed", range(40))
def test_random_shapes_ordered_equal_unordered(pkg, dev, seed):
    # one row width per case (the order needs one tiled row shape): any width and dtype; widths
    # that are not whole 16-byte vectors take the generic kernel, which must refuse the order
    rng = np.random.default_rng(9000 + seed)
    tdt = ["f32", "bf16", "f16"][seed % 3]
    D = int(rng.choice([1, 4, 8, 16, 24, 32, 64, 96, 128, 256, 512, 1024]))
    F, B = int(rng.integers(1, 41)), int(rng.integers(1, 601))
    Vs = int(rng.integers(1, 3000))
    tables = [to_dev(make_table(rng, Vs, D, tdt), tdt, dev) for _ in range(F)]
    odt = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    plain = pkg.PooledEmbedding(tables, out_dtype=odt, pooling=["sum", "mean"][seed % 2])
    ordered = pkg.PooledEmbedding(tables, out_dtype=odt, pooling=["sum", "mean"][seed % 2], dispatch_order=True)
    batches = []
    for k in range(3):
        L = rng.integers(0, int(rng.integers(1, 80)) + 1, size=(F, B))
        if k == 1:
            L[:, ::int(rng.integers(2, 9))] = int(rng.integers(50, 400))
        off = np.zeros(F * B + 1, np.int64)
        np.cumsum(L.reshape(-1), out=off[1:])
        batches.append((torch.from_numpy(make_ids(rng, int(off[-1]), Vs)).to(dev), torch.from_numpy(off).to(dev)))
    # the tiled kernels take rows of 1, 2, 4, ..., 64, 128 or 256 whole 16-byte vectors
    row_bytes = D * (4 if tdt == "f32" else 2)
    tiled = row_bytes % 16 == 0 and row_bytes // 16 in {1, 2, 4, 8, 16, 32, 64, 128, 256}
    try:
        for k, (v, o) in enumerate(batches):
            got = ordered(v, o, next_offsets=batches[k + 1][1] if k + 1 < len(batches) else None)
            want = plain(v, o)
            torch.cuda.synchronize()
            assert torch.equal(_bits(got) if got.element_size() == 4 else got.view(torch.int16),
                               _bits(want) if want.element_size() == 4 else want.view(torch.int16)), k
    except pkg._capi.EbagError as e:
        assert not tiled and e.status == pkg._capi.EUNSUPPORTED, e  # refused before any launch
    else:
        assert tiled, "a job of the generic kernel took a dispatch order"


# ---- orders made on the host where the offsets are produced (cti_ebag_order_host) -------------
HOST_SHAPES = [  # (table dtype, dim, slots, batch, max bag length)
    ("bf16", 128, 28, 700, 60),
    ("f32", 64, 5, 333, 300),
    ("bf16", 512, 3, 100, 30),
    ("f32", 1024, 2, 50, 20),
    ("bf16", 128, 1, 5, 48),
]


def _reference_batch(rng, S, B, max_len, long_every=0):
    L = rng.integers(0, max_len + 1, size=(S, B))
    if long_every:
        L[:, ::long_every] = rng.integers(100, 250, size=L[:, ::long_every].shape)
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    return make_ids(rng, int(L.sum()), V), ro.reshape(-1), vo


@pytest.mark.parametrize("shape", range(len(HOST_SHAPES)))
def test_host_order_launch_equals_plain(pkg, dev, shape):
    """The drop-in launch following a host-made order equals the plain launch bit for bit, for its
    own batch, for the order of another batch of the same size, and with an order made for
    another batch size (not followed); bags of at most SHORT rows also equal the oracle."""
    tdt, D, S, B, max_len = HOST_SHAPES[shape]
    print(f"host order: {tdt} D={D} S={S} B={B}", flush=True)
    rng = np.random.default_rng(200 + shape)
    table = make_table(rng, V, D, tdt)
    w = to_dev(table, tdt, dev)
    tdt_t = {"bf16": torch.bfloat16, "f32": torch.float32}[tdt]
    batches = [_reference_batch(rng, S, B, max_len, long_every=5 if k == 1 else 0) for k in range(3)]
    small = _reference_batch(rng, S, max(1, B // 3), max_len)
    for k, (v, ro, vo) in enumerate(batches):
        dv, dro, dvo = (torch.from_numpy(x).to(dev) for x in (v, ro, vo))
        plain = torch.empty((B, S * D), dtype=tdt_t, device=dev)
        pkg.fused_all_slots_embedding(dv, dvo, dro, w, plain, B, D, V - 1)
        own = pkg.make_tile_order(torch.from_numpy(ro), B, S, tdt_t, D)
        other = pkg.make_tile_order(torch.from_numpy(batches[(k + 1) % 3][1]), B, S, tdt_t, D)
        # an order made for another batch size, in a buffer large enough for this launch (a smaller
        # buffer is refused on the host: the launch would read past it)
        foreign = pkg.make_tile_order(torch.from_numpy(small[1]), max(1, B // 3), S, tdt_t, D,
                                      out=torch.zeros(pkg.order_bytes(B, S) // 4, dtype=torch.int32))
        short = torch.from_numpy(own.numpy()[:4].copy())  # the header alone: smaller than any launch needs
        with pytest.raises(pkg.EbagError, match="order buffers"):
            pkg.fused_all_slots_embedding(dv, dvo, dro, w, torch.empty_like(plain), B, D, V - 1,
                                          tile_order=short.to(dev))
        for order in (own, other, foreign):
            got = torch.empty_like(plain)
            pkg.fused_all_slots_embedding(dv, dvo, dro, w, got, B, D, V - 1, tile_order=order.to(dev))
            torch.cuda.synchronize()
            assert torch.equal(_bits(got), _bits(plain))
        if int(np.diff(ro.reshape(S, B + 1), axis=1).max(initial=0)) <= SHORT:
            want = orc.pool_c(v, ro, [table] * S, tdt, "sum", tdt, batch=B, val_base=vo)
            assert np.array_equal(to_np(plain, tdt), want)


def test_stager_with_orders_matches_oracle(pkg, dev):
    """InputStager(order_for=...) sends each batch's host-made order in the same copy; the staged,
    ordered pooling equals the oracle's pooling of the host batch bit for bit."""
    S, D = 28, 128
    rng = np.random.default_rng(17)
    table = make_table(rng, V, D, "bf16")
    w = to_dev(table, "bf16", dev)
    hosts = []
    for k in range(5):
        B = int(rng.integers(1, 300))
        v, ro, vo = _reference_batch(rng, S, B, 40)
        hosts.append(({"_flat_values": torch.from_numpy(v), "_flat_row_offsets": torch.from_numpy(ro),
                       "_val_offsets": torch.from_numpy(vo)}, B))
    # every other batch carries the order its producer made; the stager ships that one
    for k, (h, B) in enumerate(hosts):
        if k % 2:
            h["_tile_order"] = pkg.make_tile_order(h["_flat_row_offsets"], B, S, torch.bfloat16, D)
    max_nnz = max(h["_flat_values"].numel() for h, _ in hosts)
    stager = pkg.InputStager(max_nnz, S, 300, dev, depth=2, order_for=(torch.bfloat16, D))
    outs = []
    for h, B in hosts:
        staged = pkg.move_model_inputs_to_device(h, dev, S, stager=stager)
        assert staged["_tile_order"].dtype == torch.int32
        want_order = h.get("_tile_order")
        if want_order is not None:
            assert torch.equal(staged["_tile_order"].cpu(), want_order)
        outs.append(pkg.fused_embedding(staged, w, S).clone())
        stager.release(staged)
    torch.cuda.synchronize()
    for (h, B), got in zip(hosts, outs):
        want = orc.pool_c(h["_flat_values"].numpy(), h["_flat_row_offsets"].numpy(), [table] * S, "bf16", "sum",
                          batch=B, val_base=h["_val_offsets"].numpy())
        assert np.array_equal(to_np(got, "bf16"), want)


@pytest.mark.parametrize("shape", range(len(HOST_SHAPES)))
def test_plan_follows_host_order_global_layout(pkg, dev, shape):
    """PooledEmbedding(...)(values, offsets, tile_order=...) with an order made on the host from
    the global offsets equals the plain call bit for bit (own batch, another batch's order,
    another batch size's order in a large enough buffer), per-field tables, sum and mean."""
    tdt, D, S, B, max_len = HOST_SHAPES[shape]
    print(f"plan host order: {tdt} D={D} S={S} B={B}", flush=True)
    rng = np.random.default_rng(300 + shape)
    tables = [to_dev(make_table(rng, V, D, tdt), tdt, dev) for _ in range(S)]
    tdt_t = {"bf16": torch.bfloat16, "f32": torch.float32}[tdt]
    for pooling in ("sum", "mean"):
        plan = pkg.PooledEmbedding(tables, pooling=pooling)
        offs = []
        for k in range(3):
            L = rng.integers(0, max_len + 1, size=(S, B))
            if k == 1:
                L[:, ::5] = rng.integers(100, 250, size=L[:, ::5].shape)
            o = np.zeros(S * B + 1, np.int64)
            np.cumsum(L.reshape(-1), out=o[1:])
            offs.append(o)
        for k, o in enumerate(offs):
            v = torch.from_numpy(make_ids(rng, int(o[-1]), V)).to(dev)
            do = torch.from_numpy(o).to(dev)
            plain = plan(v, do)
            small_o = offs[(k + 2) % 3][:S * max(1, B // 4) + 1].copy()
            orders = [pkg.make_tile_order(torch.from_numpy(o), B, S, tdt_t, D),
                      pkg.make_tile_order(torch.from_numpy(offs[(k + 1) % 3]), B, S, tdt_t, D),
                      pkg.make_tile_order(torch.from_numpy(small_o), max(1, B // 4), S, tdt_t, D,
                                          out=torch.zeros(pkg.order_bytes(B, S) // 4, dtype=torch.int32))]
            for order in orders:
                got = plan(v, do, tile_order=order.to(dev))
                torch.cuda.synchronize()
                assert torch.equal(_bits(got), _bits(plain)), pooling
