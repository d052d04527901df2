"""Flat-layout builders and their invariants on the CPU (no GPU)."""
import numpy as np
import pytest
import torch

from _cases import random_case
from oracle import ebag_oracle as orc


def _samples(rng, n, S, V=1000, p_missing=0.2, max_len=5):
    out = []
    for _ in range(n):
        d = {}
        for s in range(1, S + 1):
            if rng.random() >= p_missing:
                d[s] = list(rng.integers(0, V, rng.integers(0, max_len + 1)))
        out.append(d)
    return out


def test_collate_builder_matches_restatement(pkg):
    rng = np.random.default_rng(0)
    feas = _samples(rng, 37, 28)
    got = pkg.collate_flat_layout(feas, 28)
    fv, fro, vo, slots = orc.collate_layout(feas, 28)
    assert np.array_equal(got["_flat_values"].numpy(), fv)
    assert np.array_equal(got["_flat_row_offsets"].numpy(), fro)
    assert np.array_equal(got["_val_offsets"].numpy(), vo)
    for s in range(28):
        assert np.array_equal(got[s + 1][0].numpy(), slots[s][0])
        assert np.array_equal(got[s + 1][1].numpy(), slots[s][1])


def test_collate_brute_force_tiny():
    feas = [{1: [5, 6], 2: [7]}, {2: [8, 9, 10]}, {}]
    fv, fro, vo, _ = orc.collate_layout(feas, 2)
    assert list(fv) == [5, 6, 7, 8, 9, 10]
    assert list(fro) == [0, 2, 2, 2, 0, 1, 4, 4]
    assert list(vo) == [0, 2]


def test_prebuild_matches_collate(pkg):
    rng = np.random.default_rng(1)
    feas = _samples(rng, 20, 28)
    collated = pkg.collate_flat_layout(feas, 28)
    batch = {s: collated[s] for s in range(1, 29)}
    assert pkg.prebuild_flat_layout(batch, 28)
    for k in ("_flat_values", "_flat_row_offsets", "_val_offsets"):
        assert torch.equal(batch[k], collated[k])
    assert not pkg.prebuild_flat_layout(batch, 28)  # already has the flat tensors
    assert not pkg.prebuild_flat_layout({1: collated[1]}, 28)  # missing slots


def test_global_offsets_closed_form():
    case = random_case(3, F=5, B=11)
    ro, vo = case.reference_layout()
    g = orc.to_global_offsets(vo, ro, case.B, len(case.values))
    assert np.array_equal(g, case.offsets)


def _layout_of(case):
    ro, vo = case.reference_layout()
    return case.values, ro, vo


def test_merge_restatement_brute_force_tiny():
    a = (np.array([1, 2, 3]), np.array([0, 1, 2, 0, 1, 1]), np.array([0, 2]))   # S=2, B=2
    b = (np.array([4, 5]), np.array([0, 1, 0, 1]), np.array([0, 1]))            # S=2, B=1
    v, ro, vo = orc.merge_layouts([a, b], 2)
    assert list(v) == [1, 2, 4, 3, 5]
    assert list(ro) == [0, 1, 2, 3, 0, 1, 1, 2]
    assert list(vo) == [0, 3]


@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_merge_then_pool_equals_pool_then_concat(pooling):
    """Invariant: pooling a merged batch = stacking the sub-batches' pooled rows."""
    S = 6
    subs = [random_case(40 + k, F=S, B=B, dims=(32,), V=(300,), tdt="bf16") for k, B in enumerate((5, 9, 1, 7))]
    table = subs[0].tables[0]
    pooled = []
    for c in subs:
        ro, vo = c.reference_layout()
        pooled.append(orc.pool_c(c.values, ro, [table] * S, "bf16", pooling, "f32", batch=c.B, val_base=vo))
    v, ro, vo = orc.merge_layouts([_layout_of(c) for c in subs], S)
    B = sum(c.B for c in subs)
    merged = orc.pool_c(v, ro, [table] * S, "bf16", pooling, "f32", batch=B, val_base=vo)
    assert np.array_equal(merged, np.concatenate(pooled, axis=0))


def test_pair_merge_int32_round_trip():
    S = 3
    subs = [random_case(60 + k, F=S, B=4, V=(1000,), clamp_frac=0) for k in range(2)]
    lays = [_layout_of(c) for c in subs]
    a = orc.merge_layouts(lays, S)
    b = orc.merge_pair_layouts(lays, S)
    big = [(lays[0][0] + 2 ** 31, lays[0][1], lays[0][2]), lays[1]]
    c = orc.merge_pair_layouts(big, S)
    ids_ok = all((x >= 0).all() and (x < 2 ** 31).all() for x, _, _ in lays)
    assert ids_ok and all(np.array_equal(x, y) for x, y in zip(a, b))
    assert not np.array_equal(c[0], orc.merge_layouts(big, S)[0])  # ids >= 2^31 wrap there only


def test_pair_merge_wraps_as_int32_does():
    """The pair merge's .int() / .long() (online_best/infer.py:3008-3009, :3019-3020) is a
    two's-complement wrap to int32: closed forms (2^31 + k -> k - 2^31, -2^31 - 5 -> 2^31 - 5,
    2^32 + 7 -> 7) and torch's own .int().long() on the same ids. A saturating cast fails both."""
    import torch

    ids = np.array([2 ** 31 + 3, -2 ** 31 - 5, 2 ** 32 + 7, 2 ** 31 - 1, -2 ** 31, 5, -1, 2 ** 40 + 2 ** 31],
                   dtype=np.int64)
    want = np.array([3 - 2 ** 31, 2 ** 31 - 5, 7, 2 ** 31 - 1, -2 ** 31, 5, -1, -2 ** 31], dtype=np.int64)
    S, B = 2, 2
    lay = (ids, np.array([0, 3, 4, 0, 1, 4], np.int64), np.array([0, 4], np.int64))
    empty = (np.zeros(0, np.int64), np.zeros(S * (B + 1), np.int64), np.zeros(S, np.int64))
    v, o, vo = orc.merge_pair_layouts([lay, empty], S)
    assert np.array_equal(v, want)
    assert np.array_equal(v, torch.from_numpy(ids).int().long().numpy())
    # offsets pass through the same casts; at these sizes they are unchanged
    assert np.array_equal(o, orc.merge_layouts([lay, empty], S)[1]) and np.array_equal(vo, [0, 4])
    # a saturating cast (the mistake this rejects) gives other ids
    assert not np.array_equal(np.clip(ids, -2 ** 31, 2 ** 31 - 1), want)


def test_workload_shapes(pkg):
    W = pkg.workloads
    wl = W.make("small-fp32", seed=0)
    assert wl.num_fields == 28 and wl.batch == 256
    L = wl.lengths()
    assert L.max() <= 32 and 0.05 < (L == 0).mean() < 0.15
    assert wl.offsets[0] == 0 and wl.offsets[-1] == wl.nnz
    assert wl.values.min() >= 0 and wl.values.max() < 10_000
    wl2 = W.make("small-fp32", seed=0)
    assert np.array_equal(wl.values, wl2.values)
    # lazy-32k: the merged layout equals the field-wise merge of its sub-batches
    lz = W.make("lazy-32k", seed=3, sub_batch=64, vocab=5000)
    lays = []
    for sb in lz.sub_batches:
        ro = np.concatenate([np.concatenate([[0], np.cumsum(sb.lengths()[f * 64:(f + 1) * 64])]) for f in range(28)])
        vo = sb.offsets[::64][:28]
        lays.append((sb.values, ro, vo))
    v, ro, vo = orc.merge_layouts(lays, 28)
    assert np.array_equal(v, lz.values)
    assert np.array_equal(orc.to_global_offsets(vo, ro, lz.batch, lz.nnz), lz.offsets)
