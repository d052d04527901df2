"""Calls whose fields have rows of several widths (online_best/infer.py:805-827 per field, with
per-field tables as in baseline/infer.py:256-263).

Fields whose rows are 4 to 64 lanes of one 16-byte vector (8-byte for int8) share one launch
sequence: one binning pass, one main kernel that runs each tile's own row shape, and one list
kernel that picks each listed bag's shape at run time. Rows of other widths keep launches of
their own. Every path pools a bag in the same element order and combines partial sums in the
same order as a call holding that field alone, so a mixed call must equal the per-field calls
bit for bit, with and without binning; the oracle pins the unsplit bags bit for bit as well.
"""
import numpy as np
import pytest
import torch

from _cases import random_case
from oracle import ebag_oracle as orc
from test_gpu_parity import TORCH_DT, to_dev, to_np

pytestmark = pytest.mark.gpu

# widths per table type: the mixed range (64 B - 1 KB rows), narrower rows (own launches) and a
# width that is not a whole number of lane vectors (element-wise kernel)
DIMS = {"bf16": (32, 64, 128, 256, 512, 8, 16, 40),
        "f32": (16, 32, 64, 128, 256, 4, 8, 20),
        "f16": (32, 128, 512, 16, 24)}
BIN_SETTINGS = [dict(use_bins=False), dict(use_bins=True, block_threshold=24, split_threshold=100),
                dict(use_bins=True, block_threshold=1, split_threshold=0)]


def _pool(pkg, dev, values, offsets, tables, pooling, odt, **kw):
    v = torch.from_numpy(np.ascontiguousarray(values)).to(dev)
    o = torch.from_numpy(np.ascontiguousarray(offsets)).to(dev)
    out = pkg.embedding_bag_pooled(v, o, tables, pooling=pooling, out_dtype=TORCH_DT[odt], **kw)
    torch.cuda.synchronize()
    return to_np(out, odt)


def _per_field(pkg, dev, case, tables, pooling, odt, **kw):
    """Each field pooled by a call of its own (one row shape per launch), columns concatenated."""
    B = case.B
    cols = []
    for f in range(case.F):
        off = case.offsets[f * B:(f + 1) * B + 1]
        cols.append(_pool(pkg, dev, case.values, off, [tables[f]], pooling, odt, **kw))
    return np.concatenate(cols, axis=1)


@pytest.mark.parametrize("tdt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("bins", range(len(BIN_SETTINGS)))
def test_mixed_call_equals_per_field_calls(pkg, dev, tdt, pooling, bins):
    dims = DIMS[tdt]
    case = random_case(4100 + len(dims) + bins, F=2 * len(dims), B=77, dims=dims, V=(300, 2000), tdt=tdt,
                       max_len=40, long_every=9, long_len=260)
    tables = [to_dev(t, tdt, dev) for t in case.tables]
    odt = "f32" if tdt == "f32" else "bf16"
    kw = BIN_SETTINGS[bins]
    got = _pool(pkg, dev, case.values, case.offsets, tables, pooling, odt, **kw)
    want = _per_field(pkg, dev, case, tables, pooling, odt, **kw)
    assert np.array_equal(got, want)
    # bags that stay in the main kernel (up to 24 rows; with block_threshold 1 only single rows) are
    # pooled by one lane group in element order: oracle bit for bit
    ref = orc.pool_c(case.values, case.offsets, case.tables, tdt, pooling, odt)
    limit = 1 if kw.get("block_threshold") == 1 else 24
    col = 0
    for f in range(case.F):
        d = case.tables[f].shape[1]
        short = case.lengths[f] <= limit
        assert np.array_equal(got[short, col:col + d], ref[short, col:col + d]), f
        col += d


@pytest.mark.parametrize("bins", range(len(BIN_SETTINGS)))
def test_mixed_int8_call_equals_per_field_calls(pkg, dev, bins):
    dims = (32, 64, 128, 256, 512, 16)
    case = random_case(4200 + bins, F=12, B=65, dims=dims, V=(400,), tdt="bf16", max_len=40, long_every=7,
                       long_len=300)
    tables = [pkg.quantize_embedding_int8(to_dev(t, "bf16", dev)) for t in case.tables]
    kw = BIN_SETTINGS[bins]
    got = _pool(pkg, dev, case.values, case.offsets, tables, "sum", "f32", **kw)
    want = _per_field(pkg, dev, case, tables, "sum", "f32", **kw)
    assert np.array_equal(got, want)


def test_mixed_integer_tables_exact(pkg, dev):
    # integer-valued rows: every partial sum is exact, so every path equals the oracle bit for bit
    dims = (32, 64, 128, 256, 512)
    case = random_case(4300, F=10, B=90, dims=dims, V=(700,), tdt="bf16", kind="int", max_len=60, long_every=5,
                       long_len=1200)
    tables = [to_dev(t, "bf16", dev) for t in case.tables]
    want = orc.pool_c(case.values, case.offsets, case.tables, "bf16", "sum", "f32")
    for kw in BIN_SETTINGS + [dict(long_threshold=-1)]:
        got = _pool(pkg, dev, case.values, case.offsets, tables, "sum", "f32", **kw)
        assert np.array_equal(got, want), kw
