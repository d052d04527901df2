"""The allocation-free entry point cti_ebag_forward_static, through the C ABI, on the GPU.

Bar: on two calls in a row (the second with a smaller batch, fewer fields and other lengths) its
output equals, bit for bit, cti_ebag_forward's with a workspace the caller allocated, for the
length-binning path (which is the one that uses the static workspace), a plain call and a
mixed-width call; a binned job larger than the static workspace is refused before any launch.
"""
import ctypes
import types

import numpy as np
import pytest
import torch

from _cases import random_case

pytestmark = pytest.mark.gpu


def _tables(pkg, case, dev):
    tt = [torch.from_numpy(np.ascontiguousarray(t)).view(torch.int16).view(torch.bfloat16).to(dev)
          for t in case.tables]
    descs, _, code, width, _ = pkg.ops._table_descs(tt)
    return tt, descs, code, width


def _call(pkg, dev, case, use_bins, static):
    c = pkg._capi
    lib = c.lib()
    tt, descs, code, width = _tables(pkg, case, dev)
    v = torch.from_numpy(case.values).to(dev)
    o = torch.from_numpy(case.offsets).to(dev)
    out = torch.full((case.B, width), float("nan"), dtype=torch.float32, device=dev)
    opts = c.Options()
    opts.use_bins = int(use_bins)
    opts.block_threshold = 32
    opts.split_threshold = 192
    stream = torch.cuda.current_stream(dev).cuda_stream
    if static:
        rc = lib.cti_ebag_forward_static(v.data_ptr(), c.I64, v.numel(), o.data_ptr(), case.B, case.F, descs, code,
                                         c.SUM, out.data_ptr(), c.F32, width, ctypes.byref(opts), stream)
    else:
        ws_bytes = lib.cti_ebag_workspace_bytes(case.B, case.F)
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
        rc = lib.cti_ebag_forward(v.data_ptr(), c.I64, v.numel(), o.data_ptr(), case.B, case.F, descs, code, c.SUM,
                                  out.data_ptr(), c.F32, width, ws.data_ptr(), ws_bytes, ctypes.byref(opts), stream)
    c.check(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_first_call_inside_graph_capture(pkg, dev):
    """Defined first in the last-collected file, so that in a test run (and in a process of its
    own) this is the first call of the entry on the device: it is made inside a HIP graph capture
    (the setup on first use, a symbol lookup and a fill kernel for the list counters, is captured
    with it), then the graph is replayed on two batches written into the captured buffers; each
    replay equals cti_ebag_forward with a caller-allocated workspace, bit for bit."""
    c = pkg._capi
    lib = c.lib()
    cases = [random_case(40 + k, F=7, B=120, dims=(128,), V=(900,), max_len=25, tdt="bf16", long_every=9,
                         long_len=260 + 10 * k) for k in range(2)]
    nnz = max(x.values.size for x in cases)
    tt, descs, code, width = _tables(pkg, cases[0], dev)
    v = torch.zeros(nnz, dtype=torch.int64, device=dev)
    o = torch.zeros(cases[0].offsets.size, dtype=torch.int64, device=dev)
    out = torch.zeros((cases[0].B, width), dtype=torch.float32, device=dev)
    opts = c.Options()
    opts.use_bins, opts.block_threshold, opts.split_threshold = 1, 32, 192
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.cti_ebag_forward_static(v.data_ptr(), c.I64, nnz, o.data_ptr(), cases[0].B, cases[0].F, descs, code,
                                         c.SUM, out.data_ptr(), c.F32, width, ctypes.byref(opts), stream)
    c.check(rc)
    torch.cuda.synchronize()
    for rep in range(2):
        for case in cases:
            ids = np.zeros(nnz, np.int64)
            ids[:case.values.size] = case.values
            # bags past the case's nnz are never read: the offsets end at case.values.size
            v.copy_(torch.from_numpy(ids))
            o.copy_(torch.from_numpy(case.offsets))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = out.cpu().numpy().copy()
            # the same batch over the captured tables (the first case's), eagerly
            same_tables = types.SimpleNamespace(values=case.values, offsets=case.offsets, tables=cases[0].tables,
                                                F=case.F, B=case.B)
            want = _call(pkg, dev, same_tables, True, static=False)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rep, case.values.size)


CASES = [  # (seed, F, B, dims, max_len, long_every, long_len): the second call of each pair is smaller
    ((1, 12, 400, (128,), 40, 7, 700), (2, 5, 90, (128,), 30, 5, 250)),
    ((3, 9, 300, (32, 64, 128), 50, 6, 900), (4, 3, 40, (64, 32), 20, 4, 300)),
]


@pytest.mark.parametrize("use_bins", [True, False])
@pytest.mark.parametrize("pair", range(len(CASES)))
def test_static_entry_equals_workspace_entry(pkg, dev, use_bins, pair):
    for seed, F, B, dims, max_len, every, long_len in CASES[pair]:
        print(f"static entry: seed={seed} F={F} B={B} dims={dims} bins={use_bins}", flush=True)
        case = random_case(seed, F=F, B=B, dims=dims, V=(3000, 700), max_len=max_len, tdt="bf16",
                           long_every=every, long_len=long_len)
        got = _call(pkg, dev, case, use_bins, static=True)
        want = _call(pkg, dev, case, use_bins, static=False)
        assert not np.isnan(got).any()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_static_entry_refuses_jobs_beyond_its_workspace(pkg, dev):
    c = pkg._capi
    lib = c.lib()
    opts = c.Options()
    opts.use_bins = 1
    rows = 1_398_090  # batch_size * min(num_fields, 64) the static workspace holds
    descs = (c.Table * 2)()
    for d in descs:
        d.data, d.rows, d.row_stride, d.dim, d.out_col = 16, 10, 64, 64, 0
    rc = lib.cti_ebag_forward_static(16, c.I64, 10, 16, rows // 2 + 1, 2, descs, c.BF16, c.SUM, 16, c.BF16, 64,
                                     ctypes.byref(opts), None)
    assert rc == c.EWORKSPACE and "allocation-free" in c.last_error()
