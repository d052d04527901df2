"""The C ABI without a GPU: the library loads, exports what include/cti_ebag.h declares, and
rejects malformed arguments on the host (no HIP call is reached)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cti_ebag.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cti_ebag_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("cti_ebag_fused_all_slots", "cti_ebag_forward", "cti_ebag_pack_slots", "cti_ebag_merge_batches",
              "cti_ebag_workspace_bytes", "cti_ebag_last_error", "cti_ebag_abi_version", "cti_ebag_layernorm",
              "cti_ebag_fused_all_slots_int8", "cti_ebag_quantize_int8", "cti_ebag_fused_all_slots_typed",
              "cti_ebag_narrow_ids", "cti_ebag_stage_copy", "cti_ebag_stage_offset",
              "cti_ebag_fused_all_slots_layernorm", "cti_ebag_order_bytes", "cti_ebag_layernorm_linear",
              "cti_ebag_layernorm_linear_workspace_bytes"):
        assert n in names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    raw = ctypes.CDLL(pkg._capi.LIB_PATH)
    for name in declared_functions():
        assert hasattr(raw, name), name
        assert name in pkg._capi.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.cti_ebag_abi_version() == pkg._capi.ABI_VERSION
    ver = int(re.search(r"#define CTI_EBAG_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert ver == pkg._capi.ABI_VERSION


def test_status_codes_match_header(pkg):
    text = open(HEADER).read()
    for name in ("OK", "EINVAL", "EUNSUPPORTED", "EHIP", "EWORKSPACE"):
        v = int(re.search(rf"#define CTI_EBAG_{name} \(?(-?\d+)\)?", text).group(1))
        assert getattr(pkg._capi, name) == v
    for name, attr in (("F32", "F32"), ("BF16", "BF16"), ("F16", "F16"), ("I8", "I8"), ("I64", "I64"),
                       ("I32", "I32"), ("SUM", "SUM"), ("MEAN", "MEAN")):
        v = int(re.search(rf"#define CTI_EBAG_{name} (\d+)", text).group(1))
        assert getattr(pkg._capi, attr) == v


def _forward(pkg, **kw):
    c = pkg._capi
    args = dict(values=1, index_type=c.I64, nnz=10, offsets=1, batch=4, num_fields=1, tables=None, tdt=c.BF16,
                pooling=c.SUM, out=1, odt=c.BF16, stride=128, ws=None, ws_bytes=0, opts=None, stream=None)
    args.update(kw)
    return c.lib().cti_ebag_forward(args["values"], args["index_type"], args["nnz"], args["offsets"], args["batch"],
                                    args["num_fields"], args["tables"], args["tdt"], args["pooling"], args["out"],
                                    args["odt"], args["stride"], args["ws"], args["ws_bytes"], args["opts"],
                                    args["stream"])


def _table(pkg, **kw):
    t = (pkg._capi.Table * 1)()
    t[0].data = kw.get("data", 64)
    t[0].rows = kw.get("rows", 100)
    t[0].row_stride = kw.get("row_stride", 128)
    t[0].dim = kw.get("dim", 128)
    t[0].out_col = kw.get("out_col", 0)
    t[0].row_scale = kw.get("row_scale", None)
    return t


def test_table_struct_matches_header(pkg):
    """Field order and size of cti_ebag_table as the header declares it."""
    text = open(HEADER).read()
    body = re.search(r"typedef struct cti_ebag_table \{(.*?)\} cti_ebag_table;", text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = re.findall(r"(\w+)\s*;", body)
    assert fields == [f[0] for f in pkg._capi.Table._fields_]
    assert ctypes.sizeof(pkg._capi.Table) == 40


@pytest.mark.parametrize("kw,needle", [
    (dict(index_type=7), "index type"),
    (dict(tdt=9), "table dtype"),
    (dict(odt=-1), "output dtype"),
    (dict(pooling=5), "pooling"),
    (dict(nnz=-1), "nnz"),
    (dict(batch=-2), "batch_size"),
    (dict(num_fields=-1), "num_fields"),
    (dict(stride=0), "out_row_stride"),
    (dict(tables=None), "tables"),
    (dict(offsets=None), "NULL"),
    (dict(out=None), "NULL"),
    (dict(values=None), "NULL"),
])
def test_forward_rejects_bad_arguments(pkg, kw, needle):
    if "tables" not in kw:
        kw["tables"] = _table(pkg)
    rc = _forward(pkg, **kw)
    assert rc == pkg._capi.EINVAL
    assert needle in pkg._capi.last_error()


@pytest.mark.parametrize("tkw,needle", [
    (dict(data=None), "data is NULL"),
    (dict(rows=0), "rows"),
    (dict(dim=0), "dim"),
    (dict(row_stride=64), "row_stride"),
    (dict(out_col=64), "outside the output row"),
    (dict(out_col=-1), "outside the output row"),
])
def test_forward_rejects_bad_tables(pkg, tkw, needle):
    rc = _forward(pkg, tables=_table(pkg, **tkw))
    assert rc == pkg._capi.EINVAL
    assert needle in pkg._capi.last_error()


def test_forward_zero_sized_calls_are_no_ops(pkg):
    assert _forward(pkg, batch=0, tables=None, values=None, offsets=None, out=None) == pkg._capi.OK
    assert _forward(pkg, num_fields=0, tables=None) == pkg._capi.OK
    assert pkg._capi.last_error() == ""


def test_fused_all_slots_rejects_bad_arguments(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_fused_all_slots
    assert f(1, 1, 1, 1, c.BF16, 1, 4, 28, 0, 10, 5, None) == c.EINVAL
    assert "emb_dim" in c.last_error()
    assert f(1, 1, 1, 1, c.BF16, 1, 4, 28, 64, -1, 5, None) == c.EINVAL
    assert "max_idx" in c.last_error()
    assert f(1, 1, 1, 1, 3, 1, 4, 28, 64, 10, 5, None) == c.EINVAL
    assert f(1, None, 1, 1, c.BF16, 1, 4, 28, 64, 10, 5, None) == c.EINVAL
    assert f(None, 1, 1, 1, c.BF16, 1, 4, 28, 64, 10, 5, None) == c.EINVAL  # values NULL with nnz > 0
    assert f(None, None, None, None, c.BF16, None, 0, 28, 64, 10, 0, None) == c.OK  # empty batch


def test_pack_and_merge_reject_bad_arguments(pkg):
    c = pkg._capi
    lib = c.lib()
    nnz = (ctypes.c_int64 * 1)(-1)
    ptrs = (ctypes.c_void_p * 1)(16)
    assert lib.cti_ebag_pack_slots(ptrs, ptrs, nnz, 1, 4, 16, 16, 16, None, None) == c.EINVAL
    assert lib.cti_ebag_pack_slots(None, ptrs, nnz, 1, 4, 16, 16, 16, None, None) == c.EINVAL
    assert lib.cti_ebag_pack_slots(ptrs, ptrs, nnz, 0, 4, None, None, None, None, None) == c.OK
    bs = (ctypes.c_int64 * 33)(*([1] * 33))
    many = (ctypes.c_void_p * 33)(*([16] * 33))
    assert lib.cti_ebag_merge_batches(many, many, many, bs, bs, 33, 28, 16, 16, 16, None, None) == c.EUNSUPPORTED
    assert lib.cti_ebag_merge_batches(many, many, many, bs, bs, 2, 40000, 16, 16, 16, None, None) == c.EUNSUPPORTED
    neg = (ctypes.c_int64 * 2)(-1, 1)
    assert lib.cti_ebag_merge_batches(many, many, many, neg, bs, 2, 28, 16, 16, 16, None, None) == c.EINVAL
    # the pair merge's int32 form checks its arguments the same way
    assert lib.cti_ebag_merge_batches_int32(many, many, many, bs, bs, 33, 28, 16, 16, 16, None, None) == c.EUNSUPPORTED
    assert lib.cti_ebag_merge_batches_int32(many, many, many, neg, bs, 2, 28, 16, 16, 16, None, None) == c.EINVAL
    assert lib.cti_ebag_merge_batches_int32(many, many, many, bs, bs, 0, 28, None, None, None, None, None) == c.OK


def test_workspace_query(pkg):
    lib = pkg._capi.lib()
    assert lib.cti_ebag_workspace_bytes(4096, 28) == 256 + 24 * 4096 * 28
    assert lib.cti_ebag_workspace_bytes(10, 100) == 256 + 24 * 10 * 64
    assert lib.cti_ebag_workspace_bytes(-1, 28) < 0


def test_order_query(pkg):
    lib = pkg._capi.lib()
    assert lib.cti_ebag_order_bytes(4096, 28) == 16 + 4 * 4096 * 28
    assert lib.cti_ebag_order_bytes(10, 100) == 16 + 4 * 10 * 64
    assert lib.cti_ebag_order_bytes(-1, 28) < 0


def test_options_struct_matches_header(pkg):
    text = open(HEADER).read()
    body = re.search(r"typedef struct cti_ebag_options \{(.*?)\} cti_ebag_options;", text, re.S).group(1)
    fields = re.findall(r"(\w+)\s*;", re.sub(r"/\*.*?\*/", "", body, flags=re.S))
    assert fields == [f for f, _ in pkg._capi.Options._fields_]
    assert ctypes.sizeof(pkg._capi.Options) == 48


def test_dispatch_order_rejects_bad_arguments(pkg):
    """Every case fails a host-side check, so nothing is launched (the pointers are not real).
    One field of bf16 rows of 128 (16 lanes x 8 values, 8 bags per tile), batch 4: one tile."""
    c = pkg._capi

    def call(tables=None, num_fields=1, out=256, stride=128, ws=None, ws_bytes=0, use_bins=0, **o):
        opts = c.Options()
        opts.use_bins = use_bins
        for k, v in o.items():
            assert k in dict(c.Options._fields_)
            setattr(opts, k, v)
        return _forward(pkg, tables=tables if tables is not None else _table(pkg, data=256), num_fields=num_fields,
                        out=out, stride=stride, ws=ws, ws_bytes=ws_bytes, opts=ctypes.byref(opts))

    assert call(tile_order=258, order_bytes=1 << 20) == c.EINVAL and "aligned" in c.last_error()
    assert call(next_order=256, order_bytes=1 << 20) == c.EINVAL and "next_offsets" in c.last_error()
    assert call(tile_order=256, order_bytes=0) == c.EINVAL
    assert call(tile_order=256, next_order=264, next_offsets=512, order_bytes=64) == c.EINVAL
    assert "overlap" in c.last_error()
    assert call(tile_order=256, order_bytes=19) == c.EINVAL and "20" in c.last_error()  # 4 + 1 entries
    assert call(tile_order=256, order_bytes=64, use_bins=1, ws=256, ws_bytes=1 << 20) == c.EUNSUPPORTED
    # a misaligned output takes the generic kernel, which has no dispatch order
    assert call(tile_order=256, order_bytes=64, out=2) == c.EUNSUPPORTED
    # two row widths take the mixed-width launch
    two = (c.Table * 2)()
    for i, (d, col) in enumerate(((128, 0), (64, 128))):
        two[i].data, two[i].rows, two[i].row_stride, two[i].dim, two[i].out_col = 256, 100, d, d, col
    assert call(tables=two, stride=192, num_fields=2, tile_order=256, order_bytes=1 << 10) == c.EUNSUPPORTED


def test_binning_requires_a_workspace(pkg):
    c = pkg._capi
    opts = c.Options()
    opts.use_bins = 1
    rc = _forward(pkg, tables=_table(pkg), opts=ctypes.byref(opts))
    assert rc == c.EWORKSPACE and "workspace" in c.last_error()
    rc = _forward(pkg, tables=_table(pkg), opts=ctypes.byref(opts), ws=256, ws_bytes=100)
    assert rc == c.EWORKSPACE
    rc = _forward(pkg, tables=_table(pkg), opts=ctypes.byref(opts), ws=8, ws_bytes=1 << 20)
    assert rc == c.EINVAL and "aligned" in c.last_error()


def test_python_wrappers_validate_before_any_launch(pkg):
    w = torch.zeros(10, 8)
    v = torch.zeros(3, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.fused_all_slots_embedding(v, v[:1], torch.zeros(5, dtype=torch.int64), w, torch.zeros(4, 8), 4, 8, 9)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.embedding_bag_pooled(v, torch.zeros(5, dtype=torch.int64), [w])
    with pytest.raises(ValueError, match="at least one table"):
        pkg.embedding_bag_pooled(v, torch.zeros(5, dtype=torch.int64), [])
    with pytest.raises(TypeError):
        pkg._capi.dtype_code(torch.int8)
    with pytest.raises(ValueError):
        pkg._capi.pooling_code("max")


def test_int8_tables_need_scales(pkg):
    c = pkg._capi
    rc = _forward(pkg, tables=_table(pkg, data=256), tdt=c.I8)
    assert rc == c.EINVAL and "row_scale" in c.last_error()


def test_fused_all_slots_int8_rejects_bad_arguments(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_fused_all_slots_int8
    #      values val_off row_off weight scale out odt     B  S   D    max_idx nnz stream
    assert f(256, 256, 256, 256, None, 256, c.BF16, 4, 28, 128, 10, 5, None) == c.EINVAL
    assert "scale" in c.last_error()
    assert f(256, 256, 256, 256, 256, 256, c.I8, 4, 28, 128, 10, 5, None) == c.EINVAL
    assert "output dtype" in c.last_error()
    assert f(256, 256, 256, 256, 256, 256, c.BF16, 4, 28, 0, 10, 5, None) == c.EINVAL
    assert f(256, 256, 256, 256, 256, 256, c.BF16, 4, 28, 128, 2 ** 31, 5, None) == c.EUNSUPPORTED
    assert f(None, None, None, None, None, None, c.BF16, 0, 28, 128, 10, 0, None) == c.OK
    # the float entry point does not take the int8 code
    assert c.lib().cti_ebag_fused_all_slots(256, 256, 256, 256, c.I8, 256, 4, 28, 128, 10, 5, None) == c.EINVAL


def test_fused_layernorm_rejects_bad_arguments(pkg):
    """Every case fails a host-side check, so nothing is launched (the pointers are not real)."""
    c = pkg._capi
    f = c.lib().cti_ebag_fused_all_slots_layernorm

    def call(**kw):
        a = dict(values=256, it=c.I64, vo=256, ro=256, ot=c.I64, weight=256, dt=c.BF16, out=256, B=4, S=28, D=128,
                 max_idx=10, nnz=5, pooling=c.SUM, gamma=256, beta=256, pdt=c.F32, eps=1e-5)
        a.update(kw)
        return f(a["values"], a["it"], a["vo"], a["ro"], a["ot"], a["weight"], a["dt"], a["out"], a["B"], a["S"],
                 a["D"], a["max_idx"], a["nnz"], a["pooling"], a["gamma"], a["beta"], a["pdt"], a["eps"], None)

    assert call(it=7) == c.EINVAL and "index type" in c.last_error()
    assert call(ot=7) == c.EINVAL and "offset type" in c.last_error()
    assert call(dt=9) == c.EINVAL
    assert call(pdt=9) == c.EINVAL and "parameter dtype" in c.last_error()
    assert call(pooling=5) == c.EINVAL
    assert call(B=-1) == c.EINVAL
    assert call(D=0) == c.EINVAL
    assert call(eps=-1.0) == c.EINVAL and call(eps=float("nan")) == c.EINVAL
    assert call(max_idx=2 ** 31) == c.EUNSUPPORTED
    assert call(gamma=None) == c.EINVAL and "NULL" in c.last_error()
    assert call(dt=c.F16) == c.EUNSUPPORTED and "fp16" in c.last_error()
    assert call(pdt=c.F16) == c.EUNSUPPORTED
    assert call(S=65) == c.EUNSUPPORTED and "slots" in c.last_error()
    assert call(D=8) == c.EUNSUPPORTED and "bytes" in c.last_error()  # 16-byte bf16 rows
    assert call(D=48) == c.EUNSUPPORTED  # 96-byte rows: not a power of two
    assert call(dt=c.F32, D=512) == c.EUNSUPPORTED and "2048 bytes" in c.last_error()
    assert call(weight=264) == c.EUNSUPPORTED and "aligned" in c.last_error()
    assert call(gamma=264) == c.EUNSUPPORTED
    assert call(values=None, vo=None, ro=None, weight=None, out=None, gamma=None, beta=None, B=0, nnz=0) == c.OK


def test_fused_layernorm_python_wrapper_validates_before_any_launch(pkg):
    z = torch.zeros(5, dtype=torch.int64)
    w = torch.zeros(10, 32)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.fused_all_slots_embedding_layernorm(z, torch.zeros(2, dtype=torch.int64), torch.zeros(8, dtype=torch.int64),
                                                w, torch.zeros(3, 64), 3, 32, 9, torch.ones(64), torch.zeros(64))


def test_layernorm_linear_rejects_bad_arguments(pkg):
    """Every case fails a host-side check, so nothing is launched (the pointers are not real)."""
    c = pkg._capi
    f = c.lib().cti_ebag_layernorm_linear

    def call(**kw):
        a = dict(x=256, rows=4, cols=3584, mean=512, rstd=768, gamma=1024, beta=1280, pdt=c.BF16, w=1536, n=512,
                 bias=2048, bdt=c.BF16, y=4096, ydt=c.BF16, ws=None, wsb=0)
        a.update(kw)
        return f(a["x"], a["rows"], a["cols"], a["mean"], a["rstd"], a["gamma"], a["beta"], a["pdt"], a["w"], a["n"],
                 a["bias"], a["bdt"], a["y"], a["ydt"], a["ws"], a["wsb"], None)

    assert call(rows=-1) == c.EINVAL
    assert call(cols=0) == c.EINVAL and call(n=0) == c.EINVAL
    assert call(cols=12) == c.EUNSUPPORTED and "multiple of 8" in c.last_error()
    assert call(rstd=None) == c.EINVAL and "together" in c.last_error()
    assert call(pdt=c.F16) == c.EINVAL and call(pdt=c.I8) == c.EINVAL
    assert call(bdt=c.F16) == c.EINVAL
    assert call(ydt=c.F16) == c.EINVAL
    assert call(x=None) == c.EINVAL and call(w=None) == c.EINVAL and call(y=None) == c.EINVAL
    assert call(x=264) == c.EINVAL and "aligned" in c.last_error()
    assert call(gamma=1032) == c.EINVAL
    assert call(rows=2 ** 40) == c.EUNSUPPORTED
    assert call(wsb=1024) == c.EINVAL and "workspace" in c.last_error()  # bytes without a workspace
    assert call(wsb=-1) == c.EINVAL
    assert call(ws=8200, wsb=1024) == c.EINVAL and "aligned" in c.last_error()
    # nothing to do: no launch, whatever the pointers
    assert call(rows=0, x=None, w=None, y=None) == c.OK


def test_layernorm_linear_workspace_query(pkg):
    """Split K only for the large form (K a multiple of 128) when its 128 x 128 tiles are fewer
    than one per CU: splits of an even number of 64-wide steps, at most half the steps."""
    q = pkg._capi.lib().cti_ebag_layernorm_linear_workspace_bytes
    # 32 x 4 tiles of 128 x 128 -> 2 splits of 28 steps
    assert q(4096, 3584, 512) == 2 * 4096 * 512 * 4
    # 8 x 4 tiles, 56 steps -> 8 wanted, 8 steps each (even) -> 7 splits
    assert q(1024, 3584, 512) == 7 * 1024 * 512 * 4
    # 1 x 4 tiles, 224 steps -> 64 wanted, 4 steps each -> 56 splits
    assert q(128, 14336, 512) == 56 * 128 * 512 * 4
    # 1 x 1 tile, 8 steps -> 256 wanted, 4 at most (two steps each)
    assert q(64, 512, 64) == 4 * 64 * 64 * 4
    # one tile of 128 x 128 per CU already (8192 rows): no split
    assert q(8192, 3584, 512) == 0
    # two or more tiles of 128 x 256 per CU: no split; K not a multiple of 128: the general form
    assert q(32768, 3584, 512) == 0 and q(300, 136, 512) == 0
    # too few steps to split (K = 128: two steps)
    assert q(8, 128, 64) == 0
    assert q(0, 3584, 512) == 0 and q(-1, 3584, 512) == 0


def test_layernorm_statistics_only_needs_both_outputs(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_layernorm
    #        x    y     rows cols dtype   gamma beta pdt    eps   mean rstd stream
    assert f(256, None, 4, 64, c.BF16, None, None, c.F32, 1e-5, 512, None, None) == c.EINVAL
    assert "statistics" in c.last_error()
    assert f(256, 256, 4, 64, c.BF16, None, 256, c.F32, 1e-5, None, None, None) == c.EINVAL


def test_layernorm_linear_python_wrapper_validates_before_any_launch(pkg):
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.zeros(32, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.layer_norm_linear(x, w)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.layer_norm_stats(x)


def test_quantize_int8_rejects_bad_arguments(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_quantize_int8
    #      weight dtype  rows dim stride q   scale stream
    assert f(256, c.I8, 10, 128, 128, 256, 256, None) == c.EINVAL
    assert f(256, c.BF16, -1, 128, 128, 256, 256, None) == c.EINVAL
    assert f(256, c.BF16, 10, 0, 0, 256, 256, None) == c.EINVAL
    assert f(256, c.BF16, 10, 128, 64, 256, 256, None) == c.EINVAL and "row_stride" in c.last_error()
    assert f(256, c.BF16, 10, 128, 128, None, 256, None) == c.EINVAL
    assert f(None, c.BF16, 0, 128, 128, None, None, None) == c.OK


def test_int8_python_wrappers_validate_before_any_launch(pkg):
    q = torch.zeros(10, 16, dtype=torch.int8)
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.quantize_embedding_int8(torch.zeros(10, 16))
    with pytest.raises(ValueError, match="GPU tensor"):
        pkg.embedding_bag_pooled(torch.zeros(3, dtype=torch.int64), torch.zeros(5, dtype=torch.int64),
                                 [(q, torch.ones(10))])
    with pytest.raises(ValueError, match="pair"):
        pkg.embedding_bag_pooled(torch.zeros(3, dtype=torch.int64), torch.zeros(5, dtype=torch.int64), [(q,)])


@pytest.mark.parametrize("n,threads", [(0, 1), (1, 4), (1000, 1), (200_003, 3), (1 << 20, 16)])
def test_narrow_ids_saturates(pkg, n, threads):
    """Host-side int64 -> int32 id compaction: saturating, so the device clamp sees the same row."""
    import numpy as np

    rng = np.random.default_rng(n)
    src = rng.integers(-(2 ** 40), 2 ** 40, n, dtype=np.int64)
    if n >= 8:
        src[:8] = [np.iinfo(np.int64).min, np.iinfo(np.int64).max, 2 ** 31, 2 ** 31 - 1, -(2 ** 31), -(2 ** 31) - 1, 0, -1]
    dst = np.full(n, 7, dtype=np.int32)
    rc = pkg._capi.lib().cti_ebag_narrow_ids(src.ctypes.data if n else None, n, dst.ctypes.data if n else None,
                                               threads)
    assert rc == pkg._capi.OK
    want = np.clip(src, -(2 ** 31), 2 ** 31 - 1).astype(np.int32)
    assert np.array_equal(dst, want)
    # the property the device relies on: clamping the narrowed id gives the int64 id's row
    for rows in (1, 5_000_000, 2 ** 31 - 1):
        assert np.array_equal(np.clip(dst.astype(np.int64), 0, rows - 1), np.clip(src, 0, rows - 1))


def test_narrow_ids_rejects_bad_arguments(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_narrow_ids
    assert f(None, 10, 64, 1) == c.EINVAL
    assert f(64, -1, 64, 1) == c.EINVAL
    assert f(64, 10, 64, 0) == c.EINVAL and "num_threads" in c.last_error()


def test_stage_offsets_layout(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_stage_offset
    counts = (ctypes.c_int64 * 3)(1000, 28 * 4097, 28)
    assert [f(counts, 3, c.I32, p) for p in range(4)] == [0, 4096, 4096 + 459008, 4096 + 459008 + 256]
    assert [f(counts, 3, c.I64, p) for p in range(4)] == [0, 8192, 8192 + 917760, 8192 + 917760 + 256]
    assert f(counts, 3, 9, 1) == -1 and f(counts, 3, c.I32, 4) == -1 and f(None, 3, c.I32, 1) == -1


def test_stage_copy_rejects_bad_arguments(pkg):
    c = pkg._capi
    f = c.lib().cti_ebag_stage_copy
    src = (ctypes.c_void_p * 2)(64, 64)
    st = (ctypes.c_int32 * 2)(c.I64, c.I64)
    cnt = (ctypes.c_int64 * 2)(10, 10)
    assert f(src, st, cnt, 9, c.I32, 64, 1 << 20, 64, 4, None) == c.EINVAL
    assert f(src, st, cnt, 2, 7, 64, 1 << 20, 64, 4, None) == c.EINVAL
    assert f(src, st, cnt, 2, c.I32, 64, 100, 64, 4, None) == c.EINVAL and "staging bytes" in c.last_error()
    assert f(src, st, cnt, 2, c.I32, None, 1 << 20, 64, 4, None) == c.EINVAL
    bad = (ctypes.c_int32 * 2)(c.I64, 5)
    assert f(src, bad, cnt, 2, c.I32, 64, 1 << 20, 64, 4, None) == c.EINVAL
    zero = (ctypes.c_int64 * 2)(0, 0)
    assert f(src, st, zero, 2, c.I32, None, 0, None, 4, None) == c.OK


def test_narrow_ids_in_a_forked_child(pkg):
    """The host pool is rebuilt in a forked child (DataLoader workers fork)."""
    import numpy as np

    lib = pkg._capi.lib()
    src = np.arange(-(1 << 19), 1 << 19, dtype=np.int64) * (1 << 20)
    dst = np.zeros(src.size, np.int32)
    assert lib.cti_ebag_narrow_ids(src.ctypes.data, src.size, dst.ctypes.data, 8) == 0
    pid = os.fork()
    if pid == 0:
        code = 1
        try:
            d2 = np.zeros(src.size, np.int32)
            ok = lib.cti_ebag_narrow_ids(src.ctypes.data, src.size, d2.ctypes.data, 8) == 0
            code = 0 if ok and np.array_equal(d2, np.clip(src, -(2 ** 31), 2 ** 31 - 1).astype(np.int32)) else 1
        finally:
            os._exit(code)
    _, status = os.waitpid(pid, 0)
    assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0


def _ref_offsets(rng, S, B, max_len):
    L = rng.integers(0, max_len + 1, size=(S, B))
    L[:, ::9] = rng.integers(60, 200, size=L[:, ::9].shape)
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    return ro


@pytest.mark.parametrize("dt,D,nb", [(torch.bfloat16, 128, 8), (torch.float32, 64, 8), (torch.bfloat16, 512, 2),
                                     (torch.float32, 1024, 2), (torch.bfloat16, 16, 64), (torch.int8, 128, 8)])
@pytest.mark.parametrize("S,B", [(28, 4096), (3, 777), (1, 5), (64, 100)])
def test_host_order_is_a_sorted_permutation(pkg, dt, D, nb, S, B):
    """cti_ebag_order_host (host code): header, every XCD range a permutation of itself, each chunk
    of 2048 tiles ordered by rows per bag (most first, capped at 63) and stable within a bucket,
    for int64 and int32 offsets alike."""
    rng = np.random.default_rng(S * 1000 + B)
    ro = _ref_offsets(rng, S, B, 30)
    a = pkg.make_tile_order(torch.from_numpy(ro.reshape(-1)), B, S, dt, D)
    b = pkg.make_tile_order(torch.from_numpy(ro.reshape(-1).astype(np.int32)), B, S, dt, D)
    o = a.numpy()
    tpf = (B + nb - 1) // nb
    n = S * tpf
    assert np.array_equal(o[:4 + n], b.numpy()[:4 + n])  # entries past the order are not written
    # the same bags in the global layout (offsets[f*B + b], one closing entry) give the same order
    base = np.concatenate([[0], np.cumsum(ro[:, -1])[:-1]])
    glob = np.concatenate([(ro[:, :-1] + base[:, None]).reshape(-1), [base[-1] + ro[-1, -1]]]).astype(np.int64)
    g = pkg.make_tile_order(torch.from_numpy(glob), B, S, dt, D)
    assert np.array_equal(o[:4 + n], g.numpy()[:4 + n])
    assert o[0] == n and o[1] == 0x4F524452 and o[2] == 0 and o[3] == 0
    perm = o[4:4 + n]
    q, r = n >> 3, n & 7
    for x in range(8):
        lo = x * (q + 1) if x < r else r * (q + 1) + (x - r) * q
        cnt = q + (1 if x < r else 0)
        seg = perm[lo:lo + cnt]
        assert np.array_equal(np.sort(seg), np.arange(lo, lo + cnt))
        for c0 in range(0, cnt, 2048):
            part = seg[c0:c0 + 2048]
            assert np.array_equal(np.sort(part), np.arange(lo + c0, lo + c0 + len(part)))
            fi = part // tpf
            b0 = (part - fi * tpf) * nb
            b1 = np.minimum(b0 + nb, B)
            per_bag = np.clip((ro[fi, b1] - ro[fi, b0]) // nb, 0, 63)
            assert (np.diff(per_bag) <= 0).all()
            same = np.diff(per_bag) == 0
            assert (np.diff(part)[same] > 0).all()  # stable: tile order inside a bucket


def test_host_order_rejections(pkg):
    c = pkg._capi
    lib = c.lib()
    ro = torch.zeros(3 * 11, dtype=torch.int64)
    buf = torch.zeros(64, dtype=torch.int32)
    call = lambda *a: lib.cti_ebag_order_host(*a)  # noqa: E731
    assert call(ro.data_ptr(), c.I64, 11, 10, 3, c.BF16, 128, buf.data_ptr(), 36, 1) == c.EINVAL  # 6 tiles need 40 B
    assert call(ro.data_ptr(), c.I64, 11, 10, 3, c.BF16, 128, buf.data_ptr(), 40, 1) == c.OK
    assert call(ro.data_ptr(), c.I64, 10, 10, 3, c.BF16, 128, buf.data_ptr(), 40, 1) == c.OK  # global offsets
    assert call(ro.data_ptr(), c.I64, 12, 10, 3, c.BF16, 128, buf.data_ptr(), 40, 1) == c.EINVAL  # stride
    assert call(ro.data_ptr(), c.I64, 11, 10, 3, c.BF16, 100, buf.data_ptr(), 1 << 20, 1) == c.EUNSUPPORTED  # generic
    assert call(ro.data_ptr(), 7, 11, 10, 3, c.BF16, 128, buf.data_ptr(), 1 << 20, 1) == c.EINVAL
    assert call(None, c.I64, 11, 10, 3, c.BF16, 128, buf.data_ptr(), 1 << 20, 1) == c.EINVAL
    assert call(ro.data_ptr(), c.I64, 1, 0, 3, c.BF16, 128, buf.data_ptr(), 1 << 20, 1) == c.EINVAL
    assert call(ro.data_ptr(), c.I64, 11, 10, 3, c.BF16, 128, buf.data_ptr(), 40, 0) == c.EINVAL  # threads
    big = torch.zeros(65 * 11, dtype=torch.int64)
    assert call(big.data_ptr(), c.I64, 11, 10, 65, c.BF16, 128, buf.data_ptr(), 1 << 20, 1) == c.EUNSUPPORTED
    with pytest.raises(ValueError):
        pkg.make_tile_order(torch.zeros(7, dtype=torch.int64), 10, 3, torch.bfloat16, 128)
