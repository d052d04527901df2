"""ORACLE — test infrastructure, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only to check results against (or as the timed CPU baseline). The product path never calls it.

CPU restatements of the fused sparse-feature embedding-bag path:
  pool / pool_c      the pooling step, in C (ebag_oracle.c, OpenMP over samples)
  pool_np            the same step in numpy, vectorised over bags but sequential in element order
  collate_layout     online_best/infer.py:446-474 (flat layout of a list of samples)
  prebuild_layout    online_best/infer.py:139-154 (flat layout from per-slot pairs)
  to_global_offsets  the closed-form conversion reference layout -> offsets[S*B+1]
  merge_layouts      online_best/infer.py:581-631 (per-slot concatenation of sub-batches)
  merge_pair_layouts online_best/infer.py:2977-3037 (same, with its int32 round trip)
  layer_norm_np      online_best/infer.py:829-858 (row LayerNorm of the pooled block, fp32)
  normalize_np       its output step for given per-row mean / rstd
  layer_norm_linear_np  online_best/infer.py:1061-1085 (the LayerNorm stored in bf16, then the
                     encoder's Linear in float64)
  quantize_int8_np / quantize_int8_c   online_best/infer.py:895-901 (int8 rows + fp32 scales)
  fma_np             fp32 fused multiply-add emulated exactly in float64 (round to odd)
  bf16 / fp16 encoders and decoders (IEEE round to nearest even)

Table arrays: float32 arrays for 'f32'; uint16 bit patterns for 'bf16' and 'f16'; for 'i8' a
pair (int8 [rows, dim], float32 scale [rows]) pooled as acc = fma(q, scale[row], acc)
(online_best/infer.py:904-942).
Pooling semantics (online_best/infer.py:805-827, baseline/infer.py:256-263): row index
clamp(v, 0, rows-1); fp32 accumulator starting at +0, rows added in element order; mean divides
the fp32 sum by the bag length; empty bag -> 0; one rounding to the output type.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_ebag.so")

DTYPES = {"f32": 0, "bf16": 1, "f16": 2, "i8": 3}


# ------------------------------------------------------------------------------------------------
# element encodings
# ------------------------------------------------------------------------------------------------
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact: the bf16 word is the high half of the fp32 word)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest, ties to even; NaN stays (quiet) NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, ((u >> 16) | np.uint32(0x40)).astype(np.uint16), rounded)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> fp16 bit patterns (numpy's cast rounds to nearest even)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def decode(arr: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return np.asarray(arr, dtype=np.float32)
    if dt == "bf16":
        return bf16_to_f32(arr)
    if dt == "f16":
        return f16_to_f32(arr)
    raise ValueError(dt)


def encode(x: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return np.asarray(x, dtype=np.float32)
    if dt == "bf16":
        return f32_to_bf16(x)
    if dt == "f16":
        return f32_to_f16(x)
    raise ValueError(dt)


# ------------------------------------------------------------------------------------------------
# pooling: numpy restatement
# ------------------------------------------------------------------------------------------------
def _bag_bounds(offsets, val_base, stride, f, batch, nnz):
    o = np.asarray(offsets, dtype=np.int64)
    base = 0 if val_base is None else int(val_base[f])
    s = o[f * stride: f * stride + batch] + base
    e = o[f * stride + 1: f * stride + batch + 1] + base
    s = np.clip(s, 0, nnz)
    e = np.clip(e, s, nnz)
    return s, e


def _rows_of(tab):
    """The row array of a table ('i8' tables are (q, scale) pairs)."""
    return tab[0] if isinstance(tab, tuple) else tab


def fma_np(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """fp32 fma(a, b, c) = RN32(a*b + c) with one rounding, for finite inputs.

    a*b is exact in float64 (24 + 24 bits). The sum a*b + c is formed in float64 rounded to odd
    (TwoSum gives the rounding error; a non-zero error with an even last bit moves the sum one
    float64 step towards the exact value), and rounding that to fp32 is the correctly rounded
    result since 53 >= 24 + 2 (Boldo & Melquiond, "Emulation of FMA and correctly rounded sums:
    proved algorithms using rounding to odd", IEEE Trans. Computers 57(4), 2008).
    """
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64
    p, c64 = np.broadcast_arrays(p, c64)
    ssum = p + c64
    bb = ssum - p
    err = (p - (ssum - bb)) + (c64 - bb)
    even = (ssum.view(np.uint64) & np.uint64(1)) == 0
    bump = (err != 0) & even
    towards = np.where(err > 0, np.inf, -np.inf)
    ro = np.where(bump, np.nextafter(ssum, towards), ssum)
    return ro.astype(np.float32)


def quantize_int8_np(w: np.ndarray):
    """online_best/infer.py:895-901 as torch evaluates it on the device, in fp32.

    w: float32 [rows, dim] (decoded table). row_max = max |w| (:897); scale = row_max / 127.0,
    which torch's device kernel computes as row_max * RN32(1/127) (a Python-scalar divisor is
    turned into a multiply by its fp32 reciprocal) (:898); clamp(min=1e-8) (:899);
    q = round_half_even(w / scale), IEEE fp32 division, clamp to [-128, 127], int8 (:900).
    Returns (q int8 [rows, dim], scale float32 [rows]).
    """
    w = np.asarray(w, np.float32)
    m = np.abs(w).max(axis=1) if w.shape[1] else np.zeros(w.shape[0], np.float32)
    inv127 = np.float32(1.0) / np.float32(127.0)
    scale = np.maximum((m * inv127).astype(np.float32), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint((w / scale[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    return q, scale


def pool_np(values: np.ndarray, offsets: np.ndarray, tables: Sequence[np.ndarray], table_dtype: str,
            pooling: str = "sum", out_dtype: Optional[str] = None, batch: Optional[int] = None,
            val_base: Optional[np.ndarray] = None, out_cols: Optional[Sequence[int]] = None,
            out_width: Optional[int] = None) -> np.ndarray:
    """Pool F fields into [B, width] (encoded in out_dtype).

    Global layout: offsets[F*B+1], val_base None. Reference layout: offsets = row_offsets
    [F*(B+1)] and val_base = val_offsets (then ``batch`` must be given).
    """
    out_dtype = out_dtype or table_dtype
    F = len(tables)
    values = np.asarray(values).astype(np.int64)
    nnz = values.shape[0]
    if val_base is None:
        batch = (len(offsets) - 1) // F if batch is None else batch
        stride = batch
    else:
        stride = batch + 1
    dims = [_rows_of(t).shape[1] for t in tables]
    cols = list(np.cumsum([0] + dims[:-1])) if out_cols is None else list(out_cols)
    width = sum(dims) if out_width is None else out_width
    out = np.zeros((batch, width), dtype=np.float32)
    for f, tab in enumerate(tables):
        rows_f = _rows_of(tab).shape[0]
        s, e = _bag_bounds(offsets, val_base, stride, f, batch, nnz)
        L = e - s
        acc = np.zeros((batch, dims[f]), dtype=np.float32)
        maxL = int(L.max()) if batch else 0
        for k in range(maxL):
            m = L > k
            rows = np.clip(values[s[m] + k], 0, rows_f - 1)
            if table_dtype == "i8":
                q, sc = tab
                acc[m] = fma_np(q[rows].astype(np.float32), np.asarray(sc, np.float32)[rows][:, None], acc[m])
            else:
                acc[m] = acc[m] + decode(tab[rows], table_dtype)
        if pooling == "mean":
            nz = L > 0
            acc[nz] = acc[nz] / L[nz].astype(np.float32)[:, None]
        out[:, cols[f]: cols[f] + dims[f]] = acc
    return encode(out, out_dtype)


# ------------------------------------------------------------------------------------------------
# pooling: C restatement
# ------------------------------------------------------------------------------------------------
class _Table(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("rows", ctypes.c_int64), ("row_stride", ctypes.c_int64),
                ("dim", ctypes.c_int32), ("out_col", ctypes.c_int32), ("row_scale", ctypes.c_void_p)]


_clib = None


def build_c(force: bool = False) -> str:
    """Compile ebag_oracle.c into liboracle_ebag.so (gcc, -ffp-contract=off, OpenMP)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


def clib() -> ctypes.CDLL:
    global _clib
    if _clib is None:
        build_c()
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_pool.restype = ctypes.c_int
        lib.oracle_pool.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(_Table),
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                    ctypes.c_void_p]
        for n in ("oracle_f32_to_bf16_array", "oracle_f32_to_f16_array", "oracle_f16_to_f32_array"):
            getattr(lib, n).restype = None
            getattr(lib, n).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_quantize_int8.restype = ctypes.c_int
        lib.oracle_quantize_int8.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_fmaf_array.restype = None
        lib.oracle_fmaf_array.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64]
        lib.oracle_num_threads.restype = ctypes.c_int
        lib.oracle_set_num_threads.argtypes = [ctypes.c_int]
        _clib = lib
    return _clib


def pool_c(values: np.ndarray, offsets: np.ndarray, tables: Sequence[np.ndarray], table_dtype: str,
           pooling: str = "sum", out_dtype: Optional[str] = None, batch: Optional[int] = None,
           val_base: Optional[np.ndarray] = None, out_cols: Optional[Sequence[int]] = None,
           out_width: Optional[int] = None, table_rows: Optional[Sequence[int]] = None) -> np.ndarray:
    """Same contract as pool_np, computed by the C restatement.

    ``table_rows`` overrides the clamp bound of each field (default: the array's row count);
    callers that pass a compacted table of touched rows use it to keep the original bound.
    """
    out_dtype = out_dtype or table_dtype
    F = len(tables)
    values = np.ascontiguousarray(values)
    idx32 = values.dtype == np.int32
    if not idx32:
        values = np.ascontiguousarray(values, dtype=np.int64)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    if val_base is None:
        batch = (len(offsets) - 1) // F if batch is None else batch
        stride = batch
        vb = None
    else:
        stride = batch + 1
        vb = np.ascontiguousarray(val_base, dtype=np.int64)
    dims = [_rows_of(t).shape[1] for t in tables]
    cols = list(np.cumsum([0] + dims[:-1])) if out_cols is None else list(out_cols)
    width = sum(dims) if out_width is None else out_width
    descs = (_Table * F)()
    keep = []
    for f, t in enumerate(tables):
        if table_dtype == "i8":
            sc = np.ascontiguousarray(t[1], dtype=np.float32)
            t = np.ascontiguousarray(t[0], dtype=np.int8)
            keep.append(sc)
            descs[f].row_scale = sc.ctypes.data
        else:
            t = np.ascontiguousarray(t)
        keep.append(t)
        descs[f].data = t.ctypes.data
        descs[f].rows = t.shape[0] if table_rows is None else int(table_rows[f])
        descs[f].row_stride = t.shape[1]
        descs[f].dim = t.shape[1]
        descs[f].out_col = int(cols[f])
    out = np.zeros((batch, width), dtype=np.float32 if out_dtype == "f32" else np.uint16)
    rc = clib().oracle_pool(values.ctypes.data if values.size else None, int(idx32), values.shape[0],
                            offsets.ctypes.data, vb.ctypes.data if vb is not None else None, stride, batch, F,
                            descs, DTYPES[table_dtype], int(pooling == "mean"), out.ctypes.data,
                            DTYPES[out_dtype], width, None)
    if rc != 0:
        raise ValueError("oracle_pool rejected its arguments")
    return out


pool = pool_c


def quantize_int8_c(table: np.ndarray, table_dtype: str = "f32"):
    """The C restatement of quantize_int8_np; ``table`` in the encoding of ``table_dtype``."""
    table = np.ascontiguousarray(table)
    rows, dim = table.shape
    q = np.empty((rows, dim), dtype=np.int8)
    scale = np.empty(rows, dtype=np.float32)
    rc = clib().oracle_quantize_int8(table.ctypes.data, DTYPES[table_dtype], rows, dim, dim, q.ctypes.data,
                                     scale.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_quantize_int8 rejected its arguments")
    return q, scale


def c_fmaf(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """C99 fmaf elementwise (the operation the C oracle pools int8 tables with)."""
    a, b, c = (np.ascontiguousarray(np.broadcast_to(x, np.broadcast_shapes(np.shape(a), np.shape(b), np.shape(c))),
                                    dtype=np.float32) for x in (a, b, c))
    y = np.empty(a.shape, dtype=np.float32)
    clib().oracle_fmaf_array(a.ctypes.data, b.ctypes.data, c.ctypes.data, y.ctypes.data, a.size)
    return y


def c_f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    clib().oracle_f32_to_bf16_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def c_f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    clib().oracle_f32_to_f16_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def c_f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    y = np.empty(bits.shape, dtype=np.float32)
    clib().oracle_f16_to_f32_array(bits.ctypes.data, y.ctypes.data, bits.size)
    return y


# ------------------------------------------------------------------------------------------------
# layout restatements (integer, exact)
# ------------------------------------------------------------------------------------------------
def collate_layout(feasigns: Sequence[Dict[int, Sequence[int]]], max_slot_id: int):
    """online_best/infer.py:446-474: (flat_values, flat_row_offsets, val_offsets, per-slot pairs)."""
    slots = []
    for slot in range(1, max_slot_id + 1):
        vals: List[int] = []
        offs = [0]
        for fs in feasigns:
            if slot in fs:
                vals.extend(int(v) for v in fs[slot])
            offs.append(len(vals))
        slots.append((np.array(vals, dtype=np.int64), np.array(offs, dtype=np.int64)))
    return prebuild_layout(slots) + (slots,)


def prebuild_layout(slots: Sequence[Tuple[np.ndarray, np.ndarray]]):
    """online_best/infer.py:139-154: concatenate per-slot pairs; val_offsets = exclusive prefix."""
    lens = [0]
    for v, _ in slots:
        lens.append(lens[-1] + len(v))
    flat_values = np.concatenate([np.asarray(v, dtype=np.int64) for v, _ in slots]) if slots else np.zeros(0, np.int64)
    flat_row_offsets = np.concatenate([np.asarray(o, dtype=np.int64) for _, o in slots]) if slots else np.zeros(0, np.int64)
    return flat_values, flat_row_offsets, np.array(lens[:-1], dtype=np.int64)


def to_global_offsets(val_offsets: np.ndarray, row_offsets: np.ndarray, batch: int, nnz: int) -> np.ndarray:
    """offsets[s*B+b] = val_offsets[s] + row_offsets[s*(B+1)+b]; offsets[S*B] = nnz."""
    S = len(val_offsets)
    ro = np.asarray(row_offsets, dtype=np.int64).reshape(S, batch + 1)
    g = (ro[:, :batch] + np.asarray(val_offsets, dtype=np.int64)[:, None]).reshape(-1)
    return np.concatenate([g, np.array([nnz], dtype=np.int64)])


def slot_slices(flat_values, flat_row_offsets, val_offsets, slot_num):
    """Per-slot (values, local offsets) of a flat layout (online_best/infer.py:604-607)."""
    B = len(flat_row_offsets) // slot_num - 1
    out = []
    for s in range(slot_num):
        start = int(val_offsets[s])
        end = int(val_offsets[s + 1]) if s + 1 < slot_num else len(flat_values)
        out.append((np.asarray(flat_values[start:end], dtype=np.int64),
                    np.asarray(flat_row_offsets[s * (B + 1):(s + 1) * (B + 1)], dtype=np.int64)))
    return out


def merge_layouts(layouts: Sequence[Tuple[np.ndarray, np.ndarray, np.ndarray]], slot_num: int):
    """online_best/infer.py:581-631: per slot, concatenate the sub-batches' value slices and their
    local offsets (without the closing entry) shifted by the slot's running value count, then
    close with the slot total; val_offsets = exclusive prefix of slot totals."""
    vparts, oparts, vo = [], [], [0]
    per = [slot_slices(*lay, slot_num) for lay in layouts]
    for s in range(slot_num):
        sv, so = [], []
        base = 0
        for k in range(len(layouts)):
            v, o = per[k][s]
            sv.append(v)
            so.append(o[:-1] + base)
            base += len(v)
        vparts.append(np.concatenate(sv))
        oparts.append(np.concatenate(so + [np.array([base], dtype=np.int64)]))
        vo.append(vo[-1] + base)
    return np.concatenate(vparts), np.concatenate(oparts), np.array(vo[:-1], dtype=np.int64)


def merge_pair_layouts(layouts, slot_num: int):
    """online_best/infer.py:2977-3037: as merge_layouts, but values and offsets pass through
    int32 (.int() then .long(), :3008-3009 and :3019-3020), so ids >= 2**31 wrap."""
    v, o, vo = merge_layouts(layouts, slot_num)
    return v.astype(np.int32).astype(np.int64), o.astype(np.int32).astype(np.int64), vo


# ------------------------------------------------------------------------------------------------
# input LayerNorm of the pooled block
# ------------------------------------------------------------------------------------------------
def layer_norm_np(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float):
    """Row LayerNorm, online_best/infer.py:829-858, in fp32.

    x: float32 [rows, cols] (the pooled block decoded to fp32, :843); gamma, beta: float32 [cols].
    mean = sum(x)/cols (:845); var = sum((x - mean)^2)/cols, two passes (:846-848);
    rstd = 1/sqrt(var + eps) (:849); y = (x - mean) * rstd * gamma + beta (:856), each operation
    rounded to fp32. The sums are taken in float64 and rounded once (the reference's reduction
    order is not observable; the HIP kernel's is fixed), so comparisons use a tolerance.
    Returns (y float32 [rows, cols], mean float32 [rows], rstd float32 [rows]).
    """
    x = np.asarray(x, np.float32)
    n = np.float32(x.shape[1])
    mean = (x.astype(np.float64).sum(axis=1).astype(np.float32) / n).astype(np.float32)
    d = (x - mean[:, None]).astype(np.float32)
    var = ((d.astype(np.float64) ** 2).sum(axis=1).astype(np.float32) / n).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return normalize_np(x, mean, rstd, gamma, beta), mean, rstd


def normalize_np(x: np.ndarray, mean: np.ndarray, rstd: np.ndarray, gamma: np.ndarray, beta: np.ndarray):
    """The LayerNorm's output step, online_best/infer.py:855-856, for given per-row mean and rstd:
    y = ((x - mean) * rstd) * gamma + beta, each operation rounded to fp32 (no fused multiply-add).
    x float32 [rows, cols]; mean, rstd float32 [rows]; gamma, beta float32 [cols]."""
    x = np.asarray(x, np.float32)
    d = (x - np.asarray(mean, np.float32)[:, None]).astype(np.float32)
    y = ((d * np.asarray(rstd, np.float32)[:, None]).astype(np.float32) * np.asarray(gamma, np.float32))
    return (y.astype(np.float32) + np.asarray(beta, np.float32)).astype(np.float32)


def layer_norm_linear_np(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float, weight: np.ndarray,
                         bias: Optional[np.ndarray], mean: Optional[np.ndarray] = None,
                         rstd: Optional[np.ndarray] = None):
    """online_best/infer.py:1061-1085: the input LayerNorm writes its output into a tensor like
    the pooled block (bf16 in the reference's model, :1063), and ``self.linear`` maps it to
    d_model (:1085) with fp32 accumulation and one rounding of the result.

    x float32 [rows, cols] (the bf16 pooled block, decoded); gamma, beta float32 [cols];
    weight float32 [n, cols] (bf16 values, decoded; nn.Linear's layout); bias float32 [n] or
    None. mean / rstd: the statistics to normalise with (default: layer_norm_np's).
    Returns (y, a, absum): y float64 [rows, n] = a @ weight.T + bias summed in float64 (the
    accumulation order of the reference's GEMM is not observable: comparisons use a bound),
    a float32 [rows, cols] the normalised rows rounded to bf16, absum float64 [rows, n] =
    |a| @ |weight|.T (for the fp32 accumulation bound).
    """
    if mean is None or rstd is None:
        y, mean, rstd = layer_norm_np(x, gamma, beta, eps)
    else:
        y = normalize_np(x, mean, rstd, gamma, beta)
    a = decode(encode(y, "bf16"), "bf16")
    w = np.asarray(weight, np.float64)
    out = a.astype(np.float64) @ w.T
    if bias is not None:
        out = out + np.asarray(bias, np.float64)[None, :]
    absum = np.abs(a).astype(np.float64) @ np.abs(w).T
    return out, a, absum
