"""Host entry points of the fused sparse-feature embedding-bag path.

``fused_all_slots_embedding`` is the drop-in for the reference launch
``fused_all_slots_embedding_kernel[(B, 28)](values, val_offsets, row_offsets, weight, out,
batch_size, emb_dim, max_idx, BLOCK_SIZE)`` (online_best/infer.py:793-827, launched at
online_best/infer.py:1052-1059): same arguments in the same order (grid and BLOCK_SIZE are
chosen inside), same layout, same results, launched on torch's current stream.

``embedding_bag_pooled`` is the general form: per-field tables (possibly of different widths),
global offsets ``offsets[F*B+1]``, sum or mean pooling, and an explicit output dtype.

``quantize_embedding_int8`` and ``fused_all_slots_embedding_int8`` are the int8 row-quantised
pair (online_best/infer.py:895-942). A table argument of the general entry points may also be an
int8 pair ``(q [V, D] int8, scale [V] float32)``; its rows pool as ``acc = fma(q, scale, acc)``.

Both validate their arguments on the host (no device synchronisation) and raise ``ValueError``
/ ``TypeError`` for malformed calls and ``EbagError`` when the C ABI reports a failure.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

from . import _capi


def _require_device_tensor(name: str, t: torch.Tensor, device: Optional[torch.device] = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _require_contiguous(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _split_table(i: int, t):
    """(rows tensor, scale tensor or None) of one table argument: a tensor or an int8 pair."""
    if isinstance(t, (tuple, list)):
        if len(t) != 2:
            raise ValueError(f"tables[{i}]: an int8 table is a pair (q, scale)")
        q, scale = t
        _require_device_tensor(f"tables[{i}][0]", q)
        _require_device_tensor(f"tables[{i}][1]", scale, q.device)
        if q.dtype != torch.int8:
            raise TypeError(f"tables[{i}][0] must be int8 (got {q.dtype})")
        if scale.dtype != torch.float32 or not scale.is_contiguous() or scale.dim() != 1:
            raise TypeError(f"tables[{i}][1] must be a contiguous 1-D float32 tensor")
        if q.dim() == 2 and scale.numel() != q.shape[0]:
            raise ValueError(f"tables[{i}]: {scale.numel()} scales for {q.shape[0]} rows")
        return q, scale
    _require_device_tensor(f"tables[{i}]", t)
    return t, None


def _table_descs(tables):
    """Validate the table arguments; return (descs, device, dtype code, width, torch dtype)."""
    num_fields = len(tables)
    if num_fields == 0:
        raise ValueError("at least one table is required")
    parts = [_split_table(i, t) for i, t in enumerate(tables)]
    dev = parts[0][0].device
    tdt = parts[0][0].dtype
    quant = parts[0][1] is not None
    descs = (_capi.Table * num_fields)()
    col = 0
    for i, (t, scale) in enumerate(parts):
        _require_device_tensor(f"tables[{i}]", t, dev)
        if (scale is not None) != quant:
            raise TypeError("tables mix int8 pairs and plain tensors")
        if t.dim() != 2:
            raise ValueError(f"tables[{i}] must be 2-D, got shape {tuple(t.shape)}")
        if t.dtype != tdt:
            raise TypeError(f"tables[{i}] dtype {t.dtype} differs from tables[0] dtype {tdt}")
        if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
            raise ValueError(f"tables[{i}] must be row-major with unit column stride")
        if t.shape[0] < 1:
            raise ValueError(f"tables[{i}] has no rows")
        d = descs[i]
        d.data, d.rows, d.row_stride, d.dim, d.out_col = t.data_ptr(), t.shape[0], t.stride(0), t.shape[1], col
        d.row_scale = scale.data_ptr() if scale is not None else None
        col += int(t.shape[1])
    code = _capi.I8 if quant else _capi.dtype_code(tdt)
    return descs, dev, code, col, tdt


def quantize_embedding_int8(weight: torch.Tensor):
    """Row-quantise a GPU table to int8: ``(q [V, D] int8, scale [V] float32)``.

    Mirrors online_best/infer.py:895-901 as torch evaluates it on the device:
    ``scale = max(max_j |w_j| * fp32(1/127), 1e-8)`` (torch turns the division by the Python
    scalar 127.0 into a multiply by its fp32 reciprocal), ``q = clamp(round_half_even(w / scale),
    -128, 127)``, all in fp32; bit-identical to that expression for finite tables. ``weight`` is
    fp32 / bf16 / fp16 with unit column stride.
    """
    _require_device_tensor("weight", weight)
    if weight.dim() != 2 or weight.stride(1) != 1 or weight.stride(0) < weight.shape[1]:
        raise ValueError("weight must be a row-major 2-D tensor with unit column stride")
    rows, dim = weight.shape
    dev = weight.device
    q = torch.empty((rows, dim), dtype=torch.int8, device=dev)
    scale = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _capi.check(_capi.lib().cti_ebag_quantize_int8(
            weight.data_ptr(), _capi.dtype_code(weight.dtype), rows, dim, weight.stride(0), q.data_ptr(),
            scale.data_ptr(), _capi.current_stream_handle(dev)))
    return q, scale


def _check_flat_layout(flat_values, val_offsets, flat_row_offsets, out, dev):
    """Validate a flat-layout batch; return the (index, offset) type codes. Ids may be int64 or
    int32; val_offsets and flat_row_offsets share one type, int64 or int32."""
    for name, t in (("flat_values", flat_values), ("val_offsets", val_offsets),
                    ("flat_row_offsets", flat_row_offsets), ("out", out)):
        _require_device_tensor(name, t, dev)
        _require_contiguous(name, t)
    for name, t in (("flat_values", flat_values), ("val_offsets", val_offsets),
                    ("flat_row_offsets", flat_row_offsets)):
        if t.dtype not in (torch.int64, torch.int32):
            raise TypeError(f"{name} must be int64 or int32 (got {t.dtype})")
    return _capi.index_code(flat_values.dtype), _capi.index_code(flat_row_offsets.dtype)


def _same_offset_type(val_offsets: torch.Tensor, flat_row_offsets: torch.Tensor, nnz: int) -> torch.Tensor:
    """val_offsets in flat_row_offsets' dtype (the reference widens only val_offsets, :747)."""
    if val_offsets.dtype == flat_row_offsets.dtype:
        return val_offsets
    if flat_row_offsets.dtype == torch.int32 and nnz >= 2 ** 31:
        raise ValueError("int32 row offsets cannot address a batch of 2^31 or more ids")
    return val_offsets.to(flat_row_offsets.dtype)


def fused_all_slots_embedding_int8(
    flat_values: torch.Tensor,
    val_offsets: torch.Tensor,
    flat_row_offsets: torch.Tensor,
    weight_int8: torch.Tensor,
    scale: torch.Tensor,
    out: torch.Tensor,
    batch_size: int,
    emb_dim: int,
    max_idx: int,
) -> torch.Tensor:
    """int8 drop-in for ``fused_all_slots_embedding_kernel_int8[(B, S)](values, val_offsets,
    row_offsets, weight_int8, scale, out, batch_size, emb_dim, max_idx, BLOCK_SIZE)``
    (online_best/infer.py:904-942, launched at online_best/infer.py:991-996).

    ``weight_int8`` int8 [V, emb_dim] and ``scale`` float32 [V] as made by
    ``quantize_embedding_int8``; each bag accumulates ``fma(q, scale[row], acc)`` in fp32 in
    element order; the sum is rounded to bf16, as the reference kernel stores ``acc.to(bfloat16)``
    (:941), and written into ``out`` [B, S*emb_dim] in out's dtype (fp32 / bf16 / fp16; the
    reference's ``out`` has the table's dtype, :989). Returns ``out``.
    """
    dev = weight_int8.device
    _require_device_tensor("weight_int8", weight_int8)
    icode, ocode = _check_flat_layout(flat_values, val_offsets, flat_row_offsets, out, dev)
    val_offsets = _same_offset_type(val_offsets, flat_row_offsets, flat_values.numel())
    _require_device_tensor("scale", scale, dev)
    _require_contiguous("weight_int8", weight_int8)
    _require_contiguous("scale", scale)
    if weight_int8.dtype != torch.int8 or weight_int8.dim() != 2:
        raise TypeError(f"weight_int8 must be a 2-D int8 tensor (got {weight_int8.dtype}, {weight_int8.dim()}-D)")
    if scale.dtype != torch.float32 or scale.numel() != weight_int8.shape[0]:
        raise TypeError(f"scale must be float32 with {weight_int8.shape[0]} elements")
    batch_size, emb_dim, max_idx = int(batch_size), int(emb_dim), int(max_idx)
    num_slots = val_offsets.numel()
    if weight_int8.shape[1] != emb_dim:
        raise ValueError(f"weight_int8 has {weight_int8.shape[1]} columns, emb_dim is {emb_dim}")
    if not 0 <= max_idx < weight_int8.shape[0]:
        raise ValueError(f"max_idx {max_idx} outside [0, {weight_int8.shape[0] - 1}]")
    if batch_size < 0:
        raise ValueError(f"batch_size must be >= 0, got {batch_size}")
    if flat_row_offsets.numel() != num_slots * (batch_size + 1):
        raise ValueError(f"flat_row_offsets has {flat_row_offsets.numel()} entries, expected "
                         f"{num_slots} * ({batch_size} + 1)")
    if out.numel() != batch_size * num_slots * emb_dim or (out.dim() >= 1 and out.shape[0] != batch_size):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected ({batch_size}, {num_slots * emb_dim})")
    with torch.cuda.device(dev):
        stream = _capi.current_stream_handle(dev)
        if icode == _capi.I64 and ocode == _capi.I64:
            _capi.check(_capi.lib().cti_ebag_fused_all_slots_int8(
                flat_values.data_ptr(), val_offsets.data_ptr(), flat_row_offsets.data_ptr(), weight_int8.data_ptr(),
                scale.data_ptr(), out.data_ptr(), _capi.dtype_code(out.dtype), batch_size, num_slots, emb_dim,
                max_idx, flat_values.numel(), stream))
        else:
            _capi.check(_capi.lib().cti_ebag_fused_all_slots_typed(
                flat_values.data_ptr(), icode, val_offsets.data_ptr(), flat_row_offsets.data_ptr(), ocode,
                weight_int8.data_ptr(), _capi.I8, scale.data_ptr(), out.data_ptr(), _capi.dtype_code(out.dtype),
                batch_size, num_slots, emb_dim, max_idx, flat_values.numel(), stream))
    return out


def order_bytes(batch_size: int, num_slots: int) -> int:
    """Bytes of a dispatch order for any launch of ``batch_size`` samples and ``num_slots`` slots."""
    n = _capi.lib().cti_ebag_order_bytes(int(batch_size), int(num_slots))
    if n < 0:
        raise ValueError("batch_size and num_slots must be >= 0")
    return n


def make_tile_order(offsets: torch.Tensor, batch_size: int, num_slots: int, table_dtype: torch.dtype,
                    emb_dim: int, out: Optional[torch.Tensor] = None, threads: int = 0) -> torch.Tensor:
    """The dispatch order of the launch for this batch, made on the host from its offsets (a CPU
    int64 / int32 tensor): the reference layout's row offsets ``[num_slots*(B+1)]`` or the global
    offsets ``[num_slots*B+1]`` of ``embedding_bag_pooled`` / ``PooledEmbedding``. Each XCD's
    tiles are listed most rows per bag first. ``table_dtype`` / ``emb_dim`` are the rows' (one
    width for all slots; int8 tables: ``torch.int8``). Returns a CPU int32 tensor (``out`` if
    given, of at least ``order_bytes(B, S)`` bytes) to be moved to the device with the batch and
    passed as ``tile_order``. ``threads``: host threads (0: up to 16, within this host's CPUs).
    No counterpart in the reference."""
    if offsets.device.type != "cpu" or offsets.dtype not in (torch.int64, torch.int32):
        raise ValueError("offsets must be an int64 or int32 CPU tensor")
    offsets = offsets.contiguous()
    batch_size, num_slots = int(batch_size), int(num_slots)
    if offsets.numel() == num_slots * (batch_size + 1):
        stride = batch_size + 1
    elif offsets.numel() == num_slots * batch_size + 1:
        stride = batch_size
    else:
        raise ValueError(f"offsets has {offsets.numel()} entries, expected {num_slots} * ({batch_size} + 1) (slot "
                         f"row offsets) or {num_slots} * {batch_size} + 1 (global offsets)")
    nbytes = order_bytes(batch_size, num_slots)
    if out is None:
        out = torch.empty((nbytes + 3) // 4, dtype=torch.int32)
    elif out.device.type != "cpu" or out.dtype != torch.int32 or not out.is_contiguous() or out.numel() * 4 < nbytes:
        raise ValueError(f"out must be a contiguous CPU int32 tensor of at least {nbytes} bytes")
    tcode = _capi.I8 if table_dtype == torch.int8 else _capi.dtype_code(table_dtype)
    _capi.check(_capi.lib().cti_ebag_order_host(offsets.data_ptr(), _capi.index_code(offsets.dtype), stride,
                                                batch_size, num_slots, tcode, int(emb_dim), out.data_ptr(),
                                                out.numel() * 4, int(threads) or _host_threads()))
    return out


def _host_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def fused_all_slots_embedding(
    flat_values: torch.Tensor,
    val_offsets: torch.Tensor,
    flat_row_offsets: torch.Tensor,
    weight: torch.Tensor,
    out: torch.Tensor,
    batch_size: int,
    emb_dim: int,
    max_idx: int,
    tile_order: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Pool every slot of a flat-layout batch into ``out[B, S*emb_dim]`` (sum, fp32 accumulate).

    Arguments mirror online_best/infer.py:794-804:
      flat_values       int64 [nnz]        field-major sign ids (online_best/infer.py:471)
      val_offsets       int64 [S]          slot starts in flat_values (online_best/infer.py:473)
      flat_row_offsets  int64 [S*(B+1)]    per-slot local offsets (online_best/infer.py:472)
      (ids and offsets may also be int32, as the Triton kernel specialises on its pointer dtypes;
      the int32 forms give the same result bit for bit)
      weight            [V, emb_dim]       shared table (fp32 / bf16 / fp16), contiguous
      out               [B, S*emb_dim]     caller-allocated, weight's dtype (online_best/infer.py:1050)
      batch_size        B
      emb_dim           D
      max_idx           clamp bound, V-1 in the reference (online_best/infer.py:1057)
      tile_order        optional device int32 dispatch order of this batch (``make_tile_order``,
                        moved with the batch; no counterpart in the reference): the launch starts
                        each XCD's tiles with the most rows per bag, which shortens its drain. The
                        result is the same bit for bit with or without it.
    Returns ``out``.
    """
    dev = weight.device
    _require_device_tensor("weight", weight)
    icode, ocode = _check_flat_layout(flat_values, val_offsets, flat_row_offsets, out, dev)
    val_offsets = _same_offset_type(val_offsets, flat_row_offsets, flat_values.numel())
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [V, D], got shape {tuple(weight.shape)}")
    _require_contiguous("weight", weight)
    batch_size = int(batch_size)
    emb_dim = int(emb_dim)
    max_idx = int(max_idx)
    num_slots = val_offsets.numel()
    if weight.shape[1] != emb_dim:
        raise ValueError(f"weight has {weight.shape[1]} columns, emb_dim is {emb_dim}")
    if not 0 <= max_idx < weight.shape[0]:
        raise ValueError(f"max_idx {max_idx} outside [0, {weight.shape[0] - 1}]")
    if batch_size < 0:
        raise ValueError(f"batch_size must be >= 0, got {batch_size}")
    if flat_row_offsets.numel() != num_slots * (batch_size + 1):
        raise ValueError(
            f"flat_row_offsets has {flat_row_offsets.numel()} entries, expected "
            f"{num_slots} * ({batch_size} + 1)"
        )
    if out.dtype != weight.dtype:
        raise TypeError(f"out dtype {out.dtype} differs from weight dtype {weight.dtype}")
    if out.numel() != batch_size * num_slots * emb_dim or (out.dim() >= 1 and out.shape[0] != batch_size):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected ({batch_size}, {num_slots * emb_dim})")
    lib = _capi.lib()
    with torch.cuda.device(dev):
        stream = _capi.current_stream_handle(dev)
        if tile_order is not None:
            _require_device_tensor("tile_order", tile_order, dev)
            _require_contiguous("tile_order", tile_order)
            if tile_order.dtype != torch.int32:
                raise TypeError(f"tile_order must be int32 (got {tile_order.dtype})")
            code = _capi.dtype_code(weight.dtype)
            _capi.check(lib.cti_ebag_fused_all_slots_ordered(
                flat_values.data_ptr(), icode, val_offsets.data_ptr(), flat_row_offsets.data_ptr(), ocode,
                weight.data_ptr(), code, None, out.data_ptr(), code, batch_size, num_slots, emb_dim, max_idx,
                flat_values.numel(), tile_order.data_ptr(), tile_order.numel() * 4, stream))
        elif icode == _capi.I64 and ocode == _capi.I64:
            _capi.check(lib.cti_ebag_fused_all_slots(
                flat_values.data_ptr(), val_offsets.data_ptr(), flat_row_offsets.data_ptr(),
                weight.data_ptr(), _capi.dtype_code(weight.dtype), out.data_ptr(),
                batch_size, num_slots, emb_dim, max_idx, flat_values.numel(), stream))
        else:
            code = _capi.dtype_code(weight.dtype)
            _capi.check(lib.cti_ebag_fused_all_slots_typed(
                flat_values.data_ptr(), icode, val_offsets.data_ptr(), flat_row_offsets.data_ptr(), ocode,
                weight.data_ptr(), code, None, out.data_ptr(), code, batch_size, num_slots, emb_dim, max_idx,
                flat_values.numel(), stream))
    return out


def fused_all_slots_embedding_layernorm(
    flat_values: torch.Tensor,
    val_offsets: torch.Tensor,
    flat_row_offsets: torch.Tensor,
    weight: torch.Tensor,
    out: torch.Tensor,
    batch_size: int,
    emb_dim: int,
    max_idx: int,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    eps: float = 1e-5,
    pooling: str = "sum",
) -> torch.Tensor:
    """The fused embedding step followed by the input LayerNorm (online_best/infer.py:1050-1076):
    ``out[B, S*emb_dim] = LayerNorm(pool)``, pool as ``fused_all_slots_embedding`` writes it
    (``pooling='sum'`` as the reference; 'mean' also accepted), the LayerNorm with fp32 statistics
    over each row and ``ln_weight`` / ``ln_bias`` of ``S*emb_dim`` elements.

    One kernel keeps each pooled row on chip and writes only the normalised row. Shapes the fused
    kernel does not cover (see ``cti_ebag_fused_all_slots_layernorm``) run the pooling kernel and
    the LayerNorm kernel one after the other (same result within the LayerNorm's fp32 rounding).
    Returns ``out``.
    """
    dev = weight.device
    _require_device_tensor("weight", weight)
    icode, ocode = _check_flat_layout(flat_values, val_offsets, flat_row_offsets, out, dev)
    val_offsets = _same_offset_type(val_offsets, flat_row_offsets, flat_values.numel())
    if weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous 2-D tensor")
    batch_size, emb_dim, max_idx = int(batch_size), int(emb_dim), int(max_idx)
    num_slots = val_offsets.numel()
    if weight.shape[1] != emb_dim:
        raise ValueError(f"weight has {weight.shape[1]} columns, emb_dim is {emb_dim}")
    if not 0 <= max_idx < weight.shape[0]:
        raise ValueError(f"max_idx {max_idx} outside [0, {weight.shape[0] - 1}]")
    if flat_row_offsets.numel() != num_slots * (batch_size + 1):
        raise ValueError(f"flat_row_offsets has {flat_row_offsets.numel()} entries, expected "
                         f"{num_slots} * ({batch_size} + 1)")
    if out.dtype != weight.dtype or tuple(out.shape) != (batch_size, num_slots * emb_dim):
        raise ValueError(f"out must be ({batch_size}, {num_slots * emb_dim}) {weight.dtype}")
    width = num_slots * emb_dim
    for name, t in (("ln_weight", ln_weight), ("ln_bias", ln_bias)):
        _require_device_tensor(name, t, dev)
        _require_contiguous(name, t)
        if t.numel() != width:
            raise ValueError(f"{name} has {t.numel()} elements, expected {width}")
    if ln_weight.dtype != ln_bias.dtype:
        raise TypeError("ln_weight and ln_bias dtypes differ")
    lib = _capi.lib()
    with torch.cuda.device(dev):
        rc = lib.cti_ebag_fused_all_slots_layernorm(
            flat_values.data_ptr(), icode, val_offsets.data_ptr(), flat_row_offsets.data_ptr(), ocode,
            weight.data_ptr(), _capi.dtype_code(weight.dtype), out.data_ptr(), batch_size, num_slots, emb_dim,
            max_idx, flat_values.numel(), _capi.pooling_code(pooling), ln_weight.data_ptr(), ln_bias.data_ptr(),
            _capi.dtype_code(ln_weight.dtype), float(eps), _capi.current_stream_handle(dev))
        if rc == _capi.EUNSUPPORTED:
            if pooling != "sum":
                raise _capi.EbagError(rc, _capi.last_error() + " (the unfused fallback pools by sum only)")
            code = _capi.dtype_code(weight.dtype)
            _capi.check(lib.cti_ebag_fused_all_slots_typed(
                flat_values.data_ptr(), icode, val_offsets.data_ptr(), flat_row_offsets.data_ptr(), ocode,
                weight.data_ptr(), code, None, out.data_ptr(), code, batch_size, num_slots, emb_dim, max_idx,
                flat_values.numel(), _capi.current_stream_handle(dev)))
            return layer_norm(out, ln_weight, ln_bias, eps, out=out)
        _capi.check(rc)
    return out


def fused_embedding(batch: dict, weight: torch.Tensor, slot_num: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The fused embedding step of RepEncoder.forward (online_best/infer.py:1029-1059) on a
    batch dict holding ``_flat_values``, ``_flat_row_offsets`` and ``_val_offsets``.

    B is derived from the offsets length as at online_best/infer.py:1033; ``out`` is allocated
    in the weight dtype when not given (online_best/infer.py:1050-1051). A batch staged with a
    dispatch order (``InputStager(order_for=...)``) carries it as ``_tile_order``; the launch
    follows it.
    """
    flat_values = batch["_flat_values"]
    flat_row_offsets = batch["_flat_row_offsets"]
    val_offsets = batch["_val_offsets"]
    batch_size = flat_row_offsets.shape[0] // slot_num - 1
    emb_dim = weight.shape[1]
    if out is None:
        out = torch.empty((batch_size, slot_num * emb_dim), device=weight.device, dtype=weight.dtype)
    return fused_all_slots_embedding(flat_values, val_offsets, flat_row_offsets, weight, out,
                                     batch_size, emb_dim, weight.shape[0] - 1, tile_order=batch.get("_tile_order"))


def embedding_bag_pooled(
    values: torch.Tensor,
    offsets: torch.Tensor,
    tables: Sequence,
    pooling: str = "sum",
    out_dtype: Optional[torch.dtype] = None,
    out: Optional[torch.Tensor] = None,
    long_threshold: int = 0,
    use_bins: bool = False,
    block_threshold: int = 0,
    split_threshold: int = 0,
) -> torch.Tensor:
    """Pool F fields with per-field tables into ``out[B, sum(D_f)]``.

      values   int64 or int32 [nnz], field-major
      offsets  int64 [F*B+1]; bag (f, b) = values[offsets[f*B+b] : offsets[f*B+b+1]]
      tables   F row-major 2-D tensors [V_f, D_f] of one dtype (fp32 / bf16 / fp16); row
               stride may exceed D_f. Field f fills columns [sum_{g<f} D_g, ... + D_f).
               Or F int8 pairs (q [V_f, D_f] int8, scale [V_f] float32): element =
               q * scale[row], fused into the accumulation (one fma per element).
      pooling  'sum' or 'mean' (mean of an empty bag is 0)
      out_dtype defaults to the tables' dtype (bfloat16 for int8 tables); ``out`` (if given) must be contiguous
               [B, sum(D_f)] of that dtype.
      long_threshold  bags longer than this are split over the lane groups of a wavefront
               (0 = per-shape default, -1 = split every non-empty bag). At the default,
               256-byte rows (fp32 D=64, bf16/fp16 D=128) and int8 D=128 rows without binning
               are streamed: every bag is a sequential fp32 sum, whatever its length.
      use_bins  run the device length-binning pass: bags longer than ``block_threshold``
               (0 = default 512) are pooled by a second kernel: one wavefront per bag up to
               ``split_threshold`` rows (0 = default 192), longer bags split across the
               wavefronts of a workgroup. A workspace is allocated for the call; use
               ``PooledEmbedding`` to keep one across calls.
    Equivalent to, per field, F.embedding_bag(clamp(values_f, 0, V_f-1), table_f, offsets_f,
    mode=pooling) followed by concatenation along dim 1 (baseline/infer.py:256-263).
    """
    num_fields = len(tables)
    descs, dev, tcode, width, tdt = _table_descs(tables)
    _require_device_tensor("values", values, dev)
    _require_device_tensor("offsets", offsets, dev)
    _require_contiguous("values", values)
    _require_contiguous("offsets", offsets)
    if offsets.dtype != torch.int64:
        raise TypeError(f"offsets must be int64 (got {offsets.dtype})")
    if (offsets.numel() - 1) % num_fields != 0 or offsets.numel() < 1:
        raise ValueError(f"offsets has {offsets.numel()} entries; expected F*B+1 with F={num_fields}")
    batch_size = (offsets.numel() - 1) // num_fields
    odt = _default_out_dtype(tdt) if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((batch_size, width), device=dev, dtype=odt)
    else:
        _require_device_tensor("out", out, dev)
        _require_contiguous("out", out)
        if out.dtype != odt:
            raise TypeError(f"out dtype {out.dtype} differs from requested {odt}")
        if tuple(out.shape) != (batch_size, width):
            raise ValueError(f"out has shape {tuple(out.shape)}, expected ({batch_size}, {width})")
    opts = _capi.Options()
    opts.long_threshold = int(long_threshold)
    opts.use_bins = int(bool(use_bins))
    opts.block_threshold = int(block_threshold)
    opts.split_threshold = int(split_threshold)
    lib = _capi.lib()
    ws, ws_bytes = None, 0
    if use_bins:
        ws_bytes = lib.cti_ebag_workspace_bytes(batch_size, num_fields)
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        stream = _capi.current_stream_handle(dev)
        _capi.check(lib.cti_ebag_forward(
            values.data_ptr(), _capi.index_code(values.dtype), values.numel(), offsets.data_ptr(),
            batch_size, num_fields, descs, tcode, _capi.pooling_code(pooling),
            out.data_ptr(), _capi.dtype_code(odt), width, ws.data_ptr() if ws is not None else None, ws_bytes,
            ctypes.byref(opts), stream))
    return out


def _default_out_dtype(tdt: torch.dtype) -> torch.dtype:
    """Output dtype when none is given: the tables' dtype, bfloat16 for int8 tables (:940)."""
    return torch.bfloat16 if tdt == torch.int8 else tdt


class PooledEmbedding:
    """A prepared call of the general entry point for fixed tables: the table descriptors and
    options are built once, so each call costs one C-ABI call (a few microseconds on the host).

    ``plan(values, offsets, out=None)`` pools one batch exactly as embedding_bag_pooled would.
    With ``use_bins`` the plan owns one workspace, sized for ``max_batch`` samples, whose list
    counter every call leaves at zero (calls on one plan must not overlap).

    A call may follow an order made on the host from the batch's offsets where the batch is
    produced (``plan(values, offsets, out, tile_order=make_tile_order(...).to(device))``): each
    XCD starts its tiles with the most rows per bag, which shortens the launch's drain; the output
    is the same bit for bit. With ``dispatch_order`` instead, a serving loop that holds no host
    offsets passes the next batch's device offsets with each call
    (``plan(values, offsets, out, next_offsets=...)``): the launch also sorts that batch's tiles,
    most rows per bag first within each XCD's share, and the next call follows that order, which
    shortens the drain at the end of its launch (on tables of 256-byte rows the order's own
    workgroups cost more than the order saves: 4,096 x 28 bags, 33.5 against 31.8 us without an
    order). The plan alternates two device order buffers;
    the output is the same bit for bit with or without an order, whatever batch comes next. Only
    for jobs of one tiled row shape without binning (the library raises otherwise).
    """

    def __init__(self, tables: Sequence, pooling: str = "sum",
                 out_dtype: Optional[torch.dtype] = None, long_threshold: int = 0,
                 use_bins: bool = False, block_threshold: int = 0, max_batch: int = 0,
                 split_threshold: int = 0, dispatch_order: bool = False):
        self.tables = list(tables)  # keeps the tensors (and int8 scales) alive
        self._descs, self.device, self._tdt, self.width, tdt = _table_descs(self.tables)
        self.num_fields = len(self.tables)
        self.table_dtype = tdt
        self.out_dtype = _default_out_dtype(tdt) if out_dtype is None else out_dtype
        self._odt = _capi.dtype_code(self.out_dtype)
        self._pool = _capi.pooling_code(pooling)
        self._opts = _capi.Options()
        self._opts.long_threshold = int(long_threshold)
        self._opts.use_bins = int(bool(use_bins))
        self._opts.block_threshold = int(block_threshold)
        self._opts.split_threshold = int(split_threshold)
        self._lib = _capi.lib()
        self._fn = self._lib.cti_ebag_forward
        self._ws, self._ws_bytes, self.max_batch = None, 0, int(max_batch)
        if use_bins:
            if self.max_batch <= 0:
                raise ValueError("use_bins needs max_batch (the largest batch the plan will see)")
            self._ws_bytes = self._lib.cti_ebag_workspace_bytes(self.max_batch, self.num_fields)
            self._ws = torch.zeros(self._ws_bytes, dtype=torch.uint8, device=self.device)
        if dispatch_order and use_bins:
            raise ValueError("dispatch_order does not combine with use_bins")
        self.dispatch_order = bool(dispatch_order)
        self._orders, self._order_bytes = None, 0
        self._cur, self._have_order = 0, False  # _orders[_cur] holds the order of the coming batch

    def _order_buffers(self, batch: int):
        need = self._lib.cti_ebag_order_bytes(max(batch, self.max_batch), self.num_fields)
        if need > self._order_bytes:
            n = (need + 3) // 4
            self._orders = [torch.zeros(n, dtype=torch.int32, device=self.device) for _ in range(2)]
            self._order_bytes, self._cur, self._have_order = 4 * n, 0, False
        return self._orders

    def __call__(self, values: torch.Tensor, offsets: torch.Tensor, out: Optional[torch.Tensor] = None,
                 next_offsets: Optional[torch.Tensor] = None, tile_order: Optional[torch.Tensor] = None) -> torch.Tensor:
        if values.device != self.device or offsets.device != self.device:
            raise ValueError(f"values and offsets must be on {self.device}")
        if offsets.dtype != torch.int64 or not offsets.is_contiguous() or not values.is_contiguous():
            raise ValueError("offsets must be contiguous int64 and values contiguous")
        n_off = offsets.numel()
        if n_off < 1 or (n_off - 1) % self.num_fields:
            raise ValueError(f"offsets has {n_off} entries; expected F*B+1 with F={self.num_fields}")
        batch = (n_off - 1) // self.num_fields
        if out is None:
            out = torch.empty((batch, self.width), device=self.device, dtype=self.out_dtype)
        elif out.dtype != self.out_dtype or tuple(out.shape) != (batch, self.width) or not out.is_contiguous() \
                or out.device != self.device:
            raise ValueError(f"out must be a contiguous ({batch}, {self.width}) {self.out_dtype} tensor on {self.device}")
        if self._ws is not None and batch > self.max_batch:
            raise ValueError(f"batch {batch} exceeds the plan's max_batch {self.max_batch}")
        if next_offsets is not None:
            if not self.dispatch_order:
                raise ValueError("next_offsets needs a plan made with dispatch_order=True")
            if next_offsets.device != self.device or next_offsets.dtype != torch.int64 \
                    or not next_offsets.is_contiguous() or next_offsets.numel() != n_off:
                raise ValueError(f"next_offsets must be contiguous int64 with {n_off} entries on {self.device}")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        opts = self._opts  # read by the C call before it returns
        if tile_order is not None:
            if self.dispatch_order:
                raise ValueError("tile_order (an order made on the host) and dispatch_order=True (orders made one "
                                 "launch ahead) do not combine")
            if tile_order.device != self.device or tile_order.dtype != torch.int32 or not tile_order.is_contiguous():
                raise ValueError(f"tile_order must be a contiguous int32 tensor on {self.device}")
            opts.tile_order = tile_order.data_ptr()
            opts.next_order = opts.next_offsets = None
            opts.order_bytes = tile_order.numel() * 4
        elif not self.dispatch_order:
            opts.tile_order = opts.next_order = opts.next_offsets = None
            opts.order_bytes = 0
        if self.dispatch_order:
            orders = self._order_buffers(batch)
            opts.tile_order = orders[self._cur].data_ptr() if self._have_order else None
            opts.next_order = orders[1 - self._cur].data_ptr() if next_offsets is not None else None
            opts.next_offsets = next_offsets.data_ptr() if next_offsets is not None else None
            opts.order_bytes = self._order_bytes
        _capi.check(self._fn(values.data_ptr(), _capi.index_code(values.dtype), values.numel(), offsets.data_ptr(),
                             batch, self.num_fields, self._descs, self._tdt, self._pool, out.data_ptr(), self._odt,
                             self.width, self._ws.data_ptr() if self._ws is not None else None, self._ws_bytes,
                             opts, stream))
        if self.dispatch_order:
            if next_offsets is not None:
                self._cur, self._have_order = 1 - self._cur, True
            else:
                self._have_order = False
        return out


def layer_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float = 1e-5,
    out: Optional[torch.Tensor] = None,
    mean: Optional[torch.Tensor] = None,
    rstd: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Row LayerNorm of a 2-D GPU tensor ``x[rows, cols]`` (the encoder's input norm).

    Mirrors ``layernorm_forward_kernel[(rows,)](x, y, gamma, beta, mean, rstd, eps, Row_Size)``
    (online_best/infer.py:829-858, launched at online_best/infer.py:1063-1075): fp32 mean and
    variance over each row, ``y = (x - mean) * rstd * weight + bias`` rounded once to x's dtype.
    ``out`` (default: a new tensor like x, may be x itself), ``mean`` and ``rstd`` (optional,
    fp32 ``[rows]``) are written on torch's current stream. Returns ``out``.
    """
    _require_device_tensor("x", x)
    dev = x.device
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [rows, cols], got shape {tuple(x.shape)}")
    _require_contiguous("x", x)
    rows, cols = x.shape
    for name, t in (("weight", weight), ("bias", bias)):
        _require_device_tensor(name, t, dev)
        _require_contiguous(name, t)
        if t.numel() != cols:
            raise ValueError(f"{name} has {t.numel()} elements, expected {cols}")
    if weight.dtype != bias.dtype:
        raise TypeError(f"weight and bias dtypes differ ({weight.dtype} vs {bias.dtype})")
    if out is None:
        out = torch.empty_like(x)
    _require_device_tensor("out", out, dev)
    _require_contiguous("out", out)
    if out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError(f"out must be {tuple(x.shape)} {x.dtype}, got {tuple(out.shape)} {out.dtype}")
    for name, t in (("mean", mean), ("rstd", rstd)):
        if t is not None:
            _require_device_tensor(name, t, dev)
            if t.dtype != torch.float32 or t.numel() != rows or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 tensor of {rows} elements")
    lib = _capi.lib()
    with torch.cuda.device(dev):
        _capi.check(lib.cti_ebag_layernorm(
            x.data_ptr(), out.data_ptr(), rows, cols, _capi.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(),
            _capi.dtype_code(weight.dtype), float(eps), mean.data_ptr() if mean is not None else None,
            rstd.data_ptr() if rstd is not None else None, _capi.current_stream_handle(dev)))
    return out


def layer_norm_stats(x: torch.Tensor, eps: float = 1e-5, mean: Optional[torch.Tensor] = None,
                     rstd: Optional[torch.Tensor] = None):
    """Per-row mean and rstd of ``x[rows, cols]`` as the input LayerNorm computes them
    (online_best/infer.py:843-852, the kernel's M_ptr / R_ptr outputs), without writing the
    normalised rows. Returns ``(mean, rstd)``, fp32 ``[rows]``."""
    _require_device_tensor("x", x)
    dev = x.device
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [rows, cols], got shape {tuple(x.shape)}")
    _require_contiguous("x", x)
    rows, cols = x.shape
    if mean is None:
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
    if rstd is None:
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    for name, t in (("mean", mean), ("rstd", rstd)):
        _require_device_tensor(name, t, dev)
        if t.dtype != torch.float32 or t.numel() != rows or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor of {rows} elements")
    with torch.cuda.device(dev):
        _capi.check(_capi.lib().cti_ebag_layernorm(
            x.data_ptr(), None, rows, cols, _capi.dtype_code(x.dtype), None, None, _capi.F32, float(eps),
            mean.data_ptr(), rstd.data_ptr(), _capi.current_stream_handle(dev)))
    return mean, rstd


def layer_norm_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    mean: Optional[torch.Tensor] = None,
    rstd: Optional[torch.Tensor] = None,
    norm_weight: Optional[torch.Tensor] = None,
    norm_bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    split_k: bool = True,
) -> torch.Tensor:
    """``linear(layer_norm(x))`` of the encoder in one matrix-core kernel
    (online_best/infer.py:1061-1085): ``x`` bf16 ``[rows, cols]`` (the pooled block), ``mean`` /
    ``rstd`` fp32 ``[rows]`` (``layer_norm_stats``), ``norm_weight`` / ``norm_bias`` the
    LayerNorm's gamma / beta ``[cols]`` (fp32 or bf16), ``weight`` / ``bias`` nn.Linear's
    (bf16 ``[out_features, cols]``, bias fp32 or bf16 ``[out_features]`` or None).

    Each normalised element is computed as the LayerNorm kernel computes it and rounded to bf16
    as it stores it, then multiplied on the matrix cores with fp32 accumulation; the normalised
    block never reaches memory. With mean, rstd, norm_weight and norm_bias all None this is the
    plain Linear. Returns ``out`` ``[rows, out_features]`` (bf16 by default, or ``out_dtype``
    fp32), written on torch's current stream. With ``split_k`` (default) a shape whose output
    tiles would leave CUs idle has K split over several workgroups (fp32 partials in a workspace
    taken from torch's allocator, added in split order; a second launch), so the result can differ
    from ``split_k=False``'s in the last bits, within fp32 accumulation.
    """
    _require_device_tensor("x", x)
    dev = x.device
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError(f"x must be a 2-D bfloat16 tensor, got {tuple(x.shape)} {x.dtype}")
    _require_contiguous("x", x)
    rows, cols = x.shape
    _require_device_tensor("weight", weight, dev)
    _require_contiguous("weight", weight)
    if weight.dim() != 2 or weight.shape[1] != cols or weight.dtype != torch.bfloat16:
        raise ValueError(f"weight must be bfloat16 [out_features, {cols}], got {tuple(weight.shape)} {weight.dtype}")
    n_out = weight.shape[0]
    ln_parts = (mean, rstd, norm_weight, norm_bias)
    ln = any(t is not None for t in ln_parts)
    if ln and not all(t is not None for t in ln_parts):
        raise ValueError("mean, rstd, norm_weight and norm_bias must be given together (or none of them)")
    if ln:
        for name, t in (("mean", mean), ("rstd", rstd)):
            _require_device_tensor(name, t, dev)
            if t.dtype != torch.float32 or t.numel() != rows or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 tensor of {rows} elements")
        for name, t in (("norm_weight", norm_weight), ("norm_bias", norm_bias)):
            _require_device_tensor(name, t, dev)
            _require_contiguous(name, t)
            if t.numel() != cols or t.dtype not in (torch.float32, torch.bfloat16):
                raise ValueError(f"{name} must hold {cols} float32 / bfloat16 elements")
        if norm_weight.dtype != norm_bias.dtype:
            raise TypeError(f"norm_weight and norm_bias dtypes differ ({norm_weight.dtype} vs {norm_bias.dtype})")
    if bias is not None:
        _require_device_tensor("bias", bias, dev)
        _require_contiguous("bias", bias)
        if bias.numel() != n_out or bias.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"bias must hold {n_out} float32 / bfloat16 elements")
    if out is None:
        out = torch.empty((rows, n_out), dtype=out_dtype or torch.bfloat16, device=dev)
    _require_device_tensor("out", out, dev)
    _require_contiguous("out", out)
    if out.shape != (rows, n_out) or out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out must be [{rows}, {n_out}] float32 / bfloat16, got {tuple(out.shape)} {out.dtype}")
    ptr = (lambda t: t.data_ptr() if t is not None else None)
    lib = _capi.lib()
    # K split over several workgroups when few rows would leave CUs idle: fp32 partial products
    # in a workspace from torch's allocator (kept alive until the launches are enqueued)
    ws_bytes = lib.cti_ebag_layernorm_linear_workspace_bytes(rows, cols, n_out) if split_k else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    with torch.cuda.device(dev):
        _capi.check(lib.cti_ebag_layernorm_linear(
            x.data_ptr(), rows, cols, ptr(mean), ptr(rstd), ptr(norm_weight), ptr(norm_bias),
            _capi.dtype_code(norm_weight.dtype) if ln else _capi.F32, weight.data_ptr(), n_out, ptr(bias),
            _capi.dtype_code(bias.dtype) if bias is not None else _capi.F32, out.data_ptr(),
            _capi.dtype_code(out.dtype), ptr(ws), ws_bytes, _capi.current_stream_handle(dev)))
    return out
