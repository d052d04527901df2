"""Builders of the flat sparse-feature layout (the input format of the fused step).

The reference keeps a batch as 28 per-slot ``(values, offsets)`` pairs (int keys 1..28) and, for
the fused kernel, as three packed tensors (online_best/infer.py:446-474):

  _flat_values       int64 [nnz]       all slots' sign ids, slot-major, samples in batch order
  _flat_row_offsets  int64 [S*(B+1)]   slot s at [s*(B+1), (s+1)*(B+1)), local to the slot (starts at 0)
  _val_offsets       int64 [S]         start of each slot inside _flat_values

The general entry point takes the equivalent global form ``offsets[S*B+1]`` with
``offsets[s*B+b] = val_offsets[s] + row_offsets[s*(B+1)+b]`` and ``offsets[S*B] = nnz``.

Host builders (``collate_flat_layout``, ``prebuild_flat_layout``) follow the reference's own
host code; ``pack_slots`` and ``merge_batches`` run on the GPU (HIP kernels behind the C ABI).
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Sequence, Tuple

import torch

from . import _capi


def collate_flat_layout(feasigns: Sequence[Dict[int, Sequence[int]]], max_slot_id: int) -> dict:
    """Flat layout of a list of samples, each a dict slot -> sign ids (slots 1..max_slot_id).

    Same loop as make_collate_fn's slot section (online_best/infer.py:446-474): per slot, extend
    the values with every sample's ids in order and record the running length; missing slots
    give empty bags. Returns the int-keyed per-slot pairs plus the three flat tensors (CPU).
    """
    slot_data = {}
    values_parts: List[torch.Tensor] = []
    offsets_parts: List[torch.Tensor] = []
    val_offsets = [0]
    for slot in range(1, max_slot_id + 1):
        values: List[int] = []
        offsets = [0]
        for fs in feasigns:
            if slot in fs:
                values.extend(fs[slot])
            offsets.append(len(values))
        vt = torch.tensor(values, dtype=torch.long)
        ot = torch.tensor(offsets, dtype=torch.long)
        slot_data[slot] = (vt, ot)
        values_parts.append(vt)
        offsets_parts.append(ot)
        val_offsets.append(val_offsets[-1] + vt.numel())
    result = {
        "_flat_values": torch.cat(values_parts) if values_parts else torch.empty(0, dtype=torch.long),
        "_flat_row_offsets": torch.cat(offsets_parts) if offsets_parts else torch.empty(0, dtype=torch.long),
        "_val_offsets": torch.tensor(val_offsets[:-1], dtype=torch.long),
    }
    result.update(slot_data)
    return result


def prebuild_flat_layout(batch: dict, slot_num: int = 28) -> bool:
    """Add the flat tensors to a batch that only has per-slot pairs (online_best/infer.py:139-154).

    Returns False (and leaves the batch alone) when the batch already has ``_flat_values`` or
    lacks a slot, as the reference does.
    """
    if not (isinstance(batch, dict) and 1 in batch and "_flat_values" not in batch):
        return False
    vals, offs, lens = [], [], [0]
    for slot in range(1, slot_num + 1):
        if slot not in batch:
            return False
        v, o = batch[slot]
        vals.append(v)
        offs.append(o)
        lens.append(lens[-1] + v.shape[0])
    batch["_flat_values"] = torch.cat(vals).long()
    batch["_flat_row_offsets"] = torch.cat(offs).long()
    batch["_val_offsets"] = torch.tensor(lens[:-1], dtype=torch.long, device=vals[0].device)
    return True


def _ptr_array(tensors: Sequence[torch.Tensor]):
    arr = (ctypes.c_void_p * len(tensors))()
    for i, t in enumerate(tensors):
        arr[i] = t.data_ptr() if t.numel() > 0 else None
    return arr


def _i64_array(vals: Sequence[int]):
    arr = (ctypes.c_int64 * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr


def pack_slots(slots: Sequence[Tuple[torch.Tensor, torch.Tensor]], with_global_offsets: bool = False) -> dict:
    """Pack per-slot (values, offsets) GPU tensors into the flat layout on the GPU.

    Device counterpart of online_best/infer.py:960-974 (which uses torch.cat plus a host->device
    copy of val_offsets): one HIP kernel writes all three tensors (and optionally the global
    offsets); val_offsets comes from the tensors' sizes, so nothing is read back.
    """
    if not slots:
        raise ValueError("no slots to pack")
    dev = slots[0][0].device
    if dev.type != "cuda":
        raise ValueError(f"slot 0: all tensors must be on the same GPU ({dev})")
    di = dev.index if dev.index is not None else torch.cuda.current_device()
    batch_size = slots[0][1].numel() - 1
    vals, offs, nnz = [], [], []
    for s, (v, o) in enumerate(slots):  # few tensor attributes per slot: they dominate small calls
        if v.get_device() != di or o.get_device() != di:
            raise ValueError(f"slot {s}: all tensors must be on the same GPU ({dev})")
        if v.dtype is not torch.int64 or o.dtype is not torch.int64:
            raise TypeError(f"slot {s}: values and offsets must be int64")
        if o.numel() != batch_size + 1:
            raise ValueError(f"slot {s}: offsets has {o.numel()} entries, expected {batch_size + 1}")
        vals.append(v if v.is_contiguous() else v.contiguous())
        offs.append(o if o.is_contiguous() else o.contiguous())
        nnz.append(v.numel())
    total = sum(nnz)
    S = len(slots)
    flat_values = torch.empty(total, dtype=torch.int64, device=dev)
    flat_row_offsets = torch.empty(S * (batch_size + 1), dtype=torch.int64, device=dev)
    val_offsets = torch.empty(S, dtype=torch.int64, device=dev)
    goff = torch.empty(S * batch_size + 1, dtype=torch.int64, device=dev) if with_global_offsets else None
    lib = _capi.lib()
    with torch.cuda.device(dev):
        _capi.check(lib.cti_ebag_pack_slots(
            _ptr_array(vals), _ptr_array(offs), _i64_array(nnz), S, batch_size,
            flat_values.data_ptr() if total else None, flat_row_offsets.data_ptr(), val_offsets.data_ptr(),
            goff.data_ptr() if goff is not None else None, _capi.current_stream_handle(dev)))
    out = {"_flat_values": flat_values, "_flat_row_offsets": flat_row_offsets, "_val_offsets": val_offsets}
    if goff is not None:
        out["offsets"] = goff
    return out


def merge_batches(batches: Sequence[dict], slot_num: int = 28, with_global_offsets: bool = False,
                  int32_round_trip: bool = False) -> dict:
    """Concatenate flat-layout sub-batches slot by slot on the GPU.

    Same result as _timed_lazy_merge_group_cpu (online_best/infer.py:581-631): for each slot,
    the sub-batches' value slices in order, their local offsets rebased by the slot's running
    value count, closed by the slot total. Each batch needs ``_flat_values``,
    ``_flat_row_offsets`` and ``_val_offsets`` on one GPU; its batch size is read from the
    offsets length.

    ``int32_round_trip`` gives the pair merge's result instead (_timed_merge_batch_pair,
    online_best/infer.py:2977-3037): merged values and row offsets pass through int32 (``.int()``
    then ``.long()``, :3008-3009 and :3019-3020), so values or slot offsets of 2^31 or more wrap.
    """
    if not batches:
        raise ValueError("no batches to merge")
    dev = batches[0]["_flat_values"].device
    vals, vos, ros, bs, nnz = [], [], [], [], []
    for k, b in enumerate(batches):
        v, ro, vo = b["_flat_values"], b["_flat_row_offsets"], b["_val_offsets"]
        for name, t in (("_flat_values", v), ("_flat_row_offsets", ro), ("_val_offsets", vo)):
            if t.device != dev or dev.type != "cuda":
                raise ValueError(f"batch {k}: {name} must be on {dev}")
            if t.dtype != torch.int64:
                raise TypeError(f"batch {k}: {name} must be int64")
        if vo.numel() != slot_num or ro.numel() % slot_num != 0:
            raise ValueError(f"batch {k}: layout does not have {slot_num} slots")
        vals.append(v.contiguous())
        vos.append(vo.contiguous())
        ros.append(ro.contiguous())
        bs.append(ro.numel() // slot_num - 1)
        nnz.append(v.numel())
    B = sum(bs)
    total = sum(nnz)
    flat_values = torch.empty(total, dtype=torch.int64, device=dev)
    flat_row_offsets = torch.empty(slot_num * (B + 1), dtype=torch.int64, device=dev)
    val_offsets = torch.empty(slot_num, dtype=torch.int64, device=dev)
    goff = torch.empty(slot_num * B + 1, dtype=torch.int64, device=dev) if with_global_offsets else None
    lib = _capi.lib()
    with torch.cuda.device(dev):
        fn = lib.cti_ebag_merge_batches_int32 if int32_round_trip else lib.cti_ebag_merge_batches
        _capi.check(fn(
            _ptr_array(vals), _ptr_array(vos), _ptr_array(ros), _i64_array(bs), _i64_array(nnz),
            len(batches), slot_num, flat_values.data_ptr() if total else None, flat_row_offsets.data_ptr(),
            val_offsets.data_ptr(), goff.data_ptr() if goff is not None else None,
            _capi.current_stream_handle(dev)))
    out = {"_flat_values": flat_values, "_flat_row_offsets": flat_row_offsets, "_val_offsets": val_offsets}
    if goff is not None:
        out["offsets"] = goff
    return out
