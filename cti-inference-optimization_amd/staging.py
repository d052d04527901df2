"""Moving flat-layout batches from host memory to the GPU: the input side of the pooling step.

The reference moves its flat layout with ``.to(device, non_blocking=True)`` of int64 CPU tensors,
one copy per tensor (``move_model_inputs_to_device``, online_best/infer.py:742-779). From
pageable memory each copy is staged by the driver and does not overlap the GPU's work.
``InputStager`` keeps a ring of ``depth`` pinned host regions and matching device regions; per
batch one native call (``cti_ebag_stage_copy``):

  1. writes ids, row offsets and slot offsets into the slot's pinned region, narrowed to int32
     when ``compact`` (saturating, so the device clamp selects the same rows and the pooled
     result is the int64 result bit for bit), on a pool of host threads;
  2. enqueues one asynchronous copy of the region on a side stream;

and torch's current stream waits for that copy (an event), so the pooling launched next reads
complete inputs while the copy of the following batch overlaps it. The pooling kernels read
int32 ids and offsets directly (no widening kernel). A slot is reused only after ``release``
has recorded, on the consumer's stream, that the work reading it was enqueued; ``stage`` raises
if the slot it needs was never released.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

from . import _capi
from .layout import pack_slots

_PARTS = ("_flat_values", "_flat_row_offsets", "_val_offsets")


def _host_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


class InputStager:
    """Ring of pinned host / device regions for flat-layout batches.

    ``max_nnz``, ``num_slots`` and ``max_batch`` size the regions; ``compact`` selects int32 ids
    and offsets (else int64, as the reference sends them). ``order_for=(table dtype, emb_dim)``
    (with ``compact``) also makes each batch's dispatch order on the host from the offsets being
    staged and sends it in the same copy as ``_tile_order``, which ``fused_embedding`` and
    ``RepEncoder`` follow (results unchanged bit for bit); a batch that already carries a host
    ``_tile_order`` (made by its producer with ``make_tile_order``) has that one sent instead.
    Dropping the stager (or ``close()``)
    waits for its copies; work that still reads a staged batch must be ordered before any reuse of
    that memory by the caller.
    """

    def __init__(self, max_nnz: int, num_slots: int, max_batch: int, device=None, depth: int = 2,
                 compact: bool = True, threads: Optional[int] = None, order_for=None):
        if depth < 1:
            raise ValueError("depth must be >= 1")
        if order_for is not None and not compact:
            raise ValueError("order_for needs compact=True (the order travels as int32 in the same copy)")
        if max_nnz < 0 or num_slots < 1 or max_batch < 0:
            raise ValueError("max_nnz >= 0, num_slots >= 1 and max_batch >= 0 are required")
        if compact and max_nnz >= 2 ** 31:
            raise ValueError("int32 offsets need max_nnz < 2^31")
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.device = dev if dev.index is not None else torch.device("cuda", torch.cuda.current_device())
        self.depth, self.compact = depth, compact
        self.num_slots, self.max_nnz, self.max_batch = num_slots, max_nnz, max_batch
        self.threads = threads or _host_threads()
        self._lib = _capi.lib()
        self._code = _capi.I32 if compact else _capi.I64
        self.dtype = torch.int32 if compact else torch.int64
        # optional fourth part: the batch's dispatch order for a table of (dtype, emb_dim), made on
        # the host from the offsets being staged and sent in the same copy
        self.order_for = order_for
        self._order_elems = 0
        if order_for is not None:
            from .ops import order_bytes
            self._order_elems = (order_bytes(max_batch, num_slots) + 3) // 4
            self._order_host = torch.empty(self._order_elems, dtype=torch.int32)
        counts = [max_nnz, num_slots * (max_batch + 1), num_slots] + ([self._order_elems] if order_for else [])
        self.region_bytes = self._offset(counts, len(counts))
        self._h = [torch.empty(self.region_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self._d = [torch.empty(self.region_bytes, dtype=torch.uint8, device=self.device) for _ in range(depth)]
        self.copy_stream = torch.cuda.Stream(self.device)  # default priority
        self._copied = [torch.cuda.Event() for _ in range(depth)]
        self._consumed = [torch.cuda.Event() for _ in range(depth)]
        self._in_use = [False] * depth
        self._next = 0

    def _offset(self, counts, part: int) -> int:
        c = (ctypes.c_int64 * len(counts))(*counts)
        off = self._lib.cti_ebag_stage_offset(c, len(counts), self._code, part)
        if off < 0:
            raise ValueError(f"bad part sizes {list(counts)}")
        return off

    def bytes_per_batch(self, nnz: int, batch: int) -> int:
        """Bytes one batch moves host -> device."""
        counts = [nnz, self.num_slots * (batch + 1), self.num_slots]
        if self.order_for is not None:
            from .ops import order_bytes
            counts.append((order_bytes(batch, self.num_slots) + 3) // 4)
        return self._offset(counts, len(counts))

    def stage(self, batch: dict) -> dict:
        """Start moving one host batch (``_flat_values``, ``_flat_row_offsets``, ``_val_offsets``;
        int64 or int32 CPU tensors in the reference layout) to the device. Returns the device
        batch (same keys, plus ``_stage_slot``); torch's current stream is ordered after the copy."""
        ts = [batch[k] for k in _PARTS]
        for name, t in zip(_PARTS, ts):
            if t.device.type != "cpu" or t.dtype not in (torch.int64, torch.int32):
                raise ValueError(f"{name} must be an int64 or int32 CPU tensor")
        ts = [t.contiguous() for t in ts]
        nnz, n_off, n_vo = (t.numel() for t in ts)
        if n_vo != self.num_slots:
            raise ValueError(f"_val_offsets has {n_vo} entries, expected {self.num_slots}")
        if n_off % self.num_slots or n_off < self.num_slots or n_off // self.num_slots - 1 > self.max_batch:
            raise ValueError(f"_flat_row_offsets has {n_off} entries: more samples than max_batch={self.max_batch} "
                             f"or not a multiple of num_slots={self.num_slots}")
        if nnz > self.max_nnz:
            raise ValueError(f"batch has {nnz} ids, the stager holds {self.max_nnz}")
        slot = self._next
        if self._in_use[slot]:
            raise RuntimeError(f"staging slot {slot} is still in use: call release() on the batch staged into it "
                               "after enqueuing the work that reads it")
        self._next = (slot + 1) % self.depth
        counts = [nnz, n_off, n_vo]
        if self.order_for is not None:
            from .ops import make_tile_order, order_bytes
            batch_size = n_off // self.num_slots - 1
            n_order = (order_bytes(batch_size, self.num_slots) + 3) // 4
            made = batch.get("_tile_order")
            if made is not None:  # made by the batch's producer (e.g. its collate), shipped as it is
                if made.device.type != "cpu" or made.dtype != torch.int32 or made.numel() > self._order_elems:
                    raise ValueError(f"_tile_order must be a CPU int32 tensor of at most {self._order_elems} entries")
                ts = ts + [made.contiguous()]
            else:
                make_tile_order(ts[1], batch_size, self.num_slots, self.order_for[0], self.order_for[1],
                                out=self._order_host, threads=self.threads)
                ts = ts + [self._order_host[:n_order]]
            counts.append(ts[3].numel())
        n = len(ts)
        src = (ctypes.c_void_p * n)(*[t.data_ptr() if t.numel() else None for t in ts])
        st = (ctypes.c_int32 * n)(*[_capi.index_code(t.dtype) for t in ts])
        cnt = (ctypes.c_int64 * n)(*counts)
        self._copied[slot].synchronize()  # the previous copy out of this slot's pinned region is done
        self.copy_stream.wait_event(self._consumed[slot])  # the device region is no longer read
        _capi.check(self._lib.cti_ebag_stage_copy(src, st, cnt, n, self._code, self._h[slot].data_ptr(),
                                                  self.region_bytes, self._d[slot].data_ptr(), self.threads,
                                                  self.copy_stream.cuda_stream))
        self._copied[slot].record(self.copy_stream)
        torch.cuda.current_stream(self.device).wait_event(self._copied[slot])
        self._in_use[slot] = True
        out = {"_stage_slot": slot}
        d = self._d[slot]
        for k, c, part in zip(_PARTS + ("_tile_order",), counts, range(n)):
            off = self._offset(counts, part)
            out[k] = d[off:off + c * (4 if self.compact else 8)].view(self.dtype)
        return out

    def close(self) -> None:
        """Wait for this stager's copies: its pinned regions are then safe to free. (The copies are
        issued by the library, so torch's pinned-memory allocator does not track them.)"""
        if getattr(self, "copy_stream", None) is not None:
            self.copy_stream.synchronize()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the HIP runtime may already be gone
            pass

    def release(self, staged: dict) -> None:
        """Mark the staged batch's device region reusable once the work enqueued so far on torch's
        current stream (the work that reads it) has run."""
        slot = staged["_stage_slot"]
        self._consumed[slot].record(torch.cuda.current_stream(self.device))
        self._in_use[slot] = False


def _to_device(x, device):
    """``x`` with every tensor inside it (through dicts, lists and tuples) moved to ``device``
    with ``non_blocking=True``; anything else is returned as it is."""
    if isinstance(x, torch.Tensor):
        return x.to(device, non_blocking=True)
    if isinstance(x, dict):
        return {k: _to_device(v, device) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return type(x)(_to_device(v, device) for v in x)
    return x


def move_model_inputs_to_device(batch: dict, device, slot_num: int = 28,
                                stager: Optional[InputStager] = None) -> dict:
    """online_best/infer.py:742-779 for the embedding inputs.

    Flat-layout batches go through ``stager`` when one is given (pinned, int32-compacted,
    overlapped; release the result with ``stager.release``), else through ``.to(device,
    non_blocking=True)`` as in the reference (val_offsets widened to int64, :747). Batches that
    carry only the per-slot pairs ``{i+1: (values, offsets)}`` are moved slot by slot and packed
    on the device by one kernel (``pack_slots``) instead of two ``torch.cat`` and a host tensor
    (:750-762). The attention stage's inputs are passed on as the reference passes them
    (:763-778): ``_attn_groups`` with every tensor inside it moved to the device, and
    ``user_offsets`` only when the batch has no ``_attn_groups`` (the model takes the
    varlen-attention path when it finds ``user_offsets``). No other key is moved.
    """
    device = torch.device(device)
    if "_flat_values" in batch:
        if stager is not None:
            model_batch = stager.stage(batch)
        else:
            model_batch = {
                "_flat_values": batch["_flat_values"].to(device, non_blocking=True),
                "_flat_row_offsets": batch["_flat_row_offsets"].to(device, non_blocking=True),
                "_val_offsets": batch["_val_offsets"].to(device, non_blocking=True).long(),
            }
    else:
        slots = []
        for s in range(1, slot_num + 1):
            vals, offs = batch[s]
            slots.append((vals.to(device, non_blocking=True).long(), offs.to(device, non_blocking=True).long()))
        model_batch = dict(pack_slots(slots))
    if "_attn_groups" in batch:
        model_batch["_attn_groups"] = _to_device(batch["_attn_groups"], device)
    elif "user_offsets" in batch:
        model_batch["user_offsets"] = batch["user_offsets"].to(device, non_blocking=True)
    return model_batch
