"""RepEncoder with the fused embedding step and the input LayerNorm on the HIP path.

Mirrors the reference module online_best/infer.py:945-1100 (constructor signature, parameter
names, forward(batch) contract): the 28 slots are pooled into ``[B, slot_num*emb_dim]`` in the
table's dtype and normalised with the ``input_norm`` parameters (the reference's Triton
LayerNorm, online_best/infer.py:1061-1076) by one fused kernel
(``fused_all_slots_embedding_layernorm``; ``pooled`` alone uses ``fused_all_slots_embedding``),
and ``linear`` maps them to d_model (online_best/infer.py:1085). ``forward`` pools, normalises
the pooled block in place and runs ``linear``; ``forward(batch, fused_linear=True)`` instead runs
one matrix-core kernel that applies the LayerNorm to the pooled block's tiles as it loads them
and multiplies them with the Linear's weight (``layer_norm_linear``, after ``layer_norm_stats``).
Like the reference's Triton kernels, the pooling and the LayerNorm are forward-only (inference).

``quantize_int8_()`` is the reference's int8 switch (``_USE_INT8_EMB``, online_best/infer.py:893
and :976-1026): the table is row-quantised once on the device and every later ``pooled`` reads
the int8 rows and their fp32 scales; ``dequantize_()`` switches back to the float table.
"""
from __future__ import annotations

import torch
from torch import nn

from .layout import pack_slots
from .ops import (fused_all_slots_embedding, fused_all_slots_embedding_int8, fused_all_slots_embedding_layernorm,
                  layer_norm, layer_norm_linear, layer_norm_stats, quantize_embedding_int8)


class RepEncoder(nn.Module):
    def __init__(self, vocab_size, emb_dim, padding_idx=0, slot_num=0, d_model=0):
        super().__init__()
        self.emb = nn.Embedding(num_embeddings=vocab_size, embedding_dim=emb_dim, padding_idx=padding_idx)
        self.emb_dim = emb_dim
        self.slot_num = slot_num
        self.input_norm = nn.LayerNorm(slot_num * emb_dim)
        self.linear = nn.Linear(in_features=slot_num * emb_dim, out_features=d_model)
        self._int8_weight = None
        self._int8_scale = None

    def quantize_int8_(self):
        """Quantise the table to int8 rows + fp32 row scales (online_best/infer.py:980-987)."""
        with torch.no_grad():
            self._int8_weight, self._int8_scale = quantize_embedding_int8(self.emb.weight.detach())
        return self

    def dequantize_(self):
        self._int8_weight = self._int8_scale = None
        return self

    def flat_inputs(self, batch: dict):
        """(flat_values, val_offsets, flat_row_offsets, batch_size) of a batch.

        Batches that carry only the int-keyed per-slot pairs are packed on the GPU
        (online_best/infer.py:960-974); B comes from the offsets length (online_best/infer.py:1033).
        """
        if "_flat_values" not in batch:
            device = self.emb.weight.device
            slots = []
            for i in range(self.slot_num):
                vals, offs = batch[i + 1]
                # tensors already on a GPU are passed as they are (pack_slots checks that they are
                # on this one): .to() on them costs as much as the rest of the packing
                slots.append((vals if vals.is_cuda else vals.to(device), offs if offs.is_cuda else offs.to(device)))
            batch = pack_slots(slots)
        flat_values = batch["_flat_values"]
        flat_row_offsets = batch["_flat_row_offsets"]
        val_offsets = batch["_val_offsets"]
        batch_size = flat_row_offsets.shape[0] // self.slot_num - 1
        return flat_values, val_offsets, flat_row_offsets, batch_size

    def pooled(self, batch: dict) -> torch.Tensor:
        """The fused embedding step: ``[B, slot_num*emb_dim]`` in the table dtype (following the
        batch's ``_tile_order`` when it carries one)."""
        flat_values, val_offsets, flat_row_offsets, batch_size = self.flat_inputs(batch)
        weight = self.emb.weight
        out = torch.empty((batch_size, self.slot_num * self.emb_dim), device=weight.device, dtype=weight.dtype)
        with torch.no_grad():
            if self._int8_weight is not None:
                return fused_all_slots_embedding_int8(flat_values, val_offsets, flat_row_offsets, self._int8_weight,
                                                      self._int8_scale, out, batch_size, self.emb_dim,
                                                      self.emb.num_embeddings - 1)
            return fused_all_slots_embedding(flat_values, val_offsets, flat_row_offsets, weight.detach(), out,
                                             batch_size, self.emb_dim, self.emb.num_embeddings - 1,
                                             tile_order=batch.get("_tile_order"))

    def normalized(self, batch: dict) -> torch.Tensor:
        """Pooled rows after the input LayerNorm: ``[B, slot_num*emb_dim]`` in the table dtype.

        With the float table, pooling and LayerNorm run as one kernel (the pooled row stays on
        chip); with the int8 table, the int8 pooling is followed by the LayerNorm kernel.
        """
        norm = self.input_norm
        if self._int8_weight is not None:
            fused_embs = self.pooled(batch)
            with torch.no_grad():
                return layer_norm(fused_embs, norm.weight.detach(), norm.bias.detach(), norm.eps, out=fused_embs)
        flat_values, val_offsets, flat_row_offsets, batch_size = self.flat_inputs(batch)
        weight = self.emb.weight
        out = torch.empty((batch_size, self.slot_num * self.emb_dim), device=weight.device, dtype=weight.dtype)
        with torch.no_grad():
            return fused_all_slots_embedding_layernorm(flat_values, val_offsets, flat_row_offsets, weight.detach(), out,
                                                       batch_size, self.emb_dim, self.emb.num_embeddings - 1,
                                                       norm.weight.detach(), norm.bias.detach(), norm.eps)

    def forward(self, batch: dict, fused_linear: bool = False) -> torch.Tensor:
        """``linear(input_norm(pooled))`` (online_best/infer.py:1029-1085).

        By default the pooled block is normalised in place by the LayerNorm kernel and mapped by
        ``linear`` (torch's GEMM), the faster order at the encoder shape (B = 4096, Linear
        3584 -> 512) and at the merged 32,768-sample batch. ``fused_linear=True`` takes the
        statistics pass and the matrix-core kernel that normalises the pooled block's tiles as it
        loads them (``layer_norm_linear``, K split over the chip when the rows are few), so the
        normalised block never reaches memory; at the reference's small warm-up batches the two
        orders are within a few microseconds of each other. It needs a bf16 table and a bf16
        ``linear`` with LayerNorm parameters in bf16 or fp32 (the reference's model after
        ``model.to(bfloat16)``, online_best/infer.py:2797).
        """
        lin, norm = self.linear, self.input_norm
        if fused_linear:
            if not (self.emb.weight.dtype == torch.bfloat16 and lin.weight.dtype == torch.bfloat16
                    and norm.weight.dtype in (torch.bfloat16, torch.float32) and norm.weight.dtype == norm.bias.dtype
                    and self._int8_weight is None):
                raise ValueError("fused_linear needs a bf16 table and Linear and bf16 or fp32 LayerNorm parameters")
            fused_embs = self.pooled(batch)
            with torch.no_grad():
                mean, rstd = layer_norm_stats(fused_embs, norm.eps)
                return layer_norm_linear(fused_embs, lin.weight.detach(),
                                         lin.bias.detach() if lin.bias is not None else None, mean=mean, rstd=rstd,
                                         norm_weight=norm.weight.detach(), norm_bias=norm.bias.detach())
        fused_embs = self.pooled(batch)
        with torch.no_grad():
            fused_embs = layer_norm(fused_embs, norm.weight.detach(), norm.bias.detach(), norm.eps, out=fused_embs)
        return self.linear(fused_embs)
