"""MI355X-native fused sparse-feature embedding-bag path (hand-written HIP kernels for gfx950).

Public surface:
  fused_all_slots_embedding  drop-in for the reference's fused_all_slots_embedding_kernel launch
  fused_embedding            the RepEncoder.forward fused step on a flat-layout batch dict
  fused_all_slots_embedding_layernorm   the fused step with the input LayerNorm in one kernel
  quantize_embedding_int8    int8 row quantisation of a table (int8 rows + fp32 row scales)
  fused_all_slots_embedding_int8   drop-in for the reference's int8 fused kernel launch
  embedding_bag_pooled       per-field tables, global offsets, sum/mean, chosen output dtype
  PooledEmbedding            the same with the table descriptors prepared once (serving loops)
  layer_norm                 the encoder's input LayerNorm over the pooled rows
  layer_norm_stats           its per-row mean and rstd only
  layer_norm_linear          the input LayerNorm and the encoder's Linear in one matrix-core kernel
  RepEncoder                 the reference module with the fused step and LayerNorm on this path
  collate_flat_layout, prebuild_flat_layout   host builders of the flat layout
  pack_slots, merge_batches                   GPU builders of the flat layout
  InputStager, move_model_inputs_to_device    pinned, int32-compacted, overlapped transfer of
                                              host batches to the GPU
  make_tile_order, order_bytes                a batch's dispatch order, made on the host
"""
from . import workloads
from ._capi import EbagError, lib as load_library
from .encoder import RepEncoder
from .layout import collate_flat_layout, merge_batches, pack_slots, prebuild_flat_layout
from .staging import InputStager, move_model_inputs_to_device
from .ops import (PooledEmbedding, embedding_bag_pooled, fused_all_slots_embedding, fused_all_slots_embedding_int8,
                  fused_all_slots_embedding_layernorm, fused_embedding, layer_norm, layer_norm_linear,
                  layer_norm_stats, make_tile_order, order_bytes, quantize_embedding_int8)

__all__ = [
    "EbagError",
    "load_library",
    "RepEncoder",
    "collate_flat_layout",
    "prebuild_flat_layout",
    "pack_slots",
    "merge_batches",
    "InputStager",
    "move_model_inputs_to_device",
    "embedding_bag_pooled",
    "PooledEmbedding",
    "fused_all_slots_embedding",
    "fused_embedding",
    "fused_all_slots_embedding_int8",
    "fused_all_slots_embedding_layernorm",
    "quantize_embedding_int8",
    "layer_norm",
    "layer_norm_stats",
    "layer_norm_linear",
    "make_tile_order",
    "order_bytes",
    "workloads",
]
