"""Checkpoint ingest of the routed-expert tables (the reference's
``glm_tpu/model_loader``, narrowed to the MoE layer's inputs).

* ``safetensors_io``: a minimal safetensors reader and writer over raw bytes
  (numpy memory maps; no deserialisation of anything but the JSON header).
* ``placement``: the reference's checkpoint-name rules for routed experts,
  shared experts and the router, and the expert-parallel coordinate of an expert.
* ``moe_ingest``: ``load_moe_layer`` stacks one layer's per-expert FP8 tensors
  into the ``[E, N, K]`` uint8 + ``[E, N/128, K/128]`` FP32 tables the kernels
  read in place (no repacking), dequantises the shared expert to bf16, and
  applies the finite-bit gate on the GPU.
"""

from glm_moe.model_loader.moe_ingest import CheckpointValidationError, MoeLayerTables, load_moe_layer
from glm_moe.model_loader.placement import expert_coordinate, routed_source, runtime_name
from glm_moe.model_loader.safetensors_io import SafetensorsFile, write_safetensors

__all__ = [
    "CheckpointValidationError",
    "MoeLayerTables",
    "SafetensorsFile",
    "expert_coordinate",
    "load_moe_layer",
    "routed_source",
    "runtime_name",
    "write_safetensors",
]
