"""Route-grouped raw-FP8 projections of the decode MoE's routed experts.

Mirrors ``glm_tpu/kernels/fp8_grouped_matmul/kernel.py``:
``RoutedProjectionConfig`` (``:53-94``) and ``fp8_routed_projection``
(``:125-299``).  On the GPU the owned slots become one-row work tiles of the
grouped gfx950 kernel (split-K over four waves); each selected expert's
weights are streamed once from HBM with 128-bit loads, decoded per 128x128
block in registers to bf16 and multiplied on MFMA with FP32 accumulation.
The TPU tile sizes of the config are validated for signature parity; the GPU
kernel picks its own tiling.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from glm_moe import _lib


@dataclass(frozen=True, slots=True)
class RoutedProjectionConfig:
    """Static tile contract of the reference's routed projection (``kernel.py:53-94``)."""

    block_shape: tuple[int, int] = (128, 128)
    output_tile: int = 512
    contraction_tile: int = 512
    write_empty_slot: bool = True

    def __post_init__(self) -> None:
        if self.write_empty_slot is not True:
            raise ValueError("optimized release always initializes empty route slots")
        if len(self.block_shape) != 2 or any(
            not isinstance(v, int) or isinstance(v, bool) or v <= 0 for v in self.block_shape
        ):
            raise ValueError("routed FP8 block shape must contain two positive integers")
        for name in ("output_tile", "contraction_tile"):
            value = getattr(self, name)
            if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if self.output_tile % self.block_shape[0]:
            raise ValueError("output_tile must be a multiple of the output scale block")
        if self.contraction_tile % self.block_shape[1]:
            raise ValueError("contraction_tile must be a multiple of the contraction scale block")
        if 8 % self.blocks_per_contraction_tile:
            raise ValueError("contraction_tile may span 1, 2, 4 or 8 scale blocks (one VMEM slab)")
        if self.blocks_per_output_tile > 128:
            raise ValueError("output_tile may span at most 128 scale blocks")

    @property
    def blocks_per_output_tile(self) -> int:
        return self.output_tile // self.block_shape[0]

    @property
    def blocks_per_contraction_tile(self) -> int:
        return self.contraction_tile // self.block_shape[1]


def fp8_routed_projection(
    lhs: torch.Tensor,
    weights: tuple[tuple[torch.Tensor, torch.Tensor], ...],
    local_expert_ids: torch.Tensor,
    owned: torch.Tensor,
    *,
    config: RoutedProjectionConfig = RoutedProjectionConfig(),
    result_dtype: Any = torch.float32,
    interpret: bool = False,
) -> torch.Tensor:
    """Project one bf16 row per route slot against that slot's selected expert.

    ``lhs`` is ``[slots, K]``; every ``weights`` entry is a ``(bits [E, N, K]
    uint8, scale [E, N/bn, K/bk] float32)`` pair sharing ``N`` and ``K``.
    ``local_expert_ids [slots]`` (clipped to ``[0, E)``) selects each slot's
    expert, ``owned [slots]`` marks the computed slots; unowned slots are exact
    zeros.  Returns ``[slots, len(weights), N]``.
    """
    del interpret
    if not isinstance(weights, tuple) or not 1 <= len(weights) <= 2:
        raise ValueError("routed FP8 projection takes one or two weight table pairs")
    if lhs.ndim != 2 or lhs.dtype != torch.bfloat16:
        raise ValueError("routed FP8 lhs must be BF16 [slots, K]")
    slots, contraction = lhs.shape
    if slots <= 0 or contraction <= 0:
        raise ValueError("routed FP8 lhs dimensions must be positive")
    first_bits = weights[0][0]
    if first_bits.ndim != 3:
        raise ValueError("routed FP8 weights must be [E, N, K] uint8")
    experts, output, weight_contraction = first_bits.shape
    if min(experts, output) <= 0 or weight_contraction != contraction:
        raise ValueError("routed FP8 weight/input geometry disagrees")
    bn, bk = config.block_shape
    if (bn, bk) != (128, 128):
        raise ValueError("the gfx950 routed projection decodes 128x128 scale blocks")
    if output % config.output_tile or contraction % config.contraction_tile:
        raise ValueError("routed FP8 requires N/K divisible by the output/contraction tiles")
    for bits, scale in weights:
        if tuple(bits.shape) != (experts, output, contraction) or bits.dtype != torch.uint8:
            raise ValueError("routed FP8 weight tables must share [E, N, K] uint8")
        if tuple(scale.shape) != (experts, output // bn, contraction // bk) or scale.dtype != torch.float32:
            raise ValueError("routed FP8 scales must be [E, N/bn, K/bk] float32")
    if tuple(local_expert_ids.shape) != (slots,) or local_expert_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("routed FP8 expert ids must be one integer per slot")
    if tuple(owned.shape) != (slots,) or owned.dtype != torch.bool:
        raise ValueError("routed FP8 ownership must be one boolean per slot")
    if result_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("routed FP8 result must be FP32 or BF16")
    ids = local_expert_ids.to(torch.int32).contiguous()
    tensors = [lhs, ids, owned] + [t for pair in weights for t in pair]
    _lib.require_device(*tensors)
    tables = len(weights)
    out = torch.empty((slots, tables, output), dtype=result_dtype, device=lhs.device)
    workspace = torch.empty(_lib.lib().glm_moe_routed_projection_workspace_bytes(slots), dtype=torch.uint8,
                            device=lhs.device)
    bits1, scale1 = weights[1] if tables == 2 else (None, None)
    _lib.call(
        "glm_moe_routed_projection",
        _lib.ptr(lhs), slots, contraction, tables, _lib.ptr(weights[0][0]), _lib.ptr(weights[0][1]),
        _lib.ptr(bits1), _lib.ptr(scale1), experts, output, _lib.ptr(ids), _lib.ptr(owned),
        _lib.F32 if result_dtype == torch.float32 else _lib.BF16, _lib.ptr(out), _lib.ptr(workspace),
        workspace.numel(), _lib.stream_of(lhs),
    )
    return out
