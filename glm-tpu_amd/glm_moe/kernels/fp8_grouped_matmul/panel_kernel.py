"""Expert-relative FP8 projection of the prefill routed experts.

Mirrors ``prefill_panel_fp8_matmul`` of
``glm_tpu/kernels/fp8_grouped_matmul/panel_kernel.py:31-153``: sorted bf16
rows against their panel's local expert, weights decoded per 128x128 block to
bf16, FP32 accumulation in ascending K blocks.  On the GPU the panels are the
work list of the grouped gfx950 kernel: the kernel reads the sorted rows in
place (no packed copy), and unowned rows / invalid plans produce zeros.
"""

from __future__ import annotations

from typing import Any

import torch

from glm_moe import _lib
from glm_moe.kernels.fp8_grouped_matmul.panels import ExpertPanels


def prefill_panel_fp8_matmul(
    lhs: torch.Tensor,
    weight_bits: torch.Tensor,
    scale: torch.Tensor,
    panels: ExpertPanels,
    *,
    result_dtype: Any = torch.float32,
    interpret: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(out [m, n], valid)`` for a plan built on this local expert shard.

    ``interpret`` is accepted for signature parity and ignored: there is one
    implementation, the HIP kernel.
    """
    del interpret
    if lhs.ndim != 2 or weight_bits.ndim != 3 or scale.ndim != 3:
        raise ValueError("panel FP8 ranks must be 2/3/3")
    m, k = lhs.shape
    groups, n, wk = weight_bits.shape
    dtype = result_dtype
    if (
        min(m, k, groups, n) <= 0
        or wk != k
        or k % 128
        or n % 256
        or n // 128 > 128
        or lhs.dtype != torch.bfloat16
        or weight_bits.dtype != torch.uint8
        or scale.dtype != torch.float32
        or tuple(scale.shape) != (groups, n // 128, k // 128)
        or tuple(panels.restore_indices.shape) != (m,)
        or panels.expert_ids.numel() != (m + 31) // 32 + groups - 1
        or dtype not in (torch.float32, torch.bfloat16)
    ):
        raise ValueError("panel FP8 geometry/dtypes disagree with M32/N256/K128")
    _lib.require_device(lhs, weight_bits, scale, panels.expert_ids, panels.row_starts, panels.live_counts)
    out = torch.empty((m, n), dtype=dtype, device=lhs.device)
    _lib.call(
        "glm_moe_panel_fp8_matmul",
        _lib.ptr(lhs), m, k, _lib.ptr(weight_bits), _lib.ptr(scale), groups, n,
        _lib.ptr(panels.expert_ids), _lib.ptr(panels.row_starts), _lib.ptr(panels.live_counts),
        _lib.ptr(panels.active_panels), panels.expert_ids.numel(), _lib.ptr(panels.owned_rows),
        _lib.ptr(panels.valid), _lib.F32 if dtype == torch.float32 else _lib.BF16, _lib.ptr(out),
        _lib.stream_of(lhs),
    )
    return out, panels.valid
