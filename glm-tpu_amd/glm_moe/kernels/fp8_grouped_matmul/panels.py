"""Device-resident expert-relative M32 panels of the prefill routed experts.

Mirrors ``glm_tpu/kernels/fp8_grouped_matmul/panels.py``: ``ExpertPanels``
(``:14-23``), ``build_expert_panels`` (``:26-83``),
``pack_expert_panel_rows`` (``:86-95``) and ``unpack_expert_panel_rows``
(``:98-104``).  The plan is computed by one HIP workgroup; invalid dynamic
metadata gives no active panels and ``valid=False`` (never an exception).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from glm_moe import _lib

PANEL_ROWS = 32


class ExpertPanels(NamedTuple):
    """Internal plan from ``build_expert_panels``; callers must gate on valid."""

    expert_ids: torch.Tensor  # int32 [capacity]
    row_starts: torch.Tensor  # int32 [capacity]
    live_counts: torch.Tensor  # int32 [capacity]
    active_panels: torch.Tensor  # int32 [] (device scalar)
    restore_indices: torch.Tensor  # int32 [rows]
    owned_rows: torch.Tensor  # bool [rows]
    valid: torch.Tensor  # bool [] (device scalar)


def build_expert_panels(group_sizes: torch.Tensor, group_offset: torch.Tensor, *, rows: int, local_groups: int) -> ExpertPanels:
    """Pack owned experts separately, with at most ceil(rows/32)+G-1 panels."""
    if (
        type(rows) is not int
        or type(local_groups) is not int
        or min(rows, local_groups) <= 0
        or group_sizes.ndim != 1
        or group_sizes.numel() < local_groups
        or group_sizes.dtype != torch.int32
        or (rows + 31) * group_sizes.numel() > 2147483647
    ):
        raise ValueError("expert panels require bounded rows and int32 group counts")
    if group_offset.shape != () or group_offset.dtype != torch.int32:
        raise ValueError("expert panels require an int32 scalar offset")
    _lib.require_device(group_sizes, group_offset)
    device = group_sizes.device
    capacity = (rows + PANEL_ROWS - 1) // PANEL_ROWS + local_groups - 1
    expert_ids = torch.empty(capacity, dtype=torch.int32, device=device)
    row_starts = torch.empty(capacity, dtype=torch.int32, device=device)
    live_counts = torch.empty(capacity, dtype=torch.int32, device=device)
    active = torch.empty((), dtype=torch.int32, device=device)
    restore = torch.empty(rows, dtype=torch.int32, device=device)
    owned = torch.empty(rows, dtype=torch.bool, device=device)
    valid = torch.empty((), dtype=torch.bool, device=device)
    _lib.call(
        "glm_moe_build_expert_panels",
        _lib.ptr(group_sizes), group_sizes.numel(), _lib.ptr(group_offset), rows, local_groups,
        _lib.ptr(expert_ids), _lib.ptr(row_starts), _lib.ptr(live_counts), _lib.ptr(active),
        _lib.ptr(restore), _lib.ptr(owned), _lib.ptr(valid), _lib.stream_of(group_sizes),
    )
    return ExpertPanels(expert_ids, row_starts, live_counts, active, restore, owned, valid)


def _row_bytes(values: torch.Tensor) -> int:
    nbytes = values.shape[-1] * values.element_size()
    if nbytes % 4:
        raise ValueError("panel rows must be a multiple of 4 bytes")
    return nbytes


def pack_expert_panel_rows(values: torch.Tensor, panels: ExpertPanels) -> torch.Tensor:
    """Gather aligned [panel,32,feature] rows; every padding row is zero."""
    if values.ndim != 2 or values.shape[0] != panels.restore_indices.numel():
        raise ValueError("panel packing row geometry disagrees")
    _lib.require_device(values, panels.row_starts, panels.live_counts)
    capacity = panels.expert_ids.numel()
    out = torch.empty((capacity, PANEL_ROWS, values.shape[1]), dtype=values.dtype, device=values.device)
    _lib.call(
        "glm_moe_pack_expert_panel_rows",
        _lib.ptr(values), values.shape[0], _row_bytes(values), _lib.ptr(panels.row_starts),
        _lib.ptr(panels.live_counts), capacity, _lib.ptr(out), _lib.stream_of(values),
    )
    return out


def unpack_expert_panel_rows(values: torch.Tensor, panels: ExpertPanels) -> torch.Tensor:
    """Restore sorted rows with no scatter overlap and zeros for unowned rows."""
    if values.ndim != 3 or tuple(values.shape[:2]) != (panels.expert_ids.numel(), PANEL_ROWS):
        raise ValueError("panel unpacking geometry disagrees")
    _lib.require_device(values, panels.restore_indices, panels.owned_rows)
    rows = panels.restore_indices.numel()
    flat = values.reshape(-1, values.shape[-1])
    out = torch.empty((rows, values.shape[-1]), dtype=values.dtype, device=values.device)
    _lib.call(
        "glm_moe_gather_rows",
        _lib.ptr(flat), flat.shape[0], _row_bytes(flat), _lib.ptr(panels.restore_indices), 1,
        _lib.ptr(panels.owned_rows), rows, _lib.ptr(out), _lib.stream_of(values),
    )
    return out
