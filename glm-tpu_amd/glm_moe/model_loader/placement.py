"""Checkpoint-name rules of the MoE layer's tensors.

``glm_tpu/model_loader/placement.py``: the source regexes (``:24-39``), the
runtime name of a source tensor (``_runtime_name``, ``:223-232``) and the
expert-parallel coordinate of a routed expert (``:433-435``: coordinate
``e // (E / 8)``, local index ``e % (E / 8)``).  On one GPU every expert is
local (``ep_size = 1``); ``ep_size = 8`` gives one GPU's share of the
reference's eight-way expert axis.
"""

from __future__ import annotations

import re
from typing import NamedTuple

ROUTED = re.compile(
    r"^model\.layers\.(\d+)\.mlp\.experts\.(\d+)\."
    r"(gate_proj|up_proj|down_proj)\.(weight|weight_scale_inv)$"
)
SHARED = re.compile(
    r"^model\.layers\.(\d+)\.mlp\.shared_experts\."
    r"(gate_proj|up_proj|down_proj)\.(weight|weight_scale_inv)$"
)
ROUTER = re.compile(r"^model\.layers\.(\d+)\.mlp\.gate\.(weight|e_score_correction_bias)$")
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")


class RoutedSource(NamedTuple):
    layer: int
    expert: int
    projection: str
    role: str  # "weight" or "weight_scale_inv"


def routed_source(name: str) -> RoutedSource | None:
    """The (layer, expert, projection, role) of a routed-expert source tensor."""
    m = ROUTED.fullmatch(name)
    if m is None:
        return None
    layer, expert, projection, role = m.groups()
    return RoutedSource(int(layer), int(expert), projection, role)


def runtime_name(name: str, dtype: str) -> str:
    """The final-layout name of a source tensor: routed experts lose their
    index (they are stacked along a leading expert axis), FP8 ``.weight``
    becomes ``.weight_bits`` and ``.weight_scale_inv`` becomes ``.scale_inv``."""
    routed = ROUTED.fullmatch(name)
    if routed is not None:
        layer, _, projection, role = routed.groups()
        name = f"model.layers.{layer}.mlp.experts.{projection}.{role}"
    if dtype == "F8_E4M3" and name.endswith(".weight"):
        return name[: -len(".weight")] + ".weight_bits"
    if name.endswith(".weight_scale_inv"):
        return name[: -len(".weight_scale_inv")] + ".scale_inv"
    return name


def expert_coordinate(expert: int, num_experts: int, ep_size: int = 8) -> tuple[int, int]:
    """(expert-axis coordinate, local index) of a routed expert."""
    if ep_size <= 0 or num_experts % ep_size:
        raise ValueError(f"{num_experts} experts do not divide over {ep_size} expert-parallel ranks")
    if not 0 <= expert < num_experts:
        raise ValueError(f"expert {expert} outside [0, {num_experts})")
    local = num_experts // ep_size
    return expert // local, expert % local


def source_names(layer: int, expert: int, projection: str) -> tuple[str, str]:
    """Checkpoint names of one routed expert projection: (weight, weight_scale_inv)."""
    prefix = f"model.layers.{layer}.mlp.experts.{expert}.{projection}"
    return f"{prefix}.weight", f"{prefix}.weight_scale_inv"


def shared_source_names(layer: int, projection: str) -> tuple[str, str]:
    prefix = f"model.layers.{layer}.mlp.shared_experts.{projection}"
    return f"{prefix}.weight", f"{prefix}.weight_scale_inv"


def router_source_names(layer: int) -> tuple[str, str]:
    prefix = f"model.layers.{layer}.mlp.gate"
    return f"{prefix}.weight", f"{prefix}.e_score_correction_bias"
