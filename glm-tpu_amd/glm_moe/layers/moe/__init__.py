"""The routed-expert MoE (mirrors ``glm_tpu/layers/moe``)."""

from glm_moe.layers.moe.routed_experts import (
    PrefillRoutes,
    gather_prefill_route_rows,
    group_prefill_routes,
    moe_grouped_routes,
    prefill_moe_from_routes,
    restore_prefill_route_rows,
    routed_experts,
)

__all__ = [
    "PrefillRoutes",
    "gather_prefill_route_rows",
    "group_prefill_routes",
    "moe_grouped_routes",
    "prefill_moe_from_routes",
    "restore_prefill_route_rows",
    "routed_experts",
]
