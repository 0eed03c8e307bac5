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
from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

__all__ = [
    "PrefillRoutes",
    "gather_prefill_route_rows",
    "group_prefill_routes",
    "moe_grouped_routes",
    "prefill_moe_from_routes",
    "restore_prefill_route_rows",
    "route_glm_noaux_tc_logits",
    "routed_experts",
]
