"""Numerical contract of one sparse GLM MoE layer.

Mirrors ``GlmMoeNumericalContract`` of the reference
(``glm_tpu/config/cache.py:146-218``): same fields, defaults and validation.
On one GPU every mesh axis has size 1, so the layer bodies of this package
use ``stage_size=1`` (``local_experts == num_experts``, the full hidden size
per device) where the reference's 32-chip mesh uses 8.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True, slots=True)
class GlmMoeNumericalContract:
    """Compile-relevant arithmetic contract for one sparse GLM layer."""

    hidden_size: int = 6144
    intermediate_size: int = 2048
    num_experts: int = 256
    top_k: int = 8
    stage_size: int = 4
    routed_scaling_factor: float = 2.5
    fp8_block_shape: tuple[int, int] = (128, 128)
    activation_dtype: str = "bfloat16"
    router_dtype: str = "float32"
    fp8_scale_dtype: str = "float32"
    scoring_function: str = "sigmoid"
    routing_method: str = "noaux_tc"
    routing_tie_policy: str = "jax_lax_top_k_lowest_expert_id"
    reduction_association: str = "top_k_axis_then_stage_psum; routed_and_shared_stacked_not_mixed"

    def __post_init__(self) -> None:
        for field in ("hidden_size", "intermediate_size", "num_experts", "top_k", "stage_size"):
            value = getattr(self, field)
            if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
                raise ValueError(f"{field} must be a positive integer")
        if self.top_k > self.num_experts:
            raise ValueError("top_k cannot exceed num_experts")
        if self.num_experts % self.stage_size:
            raise ValueError("num_experts must divide evenly over the stage")
        if self.intermediate_size % self.stage_size:
            raise ValueError("shared intermediate size must divide over the stage")
        if self.routed_scaling_factor <= 0:
            raise ValueError("routed_scaling_factor must be positive")
        if len(self.fp8_block_shape) != 2 or any(
            not isinstance(item, int) or isinstance(item, bool) or item <= 0 for item in self.fp8_block_shape
        ):
            raise ValueError("fp8_block_shape must contain two positive integers")
        if self.scoring_function != "sigmoid":
            raise ValueError("GLM-5.2 requires sigmoid MoE scoring")
        if self.routing_method != "noaux_tc":
            raise ValueError("GLM-5.2 requires noaux_tc routing")

    @property
    def local_experts(self) -> int:
        return self.num_experts // self.stage_size

    @property
    def local_shared_intermediate(self) -> int:
        return self.intermediate_size // self.stage_size

    def to_dict(self) -> dict[str, Any]:
        return {
            "activation_dtype": self.activation_dtype,
            "fp8_block_shape": list(self.fp8_block_shape),
            "fp8_scale_dtype": self.fp8_scale_dtype,
            "hidden_size": self.hidden_size,
            "intermediate_size": self.intermediate_size,
            "num_experts": self.num_experts,
            "reduction_association": self.reduction_association,
            "routed_scaling_factor": self.routed_scaling_factor,
            "router_dtype": self.router_dtype,
            "routing_method": self.routing_method,
            "routing_tie_policy": self.routing_tie_policy,
            "scoring_function": self.scoring_function,
            "stage_size": self.stage_size,
            "top_k": self.top_k,
        }


def single_gpu_contract(**overrides: Any) -> GlmMoeNumericalContract:
    """The contract of one GPU holding every expert (``stage_size=1``)."""
    overrides.setdefault("stage_size", 1)
    return GlmMoeNumericalContract(**overrides)
