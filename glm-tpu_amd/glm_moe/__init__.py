"""glm_moe: MI355X (gfx950) backend of glm-tpu's route-grouped FP8 routed-expert MoE path.

Host side of ``libglm_moe.so`` (C ABI in ``include/glm_moe.h``).  The module
layout mirrors the reference package ``glm_tpu``:

* ``glm_moe.layers.moe.routed_experts`` -- ``prefill_moe_from_routes``,
  ``moe_grouped_routes``, ``group_prefill_routes`` and the fused
  ``routed_experts`` pipeline;
* ``glm_moe.kernels.fp8_grouped_matmul`` -- ``fp8_routed_projection``,
  ``prefill_panel_fp8_matmul``, ``build_expert_panels`` and panel packing;
* ``glm_moe.layers.fp8`` -- the e4m3fn block decode;
* ``glm_moe.contracts`` -- ``GlmMoeNumericalContract``.
"""

from glm_moe._lib import LIB_PATH, lib

__all__ = ["LIB_PATH", "lib"]
