"""Layer bodies of the MoE path (mirrors ``glm_tpu/layers``)."""
