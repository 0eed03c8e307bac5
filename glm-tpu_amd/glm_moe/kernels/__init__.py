"""HIP kernels of the MoE path (mirrors ``glm_tpu/kernels``)."""
