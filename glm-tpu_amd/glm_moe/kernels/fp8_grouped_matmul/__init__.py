"""FP8 grouped (routed-expert) matmuls with 128x128 block scales: decode over routed slots
(``kernel``), the prefill panel projection (``panel_kernel``) and expert-panel planning (``panels``)."""
