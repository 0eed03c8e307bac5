"""Write the golden vectors of the toy configuration (tests/golden/toy_moe.npz).

    python tests/golden/make_golden.py

Toy MoE layer: T=4 tokens, E=8 experts, H=I=256, top-2; activations bf16
N(0,1); sigmoid routing of N(0,1) logits; e4m3fn expert weights from N(0,0.02)
with 128x128 FP32 block scales amax/448 (seed 0).  Expected outputs come from
the CPU oracle (oracle/moe_oracle.py), itself pinned by tests/test_oracle.py.
The reference's own tests hold no value-level vectors for this path, so these
fixtures pin the oracle's outputs over time and give the GPU tests fixed
inputs.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "glm-tpu_amd"))

from glm_moe import synthetic as S  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().with_name("toy_moe.npz")


def build() -> dict[str, np.ndarray]:
    cfg = S.CONFIGS["toy"]
    x = S.hidden_states(cfg, 0)
    ids, w = S.routes(cfg, 0)
    tables = S.host_expert_tables(cfg, 0)
    rng = np.random.default_rng(17)
    shared_gate = O.bf16_round(rng.normal(0, 0.02, (cfg.intermediate, cfg.hidden)).astype(np.float32))
    shared_up = O.bf16_round(rng.normal(0, 0.02, (cfg.intermediate, cfg.hidden)).astype(np.float32))
    shared_down = O.bf16_round(rng.normal(0, 0.02, (cfg.hidden, cfg.intermediate)).astype(np.float32))
    routes = O.group_prefill_routes(ids, num_experts=cfg.experts)
    routed, ok = O.routed_experts(x, ids, w, **tables)
    routed_bf16sum, _ = O.routed_experts(x, ids, w, **tables, route_sum="bfloat16")
    layer, layer_ok = O.moe_layer(x, ids, w, *tables.values(), shared_gate, shared_up, shared_down)
    decode, _ = O.moe_layer(x[:1], ids[:1], w[:1], *tables.values(), shared_gate, shared_up, shared_down,
                            decode=True)
    assert ok and layer_ok
    return {
        "hidden_bits": O.bf16_bits(x),
        "route_indices": ids,
        "route_weights": w,
        **tables,
        "shared_gate_bits": O.bf16_bits(shared_gate),
        "shared_up_bits": O.bf16_bits(shared_up),
        "shared_down_bits": O.bf16_bits(shared_down),
        "sorted_flat_ids": routes.sorted_flat_ids,
        "inverse_permutation": routes.inverse_permutation,
        "group_sizes": routes.group_sizes,
        "routed_bits": O.bf16_bits(routed),
        "routed_bf16sum_bits": O.bf16_bits(routed_bf16sum),
        "layer_bits": O.bf16_bits(layer),
        "decode_layer_bits": O.bf16_bits(decode),
    }


if __name__ == "__main__":
    arrays = build()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
