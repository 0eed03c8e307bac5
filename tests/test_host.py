"""CPU tests of the host side: golden fixtures, the C ABI's exported symbols,
and the static refusals that must happen before any device call."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "toy_moe.npz"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def test_golden_vectors_match_the_oracle(golden):
    g = golden
    x = O.bf16_from_bits(g["hidden_bits"])
    tables = {k: g[k] for k in ("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale")}
    routes = O.group_prefill_routes(g["route_indices"], num_experts=8)
    np.testing.assert_array_equal(routes.sorted_flat_ids, g["sorted_flat_ids"])
    np.testing.assert_array_equal(routes.inverse_permutation, g["inverse_permutation"])
    np.testing.assert_array_equal(routes.group_sizes, g["group_sizes"])
    routed, ok = O.routed_experts(x, g["route_indices"], g["route_weights"], **tables)
    assert ok
    np.testing.assert_array_equal(O.bf16_bits(routed), g["routed_bits"])
    shared = [O.bf16_from_bits(g[k]) for k in ("shared_gate_bits", "shared_up_bits", "shared_down_bits")]
    layer, _ = O.moe_layer(x, g["route_indices"], g["route_weights"], *tables.values(), *shared)
    np.testing.assert_array_equal(O.bf16_bits(layer), g["layer_bits"])


def test_golden_shapes_are_the_toy_config(golden):
    assert golden["hidden_bits"].shape == (4, 256)
    assert golden["route_indices"].shape == (4, 2) and golden["route_indices"].dtype == np.int32
    assert golden["gate_bits"].shape == (8, 256, 256) and golden["gate_scale"].shape == (8, 2, 2)
    assert golden["down_bits"].shape == (8, 256, 256)
    # the weights are finite e4m3fn encodings (the loader gate, format.py:307-315)
    for k in ("gate_bits", "up_bits", "down_bits"):
        assert not np.any((golden[k] & 0x7F) == 0x7F)


def test_library_exports_every_declared_symbol():
    from glm_moe import _lib

    declared = _lib.header_functions()
    assert len(declared) >= 15
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(handle, name), name
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"
    assert _lib.lib().glm_moe_abi_version() == 1


def test_ctypes_signatures_match_the_header_parameter_lists():
    """Every binding passes as many arguments as its C declaration takes, and
    every declaration in the header has a definition of the same parameter
    types in the C ABI source."""
    import re
    from pathlib import Path

    from glm_moe import _lib

    root = Path(__file__).resolve().parents[1]

    def declarations(text):
        out = {}
        for m in re.finditer(r"\b(?:int|size_t|const char\*)\s+(glm_moe_\w+)\s*\(([^)]*)\)", text):
            params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
            out[m.group(1)] = [re.sub(r"\s*\w+$", "", p).replace(" ", "") for p in params]
        return out

    header = declarations((root / "include" / "glm_moe.h").read_text())
    source = declarations((root / "glm-tpu_amd" / "csrc" / "capi.hip").read_text())
    assert header and set(header) <= set(source)
    for name, types in header.items():
        assert source[name] == types, name
        _, argtypes = _lib.SIGNATURES[name]
        assert len(argtypes) == len(types), name


def test_workspace_sizes_are_host_computable():
    from glm_moe import _lib

    lib = _lib.lib()
    small = lib.glm_moe_routed_experts_workspace_bytes(1, 8, 256, 6144, 2048)
    big = lib.glm_moe_routed_experts_workspace_bytes(2048, 8, 256, 6144, 2048)
    assert 0 < small < big
    # act [n, I] + y [n, H] bf16 dominate
    assert big >= 2048 * 8 * (6144 + 2048) * 2
    assert lib.glm_moe_routed_experts_workspace_bytes(0, 8, 256, 6144, 2048) == 0
    assert lib.glm_moe_routed_projection_workspace_bytes(8) >= 4 * (3 * 8 + 1)


def test_static_refusals_raise_value_error_through_the_abi():
    from glm_moe import _lib

    lib = _lib.lib()
    null = ctypes.c_void_p(0)
    # K not a multiple of 128 (panel_kernel.py:46-66)
    status = lib.glm_moe_panel_fp8_matmul(null, 41, 1000, null, null, 2, 512, null, null, null, null, 4, null,
                                          null, 0, null, null)
    assert status == _lib.ERR_ARGUMENT
    with pytest.raises(ValueError, match="M32/N256/K128"):
        _lib.check(status)
    assert lib.glm_moe_group_routes(null, 0, 8, 256, null, null, null, null, null, 0, null) == _lib.ERR_ARGUMENT
    assert lib.glm_moe_group_routes(null, 2, 9, 8, null, null, null, null, null, 0, null) == _lib.ERR_ARGUMENT
    status = lib.glm_moe_routed_projection(null, 8, 6144, 3, null, null, null, null, 256, 2048, null, null, 0,
                                           null, null, 0, null)
    assert status == _lib.ERR_ARGUMENT
    status = lib.glm_moe_routed_experts(null, 1, 6144, null, null, 8, 256, 2048, null, null, null, null, null,
                                        null, 0, null, null, null, 0, null)
    assert status == _lib.ERR_ARGUMENT  # null tensors refused before any launch
    # the native FP8 mode is refused on decode shapes, before any device work
    fake = ctypes.c_void_p(256)
    status = lib.glm_moe_routed_experts(fake, 1, 6144, fake, fake, 8, 256, 2048, fake, fake, fake, fake, fake,
                                        fake, _lib.FP8_ACTIVATIONS, fake, fake, fake, 1 << 30, null)
    assert status == _lib.ERR_ARGUMENT
    with pytest.raises(ValueError, match="FP8 activations need a prefill shape"):
        _lib.check(status)
    # the fused layer epilogue needs the shared-expert rows and a finite scale
    status = lib.glm_moe_moe_layer(fake, 1, 6144, fake, fake, 8, 256, 2048, fake, fake, fake, fake, fake, fake, 0,
                                   null, ctypes.c_float(2.5), fake, fake, fake, 1 << 30, null)
    assert status == _lib.ERR_ARGUMENT
    status = lib.glm_moe_moe_layer(fake, 1, 6144, fake, fake, 8, 256, 2048, fake, fake, fake, fake, fake, fake, 0,
                                   fake, ctypes.c_float(float("inf")), fake, fake, fake, 1 << 30, null)
    with pytest.raises(ValueError, match="routed scale must be finite"):
        _lib.check(status)
    # the resident shared expert runs on decode shapes only, and needs I_shared == I
    status = lib.glm_moe_moe_layer_resident(fake, 300, 6144, fake, fake, 8, 256, 2048, fake, fake, fake, fake, fake,
                                            fake, 0, fake, fake, fake, 2048, ctypes.c_float(2.5), fake, fake, fake,
                                            1 << 30, null)
    with pytest.raises(ValueError, match="decode shapes"):
        _lib.check(status)
    status = lib.glm_moe_moe_layer_resident(fake, 1, 6144, fake, fake, 8, 256, 2048, fake, fake, fake, fake, fake,
                                            fake, 0, fake, fake, fake, 1024, ctypes.c_float(2.5), fake, fake, fake,
                                            1 << 30, null)
    with pytest.raises(ValueError, match="intermediate size"):
        _lib.check(status)
    # routing inside the decode layer: logits and route outputs required, <= 256 experts, decode shapes
    def from_logits(tokens, experts, logits, ids):
        return lib.glm_moe_moe_layer_from_logits(fake, tokens, 6144, logits, null, 8, experts, 2048, fake, fake, fake,
                                                 fake, fake, fake, 0, fake, fake, fake, 2048, ctypes.c_float(2.5),
                                                 ids, fake, fake, fake, fake, 1 << 30, null)

    with pytest.raises(ValueError, match="null router logits"):
        _lib.check(from_logits(1, 256, null, fake))
    with pytest.raises(ValueError, match="null router logits"):
        _lib.check(from_logits(1, 256, fake, null))
    with pytest.raises(ValueError, match="at most 256 experts"):
        _lib.check(from_logits(1, 512, fake, fake))
    with pytest.raises(ValueError, match="decode shapes"):
        _lib.check(from_logits(300, 256, fake, fake))
    # the few-row shared expert: 1..8 rows, sizes multiples of 128
    def shared_rows(tokens, hidden, inter, out):
        return lib.glm_moe_shared_expert_rows(fake, tokens, hidden, fake, fake, fake, inter, out, fake, 1 << 30, null)

    with pytest.raises(ValueError, match="1 to 8 rows"):
        _lib.check(shared_rows(9, 6144, 2048, fake))
    with pytest.raises(ValueError, match="1 to 8 rows"):
        _lib.check(shared_rows(4, 6144 + 64, 2048, fake))
    with pytest.raises(ValueError, match="null tensor"):
        _lib.check(shared_rows(4, 6144, 2048, null))
    assert lib.glm_moe_shared_expert_rows_workspace_bytes(4, 2048) == 4 * 2048 * 2
    assert lib.glm_moe_uses_decode_kernels(1, 8, 6144, 2048) == 1
    assert lib.glm_moe_uses_decode_kernels(9, 8, 6144, 2048) == 0
    assert lib.glm_moe_uses_decode_kernels(8, 8, 6144, 4096) == 0


def test_python_api_refuses_bad_geometry_and_cpu_tensors():
    from glm_moe.kernels.fp8_grouped_matmul.kernel import RoutedProjectionConfig, fp8_routed_projection
    from glm_moe.kernels.fp8_grouped_matmul.panels import build_expert_panels
    from glm_moe.layers.moe.routed_experts import group_prefill_routes, routed_experts

    with pytest.raises(ValueError, match="int32"):
        group_prefill_routes(torch.zeros((2, 8), dtype=torch.float32))
    with pytest.raises(ValueError, match="GPU tensors only"):
        group_prefill_routes(torch.zeros((2, 8), dtype=torch.int32))
    with pytest.raises(ValueError):
        build_expert_panels(torch.tensor([1, 0], dtype=torch.int32), torch.tensor([0], dtype=torch.int32),
                            rows=1, local_groups=2)
    with pytest.raises(ValueError):
        build_expert_panels(torch.tensor([1, 0], dtype=torch.int32), torch.tensor(0, dtype=torch.int32),
                            rows=True, local_groups=2)
    with pytest.raises(ValueError, match="VMEM slab"):
        RoutedProjectionConfig(contraction_tile=384)
    with pytest.raises(ValueError):
        RoutedProjectionConfig(write_empty_slot=False)
    lhs = torch.zeros((8, 256), dtype=torch.bfloat16)
    bits = torch.zeros((4, 256, 256), dtype=torch.uint8)
    scale = torch.zeros((4, 2, 2), dtype=torch.float32)
    with pytest.raises(ValueError, match="one or two"):
        fp8_routed_projection(lhs, (), torch.zeros(8, dtype=torch.int32), torch.ones(8, dtype=torch.bool))
    with pytest.raises(ValueError, match="GPU tensors only"):
        fp8_routed_projection(lhs, ((bits, scale),), torch.zeros(8, dtype=torch.int32),
                              torch.ones(8, dtype=torch.bool),
                              config=RoutedProjectionConfig(output_tile=256, contraction_tile=256))
    with pytest.raises(ValueError, match="bf16"):
        routed_experts(lhs.float(), torch.zeros((8, 2), dtype=torch.int32), torch.zeros((8, 2)), bits, scale,
                       bits, scale, bits, scale)
    ids2, w2 = torch.zeros((8, 2), dtype=torch.int32), torch.zeros((8, 2))
    with pytest.raises(ValueError, match="shared expert rows"):
        routed_experts(lhs, ids2, w2, bits, scale, bits, scale, bits, scale, shared=lhs[:4])
    with pytest.raises(ValueError, match="shared expert rows"):
        routed_experts(lhs, ids2, w2, bits, scale, bits, scale, bits, scale, shared=lhs.float())


def test_contract_mirrors_the_reference():
    from glm_moe.contracts import GlmMoeNumericalContract, single_gpu_contract

    c = GlmMoeNumericalContract()  # reference tests/layers/moe/test_router.py:65-76
    assert (c.hidden_size, c.intermediate_size, c.num_experts, c.top_k, c.stage_size) == (6144, 2048, 256, 8, 4)
    assert c.local_experts == 64 and c.local_shared_intermediate == 512
    assert c.routed_scaling_factor == 2.5 and c.fp8_block_shape == (128, 128)
    with pytest.raises(ValueError, match="divide evenly"):
        GlmMoeNumericalContract(num_experts=255)
    assert single_gpu_contract().local_experts == 256


def test_algorithmic_bytes_of_the_decode_config():
    from glm_moe import synthetic as S

    cfg = S.CONFIGS["decode_t1"]
    ids, _ = S.routes(cfg, 0)
    b = S.algorithmic_bytes(cfg, ids)
    assert b["distinct_experts"] == 8
    # 8 experts x 3 x 6144 x 2048 e4m3 bytes + scales + activations: 302.1 MB
    assert abs(b["total"] - 302.1e6) < 0.1e6
    assert S.algorithmic_flops(cfg)["total"] == 2 * 8 * 3 * 6144 * 2048


def test_router_refuses_bad_geometry():
    import torch

    from glm_moe import _lib
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    lib = _lib.lib()
    null = ctypes.c_void_p(0)
    assert lib.glm_moe_route_noaux_tc(null, 4, 8, null, 9, null, null, null) == _lib.ERR_ARGUMENT
    assert lib.glm_moe_route_noaux_tc(null, 4, 2048, null, 8, null, null, null) == _lib.ERR_ARGUMENT
    with pytest.raises(ValueError, match="router_logits must have shape"):
        route_glm_noaux_tc_logits(torch.zeros(8), torch.zeros(8))
    with pytest.raises(ValueError, match="correction_bias"):
        route_glm_noaux_tc_logits(torch.zeros(2, 8), torch.zeros(7))
    with pytest.raises(ValueError, match="top_k must be in"):
        route_glm_noaux_tc_logits(torch.zeros(2, 8), torch.zeros(8), top_k=9)
    with pytest.raises(ValueError, match="GPU tensors only"):
        route_glm_noaux_tc_logits(torch.zeros(2, 8), torch.zeros(8), top_k=2)


def test_decode_kernels_take_at_most_64_routes():
    from glm_moe.layers.moe.routed_experts import uses_decode_kernels

    assert uses_decode_kernels(1, 8, 6144, 2048)
    assert uses_decode_kernels(8, 8, 512, 256)       # 64 routes
    assert not uses_decode_kernels(9, 8, 512, 256)   # 72 routes: route plan + grouped GEMMs
    assert uses_decode_kernels(64, 1, 512, 256)
    assert not uses_decode_kernels(65, 1, 512, 256)


def test_bench_reads_measured_traffic_from_the_profiles():
    """bench.py's roofline `traffic` comes from the profiles/*_hbm_traffic.md
    summaries (their `bench-traffic:` lines), one per measured config."""
    import bench
    from glm_moe import synthetic as S

    found = bench.measured_traffic()
    assert "decode_t1" in found
    for name, rec in found.items():
        base, _, mode = name.partition(":")
        assert base in S.CONFIGS and mode in ("", "fp8"), name
        assert rec["bytes"] > 0 and rec["source"].startswith("profiles/")
