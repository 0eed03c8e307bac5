"""GPU parity of libglm_moe against the CPU oracle (oracle/moe_oracle.py).

Integer work (route grouping, panel plans, FP8 decode) must be bit-exact;
projections and the MoE outputs must be within the north-star tolerance
``max|y - y_ref| <= 2e-2`` and ``mean|y - y_ref| / mean|y_ref| <= 5e-3`` of the
oracle's bf16 output (kernel primitives use the reference's own tolerances,
tests/kernels/test_fp8_panel_matmul.py:131-137).  Every call goes through the
C ABI of libglm_moe.so.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import closeness
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "toy_moe.npz"
MAX_ABS = closeness.MAX_ABS
MEAN_REL = closeness.MEAN_REL
TABLE_KEYS = ("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale")


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bf16_dev(values_f32, device):
    return torch.from_numpy(np.ascontiguousarray(values_f32, dtype=np.float32)).to(torch.bfloat16).to(device)


def host_f32(t):
    return t.float().cpu().numpy()


def bf16_bits_of(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def assert_moe_close(got, ref, **bounds):
    """The north-star tolerance with the rounding-flip allowance of
    ``closeness.check`` (recorded and printed in the session summary)."""
    return closeness.check(got, ref, **bounds)


# ----------------------------------------------------------------------------- FP8 decode
def test_decode_fp8_table_is_bit_exact(device):
    from glm_moe.layers.fp8 import decode_fp8_table

    rng = np.random.default_rng(1)
    bits = np.tile(np.arange(256, dtype=np.uint8), (256, 384 // 256 + 1))[:, :384].copy()
    rng.shuffle(bits, axis=1)
    scale = rng.uniform(0.001, 9.0, (2, 3)).astype(np.float32)
    scale[0, 1], scale[1, 2], scale[1, 0] = 0.0, 3.25, 1.0e-30  # zero, exact, subnormal products
    got = decode_fp8_table(dev(bits, device), dev(scale, device))
    ref = O.decode_fp8_table(bits, scale)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(host_f32(got)), nan)
    np.testing.assert_array_equal(bf16_bits_of(got)[~nan], O.bf16_bits(ref)[~nan])
    # non-default blocks (reference tests/layers/moe/test_router.py:84-97)
    small = decode_fp8_table(dev(np.full((4, 6), 0x38, np.uint8), device),
                             dev(np.array([[1, 2], [3, 4]], np.float32), device), block_shape=(2, 3))
    np.testing.assert_array_equal(host_f32(small), [[1, 1, 1, 2, 2, 2]] * 2 + [[3, 3, 3, 4, 4, 4]] * 2)


# ----------------------------------------------------------------------------- SwiGLU
def test_swiglu_bf16_every_gate_value_is_bit_exact(device):
    """The epilogues' SwiGLU on every bf16 bit pattern as the gate (zeros,
    subnormals, infinities and NaNs included) against the oracle's op-by-op bf16
    SwiGLU: u = 1 isolates bf16(g * bf16(sigmoid(g))), random bf16 u adds the
    last product.  Since the kernels round g to bf16 first, this covers every
    gate value they can see."""
    from glm_moe.layers.moe.routed_experts import swiglu_bf16

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    g = (bits.astype(np.uint32) << 16).view(np.float32)
    g_dev = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(device)
    rng = np.random.default_rng(7)
    for u in (np.ones_like(g), O.bf16_round(rng.standard_normal(g.size).astype(np.float32) * 3)):
        u_dev = bf16_dev(u, device)
        # whole tensors (8 values a thread) and a misaligned, odd-length view (one a thread)
        for sl in (slice(None), slice(1, None)):
            got = swiglu_bf16(g_dev[sl], u_dev[sl])
            ref = O.swiglu_bf16(g[sl], u[sl])
            nan = np.isnan(ref)
            np.testing.assert_array_equal(np.isnan(host_f32(got)), nan)
            np.testing.assert_array_equal(bf16_bits_of(got)[~nan], O.bf16_bits(ref)[~nan])


# ----------------------------------------------------------------------------- route grouping
ROUTE_CASES = [(rows, conc) for rows in (1, 17, 128, 512) for conc in (False, True)]


@pytest.mark.parametrize("rows,concentrated", ROUTE_CASES)
def test_group_routes_is_bit_exact(device, rows, concentrated):
    from glm_moe.layers.moe.routed_experts import gather_prefill_route_rows, group_prefill_routes, \
        restore_prefill_route_rows

    rng = np.random.default_rng(183)
    count = 32 if concentrated else 256
    ids = np.stack([rng.choice(count, 8, replace=False) for _ in range(rows)]).astype(np.int32)
    got = group_prefill_routes(dev(ids, device))
    ref = O.group_prefill_routes(ids)
    np.testing.assert_array_equal(got.sorted_flat_ids.cpu().numpy(), ref.sorted_flat_ids)
    np.testing.assert_array_equal(got.inverse_permutation.cpu().numpy(), ref.inverse_permutation)
    np.testing.assert_array_equal(got.group_sizes.cpu().numpy(), ref.group_sizes)
    assert bool(got.valid) is True
    hidden = O.bf16_round(np.arange(rows * 4, dtype=np.float32).reshape(rows, 4))
    gathered = gather_prefill_route_rows(bf16_dev(hidden, device), got, top_k=8)
    np.testing.assert_array_equal(host_f32(gathered), O.gather_prefill_route_rows(hidden, ref, top_k=8))
    values = np.arange(rows * 8 * 3, dtype=np.float32).reshape(rows * 8, 3)
    restored = restore_prefill_route_rows(dev(values[ref.sorted_flat_ids], device), got, top_k=8)
    np.testing.assert_array_equal(restored.cpu().numpy(), values.reshape(rows, 8, 3))


@pytest.mark.parametrize("seed", [0, 1])
def test_group_routes_zipf_8192_is_bit_exact(device, seed):
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import group_prefill_routes

    ids, _ = S.routes(S.CONFIGS["prefill_t8192_zipf"], seed)
    got = group_prefill_routes(dev(ids, device))
    ref = O.group_prefill_routes(ids)
    np.testing.assert_array_equal(got.sorted_flat_ids.cpu().numpy(), ref.sorted_flat_ids)
    np.testing.assert_array_equal(got.inverse_permutation.cpu().numpy(), ref.inverse_permutation)
    np.testing.assert_array_equal(got.group_sizes.cpu().numpy(), ref.group_sizes)
    assert int(ref.group_sizes.max()) > 1000  # the skew the config asks for


@pytest.mark.parametrize("top_k,rows,invalid", [(6, 700, False), (8, 1000, True), (5, 3000, False)])
def test_group_routes_many_chunks_is_bit_exact(device, top_k, rows, invalid):
    """Route sets of several 2048-route chunks (whole rows: a chunk of 6-wide rows
    holds 2046 routes), with and without an invalid id in a late chunk."""
    from glm_moe.layers.moe.routed_experts import group_prefill_routes

    rng = np.random.default_rng(top_k * rows)
    ids = np.stack([rng.choice(64, top_k, replace=False) for _ in range(rows)]).astype(np.int32)
    if invalid:
        ids[rows - 3, 1] = 64
    got = group_prefill_routes(dev(ids, device), num_experts=64)
    ref = O.group_prefill_routes(ids, num_experts=64)
    np.testing.assert_array_equal(got.sorted_flat_ids.cpu().numpy(), ref.sorted_flat_ids)
    np.testing.assert_array_equal(got.inverse_permutation.cpu().numpy(), ref.inverse_permutation)
    np.testing.assert_array_equal(got.group_sizes.cpu().numpy(), ref.group_sizes)
    assert bool(got.valid) == bool(ref.valid) == (not invalid)


@pytest.mark.parametrize("bad", [-1, 256, 0, 2**31 - 1])
def test_group_routes_invalid_ids_match_reference_metadata(device, bad):
    from glm_moe.layers.moe.routed_experts import group_prefill_routes

    ids = np.tile(np.arange(8, dtype=np.int32), (3, 1))
    ids[1, 7] = bad
    got = group_prefill_routes(dev(ids, device))
    ref = O.group_prefill_routes(ids)
    assert not bool(got.valid) and not ref.valid
    np.testing.assert_array_equal(got.sorted_flat_ids.cpu().numpy(), ref.sorted_flat_ids)
    np.testing.assert_array_equal(got.group_sizes.cpu().numpy(), ref.group_sizes)


# ----------------------------------------------------------------------------- panels
def _panels_equal(got, ref):
    np.testing.assert_array_equal(got.expert_ids.cpu().numpy(), ref.expert_ids)
    np.testing.assert_array_equal(got.row_starts.cpu().numpy(), ref.row_starts)
    np.testing.assert_array_equal(got.live_counts.cpu().numpy(), ref.live_counts)
    assert int(got.active_panels) == ref.active_panels
    np.testing.assert_array_equal(got.restore_indices.cpu().numpy(), ref.restore_indices)
    np.testing.assert_array_equal(got.owned_rows.cpu().numpy(), ref.owned_rows)
    assert bool(got.valid) == ref.valid


@pytest.mark.parametrize("offset", [0, 2, 4])
def test_build_expert_panels_is_bit_exact(device, offset):
    from glm_moe.kernels.fp8_grouped_matmul.panels import build_expert_panels, pack_expert_panel_rows, \
        unpack_expert_panel_rows

    counts = np.array([1, 31, 32, 33, 0, 7], np.int32)
    m = int(counts.sum())
    got = build_expert_panels(dev(counts, device), torch.tensor(offset, dtype=torch.int32, device=device),
                              rows=m, local_groups=2)
    ref = O.build_expert_panels(counts, offset, rows=m, local_groups=2)
    _panels_equal(got, ref)
    x = np.arange(m * 4, dtype=np.float32).reshape(m, 4)
    packed = pack_expert_panel_rows(dev(x, device), got)
    np.testing.assert_array_equal(packed.cpu().numpy(), O.pack_expert_panel_rows(x, ref))
    live = np.arange(32)[None, :] < ref.live_counts[:, None]
    poisoned = torch.where(dev(live, device)[..., None], packed, torch.full_like(packed, float("nan")))
    np.testing.assert_array_equal(unpack_expert_panel_rows(poisoned, got).cpu().numpy(),
                                  O.unpack_expert_panel_rows(O.pack_expert_panel_rows(x, ref), ref))


@pytest.mark.parametrize("counts,offset", [
    ([19, 0, 0, 0], -1), ([19, 0, 0, 0], 3), ([19, 0, 0, 0], 2147483647),
    ([19, -1, 0, 0], 0), ([18, 0, 0, 0], 0), ([2147483647, 0, 0, 0], 0), ([0, 129, 0, 0], 0),
])
def test_build_expert_panels_edge_cases_are_bit_exact(device, counts, offset):
    from glm_moe.kernels.fp8_grouped_matmul.panels import build_expert_panels

    rows = 129 if counts[1] == 129 else 19
    local = 4 if rows == 129 else 2
    c = np.array(counts, np.int32)
    got = build_expert_panels(dev(c, device), torch.tensor(offset, dtype=torch.int32, device=device),
                              rows=rows, local_groups=local)
    _panels_equal(got, O.build_expert_panels(c, offset, rows=rows, local_groups=local))


# ----------------------------------------------------------------------------- panel matmul
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_panel_matmul_matches_oracle(device, dtype):
    from glm_moe.kernels.fp8_grouped_matmul.panel_kernel import prefill_panel_fp8_matmul
    from glm_moe.kernels.fp8_grouped_matmul.panels import build_expert_panels

    rng = np.random.default_rng(911)  # reference tests/kernels/test_fp8_panel_matmul.py:105-137
    counts = np.array([1, 33, 7, 0], np.int32)
    m, k, n = 41, 1152, 512
    x = O.bf16_round(rng.normal(0, 0.2, (m, k)).astype(np.float32))
    bits = torch.from_numpy(rng.normal(0, 0.15, (2, n, k)).astype(np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    scales = rng.uniform(0.1, 2.0, (2, 4, 9)).astype(np.float32)
    scales[0, 1, 8] = 0
    scales[1, 3, 8] = 3.25
    plan = build_expert_panels(dev(counts, device), torch.tensor(1, dtype=torch.int32, device=device), rows=m,
                               local_groups=2)
    got, ok = prefill_panel_fp8_matmul(bf16_dev(x, device), dev(bits, device), dev(scales, device), plan,
                                       result_dtype=dtype)
    assert bool(ok) and got.dtype == dtype
    name = "float32" if dtype == torch.float32 else "bfloat16"
    ref, _ = O.panel_fp8_matmul(x, bits, scales, O.build_expert_panels(counts, 1, rows=m, local_groups=2),
                                result_dtype=name)
    actual = host_f32(got)
    owned = np.zeros(m, bool)
    owned[1:41] = True
    np.testing.assert_array_equal(actual[~owned], 0)
    if dtype == torch.float32:
        np.testing.assert_allclose(actual, ref, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_allclose(actual, ref, rtol=2**-7, atol=2**-9)


def test_panel_matmul_closed_form_and_invalid_plan(device):
    from glm_moe.kernels.fp8_grouped_matmul.panel_kernel import prefill_panel_fp8_matmul
    from glm_moe.kernels.fp8_grouped_matmul.panels import build_expert_panels

    zero = torch.tensor(0, dtype=torch.int32, device=device)
    plan = build_expert_panels(dev(np.array([0, 129, 0, 0], np.int32), device), zero, rows=129, local_groups=4)
    x = torch.ones((129, 128), dtype=torch.bfloat16, device=device)
    w = torch.full((4, 256, 128), 0x38, dtype=torch.uint8, device=device)  # 1.0
    s = torch.ones((4, 2, 1), dtype=torch.float32, device=device)
    s[1, 1, 0] = 0
    value, ok = prefill_panel_fp8_matmul(x, w, s, plan)
    assert bool(ok)
    v = host_f32(value)
    np.testing.assert_array_equal(v[:, :128], 128)
    np.testing.assert_array_equal(v[:, 128:], 0)
    # invalid metadata: no work at all, even with NaN operands (test_fp8_panel_matmul.py:53-78)
    m = 19
    xn = torch.full((m, 128), float("nan"), dtype=torch.bfloat16, device=device)
    wn = torch.full((2, 256, 128), 127, dtype=torch.uint8, device=device)
    sn = torch.full((2, 2, 1), float("nan"), dtype=torch.float32, device=device)
    for counts, offset in (([19, 0, 0, 0], 2), ([19, 0, 0, 0], -1), ([18, 0, 0, 0], 0)):
        p = build_expert_panels(dev(np.array(counts, np.int32), device),
                                torch.tensor(offset, dtype=torch.int32, device=device), rows=m, local_groups=2)
        value, ok = prefill_panel_fp8_matmul(xn, wn, sn, p)
        np.testing.assert_array_equal(host_f32(value), 0)
        assert bool(ok) == (offset == 2)


# ----------------------------------------------------------------------------- routed projection
@pytest.mark.parametrize("tables", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_routed_projection_matches_oracle(device, tables, dtype):
    from glm_moe.kernels.fp8_grouped_matmul.kernel import RoutedProjectionConfig, fp8_routed_projection

    rng = np.random.default_rng(41)
    e, n, k, slots = 8, 512, 1152, 8
    x = O.bf16_round(rng.normal(0, 0.2, (slots, k)).astype(np.float32))
    pairs = []
    for _ in range(tables):
        bits = torch.from_numpy(rng.normal(0, 0.15, (e, n, k)).astype(np.float32)).to(
            torch.float8_e4m3fn).view(torch.uint8).numpy()
        scales = rng.uniform(0.1, 2.0, (e, n // 128, k // 128)).astype(np.float32)
        pairs.append((bits, scales))
    ids = np.array([3, -2, 9, 1, 0, 7, 7, 5], np.int32)
    owned = np.array([True, True, True, False, True, True, False, True])
    got = fp8_routed_projection(
        bf16_dev(x, device), tuple((dev(b, device), dev(s, device)) for b, s in pairs), dev(ids, device),
        dev(owned, device), config=RoutedProjectionConfig(output_tile=256, contraction_tile=128), result_dtype=dtype)
    name = "float32" if dtype == torch.float32 else "bfloat16"
    ref = O.routed_projection(x, tuple(pairs), ids, owned, result_dtype=name)
    actual = host_f32(got)
    np.testing.assert_array_equal(actual[~owned], 0)
    if dtype == torch.float32:
        np.testing.assert_allclose(actual, ref, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_allclose(actual, ref, rtol=2**-7, atol=2**-9)


# ----------------------------------------------------------------------------- routed experts
@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def _device_tables(tables, device):
    return {k: dev(tables[k], device) for k in TABLE_KEYS}


def test_routed_experts_toy_golden(device, golden):
    from glm_moe.layers.moe.routed_experts import routed_experts

    g = golden
    x = dev(g["hidden_bits"].view(np.int16), device).view(torch.bfloat16)
    ids, w = dev(g["route_indices"], device), dev(g["route_weights"], device)
    t = _device_tables(g, device)
    out, ok = routed_experts(x, ids, w, *(t[k] for k in TABLE_KEYS))
    assert bool(ok)
    print("toy fp32-sum:", assert_moe_close(host_f32(out), O.bf16_from_bits(g["routed_bits"])))
    out16, _ = routed_experts(x, ids, w, *(t[k] for k in TABLE_KEYS), route_sum="bfloat16")
    print("toy bf16-sum:", assert_moe_close(host_f32(out16), O.bf16_from_bits(g["routed_bf16sum_bits"])))


def test_layers_toy_golden(device, golden):
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import moe_grouped_routes, prefill_moe_from_routes

    g = golden
    contract = single_gpu_contract(hidden_size=256, intermediate_size=256, num_experts=8, top_k=2)
    x = dev(g["hidden_bits"].view(np.int16), device).view(torch.bfloat16)
    ids, w = dev(g["route_indices"], device), dev(g["route_weights"], device)
    t = _device_tables(g, device)
    shared = [dev(g[k].view(np.int16), device).view(torch.bfloat16)
              for k in ("shared_gate_bits", "shared_up_bits", "shared_down_bits")]
    out, ok = prefill_moe_from_routes(x, ids, w, *(t[k] for k in TABLE_KEYS), *shared, contract=contract)
    assert bool(ok)
    print("toy prefill layer:", assert_moe_close(host_f32(out), O.bf16_from_bits(g["layer_bits"])))
    dec = moe_grouped_routes(x[:1], ids[:1], w[:1], *(t[k] for k in TABLE_KEYS), contract=contract,
                             shared_bf16=tuple(shared))
    print("toy decode layer:", assert_moe_close(host_f32(dec), O.bf16_from_bits(g["decode_layer_bits"])))


# ----------------------------------------------------------------------------- fused layer epilogue
# glm_moe_moe_layer: out = bf16(bf16(routed * bf16(2.5)) + shared), fused into the
# kernel that finishes the route sum (routed_experts.py:125, :303).  It must equal
# the same epilogue done by torch bf16 ops after the routed call, bit for bit.
@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,route_sum", [
    (1, 16, 512, 256, 8, "bfloat16"),   # decode kernels, the decode body's bf16 route sum
    (3, 16, 512, 256, 4, "float32"),    # decode kernels, the prefill body's FP32 route sum
    (300, 64, 256, 512, 6, "float32"),  # route plan + grouped GEMMs + combine kernel
    (512, 16, 512, 256, 8, "float32"),  # prefill kernels (wide tiles)
])
def test_fused_layer_epilogue_equals_unfused(device, tokens, experts, hidden, inter, top_k, route_sum):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(tokens, experts, hidden, inter, top_k, 0.0, seed=tokens + 40)
    t = _device_tables(tables, device)
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    rng = np.random.default_rng(tokens)
    shared_f32 = (rng.standard_normal((tokens, hidden)) * 0.05).astype(np.float32)
    shared = bf16_dev(shared_f32, device)
    routed, ok = routed_experts(*args, route_sum=route_sum)
    want = routed * torch.tensor(2.5, dtype=torch.bfloat16, device=device) + shared
    got, ok_fused = routed_experts(*args, route_sum=route_sum, shared=shared, routed_scale=2.5)
    assert bool(ok) and bool(ok_fused)
    np.testing.assert_array_equal(bf16_bits_of(got), bf16_bits_of(want))
    # and against the oracle's layer epilogue on its own routed output
    ref_routed, _ = O.routed_experts(x, ids, w, **tables, route_sum=route_sum)
    ref = O.bf16_round(O.bf16_round(ref_routed * np.float32(2.5)) + O.bf16_round(shared_f32))
    print(cfg, assert_moe_close(host_f32(got), ref))


@pytest.mark.parametrize("tokens,top_k", [(2, 4), (300, 4)])  # decode kernels / combine kernel
def test_fused_layer_nonfinite_output_clears_health(device, tokens, top_k):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(tokens, 16, 512, 256, top_k, 0.0, seed=7)
    t = _device_tables(tables, device)
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    shared = torch.zeros((tokens, 512), dtype=torch.bfloat16, device=device)
    _, ok = routed_experts(*args, shared=shared)
    assert bool(ok)
    shared[tokens - 1, 300] = float("inf")
    out, ok = routed_experts(*args, shared=shared)
    assert not bool(ok)  # routed_experts.py:126: the output must be finite
    assert torch.isinf(out[tokens - 1, 300].float())
    shared[tokens - 1, 300] = 0.0
    _, ok = routed_experts(*args, shared=shared)
    assert bool(ok)  # health is recomputed on every call


# ----------------------------------------------------------------------------- resident shared expert
# glm_moe_moe_layer_resident: the bf16 shared expert inside the two decode
# kernels; the whole layer against the oracle's moe_layer (routed_experts.py:
# 119-127 / 269-304) and against the hipBLASLt shared expert + fused epilogue.
@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,decode", [
    (1, 16, 512, 256, 8, True),     # the decode body: bf16 route sum
    (3, 16, 512, 256, 4, False),    # the prefill body on few rows: FP32 sum
    (8, 32, 768, 384, 8, False),    # 64 routes, the decode kernels' limit
    (2, 8, 6144, 2048, 4, True),    # production hidden / intermediate sizes
    (5, 16, 512, 256, 8, False),    # two shared token groups (4 + 1 tokens)
    (8, 8, 512, 256, 8, True),      # every token selects every expert: units of two routes, two shared groups
    (4, 256, 6144, 2048, 8, True),  # the batched decode layer (decode_t4 shape)
])
def test_resident_shared_expert_layer(device, tokens, experts, hidden, inter, top_k, decode):
    from glm_moe.layers.moe.routed_experts import _shared_swiglu, routed_experts, uses_decode_kernels

    assert uses_decode_kernels(tokens, top_k, hidden, inter)
    cfg, x, ids, w, tables = _small_case(tokens, experts, hidden, inter, top_k, 0.0, seed=tokens + 90)
    t = _device_tables(tables, device)
    rng = np.random.default_rng(tokens)
    # weights scaled so that the shared output is O(1) at every size (the absolute
    # max-abs bound is meaningful only against outputs of that magnitude)
    shared_f32 = [(rng.standard_normal(shape) * std).astype(np.float32)
                  for shape, std in (((inter, hidden), hidden ** -0.5), ((inter, hidden), hidden ** -0.5),
                                     ((hidden, inter), 2 * inter ** -0.5))]
    shared_dev = [bf16_dev(a, device) for a in shared_f32]
    kw = dict(route_sum="bfloat16", check_weights=False, drop_unowned=True) if decode else {}
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    got, ok = routed_experts(*args, shared_tables=tuple(shared_dev), **kw)
    ref, ref_ok, mag = O.moe_layer(x, ids, w, **tables, shared_gate=shared_f32[0], shared_up=shared_f32[1],
                                   shared_down=shared_f32[2], decode=decode, return_magnitude=True)
    assert bool(ok) == ref_ok
    print(cfg, "vs oracle:", assert_moe_close(host_f32(got), ref, magnitude=mag, flip_ulps=closeness.LAYER_FLIP_ULPS,
                                              max_flips=closeness.layer_max_flips(ref.size)))
    # the same layer with the shared expert on hipBLASLt: equal up to FP32 summation order
    shared = _shared_swiglu(args[0], *shared_dev)
    other, _ = routed_experts(*args, shared=shared, **kw)
    print("vs hipBLASLt shared expert:", assert_moe_close(host_f32(got), host_f32(other), magnitude=mag,
                                                          label="vs hipBLASLt", flip_ulps=closeness.LAYER_FLIP_ULPS,
                                                          max_flips=closeness.layer_max_flips(ref.size)))
    again, _ = routed_experts(*args, shared_tables=tuple(shared_dev), **kw)
    np.testing.assert_array_equal(bf16_bits_of(again), bf16_bits_of(got))  # deterministic


def test_resident_shared_expert_nonfinite_clears_health(device):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(2, 16, 512, 256, 4, 0.0, seed=5)
    t = _device_tables(tables, device)
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    shared = [torch.zeros(s, dtype=torch.bfloat16, device=device) for s in ((256, 512), (256, 512), (512, 256))]
    _, ok = routed_experts(*args, shared_tables=tuple(shared))
    assert bool(ok)
    shared[2][17, 3] = float("inf")   # shared down row 17: one output column of every token
    shared[0][3, :] = 1.0             # a non-zero activation in intermediate row 3
    shared[1][3, :] = 1.0
    out, ok = routed_experts(*args, shared_tables=tuple(shared))
    assert not bool(ok) and not bool(torch.isfinite(out[:, 17].float()).all())


def _small_case(tokens, experts, hidden, inter, top_k, zipf, seed):
    from glm_moe import synthetic as S

    cfg = S.MoeConfig("case", tokens, experts, hidden, inter, top_k, zipf)
    x = S.hidden_states(cfg, seed)
    ids, w = S.routes(cfg, seed)
    return cfg, x, ids, w, S.host_expert_tables(cfg, seed)


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,zipf", [
    (3, 16, 512, 256, 4, 0.0),      # 12 routes over several experts: the decode kernels
    (8, 64, 512, 256, 8, 0.0),      # 64 routes: the decode kernels' maximum
    (9, 64, 512, 256, 8, 0.0),      # 72 routes: the first size on the grouped path (prefill kernel)
    (64, 32, 768, 384, 8, 0.0),     # prefill kernel, multi-route experts
    (12, 128, 384, 256, 8, 0.0),    # H % 256 != 0, no prefill kernel: split-K tiles of <= 4 routes
    (40, 64, 384, 256, 8, 0.0),     # H % 256 != 0: split-K tiles of <= 16 routes
    (512, 16, 512, 256, 8, 1.2),    # wide path, skewed: multi-tile experts
    (300, 64, 256, 512, 6, 0.0),    # wide path, ragged tiles
    (64, 4, 8448, 256, 2, 0.0),     # K/128 = 66 > 64: the 64-bit-offset wide kernel instead of the prefill one
    (512, 256, 768, 256, 8, 0.0),   # prefill path over 256 experts of ~16 routes (one tile each)
    (1536, 256, 768, 256, 8, 1.2),  # 256 experts, skewed: single- and multi-tile experts side by side
    (2, 1024, 256, 128, 8, 0.0),    # the most experts a plan takes (1024): decode kernels
    (8, 8, 512, 256, 8, 0.0),       # decode kernels, every expert selected by every token (4 units each)
    (6, 12, 768, 512, 4, 1.2),      # decode kernels, skewed: experts of 1-6 routes
    (600, 1024, 256, 128, 8, 0.5),  # 1024 experts on the route plan and the prefill kernels
    (700, 384, 256, 128, 8, 0.8),   # 384 experts: the plan ranks experts two threads apiece, skewed ties
    (200, 300, 256, 128, 8, 0.0),   # 300 experts on the one-workgroup plan (1600 routes)
])
def test_routed_experts_matches_oracle(device, tokens, experts, hidden, inter, top_k, zipf):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(tokens, experts, hidden, inter, top_k, zipf, seed=tokens)
    t = _device_tables(tables, device)
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    ref, ref_ok = O.routed_experts(x, ids, w, **tables)
    assert bool(ok) == ref_ok
    print(cfg, assert_moe_close(host_f32(out), ref))


# Stripe runs: an FP8 prefill work item of the down projection on 256-row
# stripes runs up to 4 weight stripes of one tile in one continuous ring when K
# has at least 4 blocks.  H = 1280 gives 5 such stripes (a run of 4, then a
# run of 1); H = 1536 runs tall stripes (512 rows, one a work item) in both
# modes.  I = 512 gives K = 4 blocks, where the rings' 3-block look-ahead
# reaches into the next stripe's first blocks; the skewed routing of these
# seeds gives tiles of every column-group count 1 .. 8 (the 1-2 group bf16
# tiles run 4-deep rings) and multi-tile experts.
@pytest.mark.parametrize("activations", ["bfloat16", "float8_e4m3fn"])
@pytest.mark.parametrize("hidden,inter,seed", [(1536, 512, 517), (1536, 1024, 1029), (1280, 512, 517),
                                               (1280, 1024, 1029)])
def test_prefill_stripe_runs_match_oracle(device, activations, hidden, inter, seed):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(600, 16, hidden, inter, 8, 0.9, seed=seed)
    counts = np.bincount(ids.ravel(), minlength=16)
    groups = {int((c % 128 + 15) // 16) for c in counts} | {8 for c in counts if c >= 128}
    assert groups >= set(range(1, 9)) and (counts > 256).any()
    t = _device_tables(tables, device)
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                             activations=activations)
    ref, ref_ok = O.routed_experts(x, ids, w, **tables, activations=activations)
    assert bool(ok) == ref_ok
    close = assert_moe_close if activations == "bfloat16" else assert_fp8_close
    print(cfg, activations, close(host_f32(out), ref))


# Stripe geometries at their edges, both modes: tall down stripes with K = 1
# block (I = 128, the two-slot ring's look-ahead past the end from the first
# block on) beside 256-row gate/up stripes; tall gate/up with K = 2 blocks
# (H = 256) beside 256-row down stripes; tiles of 5..8 column groups on tall
# stripes in both projections (~75-120 routes an expert: the half-stage
# variants of the bf16 kernel, scales of two registers a lane in the FP8 one).
@pytest.mark.parametrize("activations", ["bfloat16", "float8_e4m3fn"])
@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,zipf", [
    (200, 16, 512, 128, 4, 0.5),
    (300, 16, 256, 512, 4, 0.0),
    (600, 16, 512, 256, 2, 0.0),
    (480, 8, 1024, 256, 2, 0.0),
])
def test_prefill_stripe_geometry_edges_match_oracle(device, activations, tokens, experts, hidden, inter, top_k,
                                                    zipf):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(tokens, experts, hidden, inter, top_k, zipf, seed=tokens + 7)
    t = _device_tables(tables, device)
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                             activations=activations)
    ref, ref_ok = O.routed_experts(x, ids, w, **tables, activations=activations)
    assert bool(ok) == ref_ok
    close = assert_moe_close if activations == "bfloat16" else assert_fp8_close
    print(cfg, activations, np.bincount(ids.ravel(), minlength=experts).tolist(), close(host_f32(out), ref))


# Seeded random geometries (H, I, E, top-k, T, skew, mode): the stripe and tile
# choices (tall or 256-row stripes, wide listings, split-K shapes, decode
# kernels) all meet the oracle, whatever combination a caller's shape picks.
def _random_geometry(i):
    rng = np.random.default_rng(9000 + i)
    hidden = int(rng.choice([256, 512, 768, 1024, 1280, 1536]))
    inter = int(rng.choice([128, 256, 384, 512]))
    experts = int(rng.choice([4, 8, 16, 32, 64]))
    top_k = int(rng.integers(1, min(experts, 8) + 1))
    tokens = int(rng.integers(9, 1500))
    zipf = float(rng.choice([0.0, 0.0, 0.8, 1.5]))
    activations = str(rng.choice(["bfloat16", "float8_e4m3fn"]))
    return tokens, experts, hidden, inter, top_k, zipf, activations


@pytest.mark.parametrize("case", range(12))
def test_prefill_random_geometries_match_oracle(device, case):
    from glm_moe.layers.moe.routed_experts import routed_experts

    tokens, experts, hidden, inter, top_k, zipf, activations = _random_geometry(case)
    cfg, x, ids, w, tables = _small_case(tokens, experts, hidden, inter, top_k, zipf, seed=case + 77)
    t = _device_tables(tables, device)
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    if activations != "bfloat16" and tokens * top_k <= 64:
        # the FP8 mode runs on the prefill kernels only (more than 64 routes)
        with pytest.raises(ValueError, match="FP8 activations need a prefill shape"):
            routed_experts(*args, activations=activations)
        return
    out, ok = routed_experts(*args, activations=activations)
    ref, ref_ok = O.routed_experts(x, ids, w, **tables, activations=activations)
    assert bool(ok) == ref_ok
    close = assert_moe_close if activations == "bfloat16" else assert_fp8_close
    print(cfg, activations, close(host_f32(out), ref))


def _routes_with_counts(counts, tokens, top_k, seed):
    """Route ids [tokens, top_k] with exactly counts[e] routes to expert e and
    distinct experts per token (each token takes the top_k experts with the
    most routes left, ties to the lower id; feasible while every count is at
    most `tokens` and the counts sum to tokens x top_k), tokens and slots then
    shuffled.  Route weights as the router gives them: positive, summing to 1."""
    left = np.asarray(counts, np.int64).copy()
    assert left.sum() == tokens * top_k and left.max() <= tokens
    ids = np.empty((tokens, top_k), np.int32)
    for t in range(tokens):
        pick = np.lexsort((np.arange(left.size), -left))[:top_k]
        assert (left[pick] > 0).all()
        ids[t] = pick
        left[pick] -= 1
    rng = np.random.default_rng(seed)
    ids = rng.permuted(ids[rng.permutation(tokens)], axis=1)
    w = rng.random((tokens, top_k)).astype(np.float32) + 0.05
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


# Wide tiles: the bf16 prefill plan cuts an expert's routes into tiles of up
# to 256, and the prefill kernel runs tiles of 129 .. 256 routes on its wide
# variants (10, 12, 14 or 16 column groups of 16 routes; an odd count takes
# the next even variant with a padding group), the rest on the narrow ones.
# The expert counts give wide tiles of every column-group count 9 .. 16, multi-
# tile experts whose last tile is narrow (300 = 256 + 44, 513 = 256 + 256 + 1,
# 600 = 256 + 256 + 88) or wide (700 = 256 + 256 + 188), and narrow tiles; the
# FP8 mode plans the same routes in tiles of 128.
# I = 256 gives the down projection K = 2 blocks (the weight ring's first
# blocks are the whole K loop), I = 1024 eight.
# Stripes: a projection whose N is a multiple of 512 (down: H) or 256 (gate/up:
# I) runs tall stripes (512 weight rows a work item), where a wide tile is
# listed twice and each listing takes half the stripe; otherwise 256-row
# stripes, which skip the second listing.  H = 1536 / I = 256, 1024: both
# projections tall; H = 768 / I = 384: neither; H = 1536 / I = 384: gate/up on
# 256-row stripes beside a tall down projection (the list holds second
# listings that the gate/up kernel skips).
WIDE_COUNTS = [129, 150, 170, 190, 200, 220, 230, 256, 300, 513, 600, 700, 1, 40, 128, 17]


@pytest.mark.parametrize("activations", ["bfloat16", "float8_e4m3fn"])
@pytest.mark.parametrize("hidden,inter,seed", [(1536, 256, 611), (1536, 1024, 613), (768, 384, 617),
                                               (1536, 384, 619)])
def test_prefill_wide_tiles_match_oracle(device, activations, hidden, inter, seed):
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    tokens, experts, top_k = 800, 32, 8
    counts = np.zeros(experts, np.int64)
    counts[: len(WIDE_COUNTS)] = WIDE_COUNTS
    rest = tokens * top_k - counts.sum()
    counts[len(WIDE_COUNTS):] = rest // (experts - len(WIDE_COUNTS))
    counts[-1] += rest - counts[len(WIDE_COUNTS):].sum()
    groups = {16 for c in counts if c >= 256} | {int(c % 256 + 15) // 16 for c in counts if c % 256}
    assert groups >= set(range(9, 17)) and (counts > 512).sum() >= 3
    ids, w = _routes_with_counts(counts, tokens, top_k, seed)
    assert (np.bincount(ids.ravel(), minlength=experts) == counts).all()
    cfg = S.MoeConfig("wide", tokens, experts, hidden, inter, top_k)
    x = S.hidden_states(cfg, seed)
    tables = S.host_expert_tables(cfg, seed)
    t = _device_tables(tables, device)
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                             activations=activations)
    ref, ref_ok = O.routed_experts(x, ids, w, **tables, activations=activations)
    assert bool(ok) and ref_ok
    close = assert_moe_close if activations == "bfloat16" else assert_fp8_close
    print(cfg, activations, close(host_f32(out), ref))


def test_routed_experts_invalid_routes_follow_reference(device):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(4, 8, 256, 256, 2, 0.0, seed=9)
    t = _device_tables(tables, device)
    bad = ids.copy()
    bad[2, 1] = 99
    args = (bf16_dev(x, device), dev(bad, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    out, ok = routed_experts(*args)
    ref, ref_ok = O.routed_experts(x, bad, w, **tables)
    assert not bool(ok) and not ref_ok
    assert_moe_close(host_f32(out), ref)
    out, _ = routed_experts(*args, drop_unowned=True, check_weights=False, route_sum="bfloat16")
    ref, _ = O.routed_experts(x, bad, w, **tables, drop_unowned=True, check_weights=False, route_sum="bfloat16")
    assert_moe_close(host_f32(out), ref)
    dup = ids.copy()
    dup[0, 1] = dup[0, 0]
    out, ok = routed_experts(bf16_dev(x, device), dev(dup, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    ref, ref_ok = O.routed_experts(x, dup, w, **tables)
    assert not bool(ok) and not ref_ok
    assert_moe_close(host_f32(out), ref)
    neg = w.copy()
    neg[1, 0] = float("nan")
    _, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(neg, device), *(t[k] for k in TABLE_KEYS))
    assert not bool(ok)


# ----------------------------------------------------------------------------- production shapes
@pytest.fixture(scope="module")
def production_tables(device):
    from glm_moe import synthetic as S

    tables = S.device_expert_tables(S.CONFIGS["decode_t1"], seed=0, device=device)
    torch.cuda.synchronize()
    yield tables
    del tables
    torch.cuda.empty_cache()


def _subproblem(tables, ids):
    """Host copies of the selected experts, renumbered 0..D-1, and the remapped ids."""
    used = np.unique(ids.reshape(-1))
    remap = {int(e): i for i, e in enumerate(used)}
    index = torch.as_tensor(used, dtype=torch.long, device=tables["gate_bits"].device)
    host = {k: tables[k].index_select(0, index).cpu().numpy() for k in TABLE_KEYS}
    return host, np.vectorize(remap.get)(ids).astype(np.int32)


def test_synthetic_weights_follow_the_recipe(device, production_tables):
    bits = production_tables["gate_bits"][:2].cpu().numpy()
    scales = production_tables["gate_scale"][:2].cpu().numpy()
    assert not np.any((bits & 0x7F) == 0x7F)  # finite encodings only
    w = O.decode_fp8_table(bits, scales)
    assert abs(float(w.std()) - 0.02) < 0.002 and abs(float(w.mean())) < 1e-3
    # every block's largest magnitude decodes to ~448 * scale (scale = amax / 448)
    blocks = np.abs(O.fp8_e4m3fn_table()[bits]).reshape(2, 16, 128, 48, 128).max(axis=(2, 4))
    assert np.all(blocks >= 416)


@pytest.mark.parametrize("name", ["decode_t1", "decode_t4"])
def test_decode_production_shape_matches_oracle(device, production_tables, name):
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg = S.CONFIGS[name]
    x = S.hidden_states(cfg, 3)
    ids, w = S.routes(cfg, 3)
    t = production_tables
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    host, local_ids = _subproblem(t, ids)
    ref, _, mag = O.routed_experts(x, local_ids, w, **host, return_route_max=True)
    assert bool(ok)
    print(name, assert_moe_close(host_f32(out), ref, magnitude=mag))
    again, _ = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    np.testing.assert_array_equal(bf16_bits_of(again), bf16_bits_of(out))  # deterministic


@pytest.mark.parametrize("top_k,unowned", [(6, False), (5, False), (8, True), (3, True)])
def test_decode_production_shape_ragged_route_pairs(device, production_tables, top_k, unowned):
    """One token at I = 2048 with fewer than 8 active routes (top-k below 8, or an
    unowned route dropped): the down kernel's four waves take two routes each
    where they exist and one or none elsewhere."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg = S.CONFIGS["decode_t1"]
    x = S.hidden_states(cfg, 5)
    ids, w = S.routes(cfg, 5)
    ids, w = np.ascontiguousarray(ids[:, :top_k]), np.ascontiguousarray(w[:, :top_k])
    t = production_tables
    host, local_ids = _subproblem(t, ids)
    if unowned:
        ids = ids.copy()
        ids[0, 1] = cfg.experts + 7  # outside [0, E): dropped from the sum
        local_ids = local_ids.copy()
        local_ids[0, 1] = -1
    kw = dict(drop_unowned=True, check_weights=False, route_sum="bfloat16") if unowned else {}
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                             **kw)
    ref, _ = O.routed_experts(x, local_ids, w, **host, **kw)
    if not unowned:
        assert bool(ok)
    print(top_k, unowned, assert_moe_close(host_f32(out), ref))


def covering_rows(ids, experts, tile=128, group=16):
    """Token rows that reach every work item of the prefill GEMMs: for every
    expert with routes, each of its ``tile``-route tiles (consecutive sorted
    routes, the route plan's work list) at the first route of every ``group``
    routes (the kernels' 16-route column groups) and at its last route."""
    k = ids.shape[1]
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    offsets = np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=experts))])
    rows = set()
    for e in range(experts):
        for start in range(int(offsets[e]), int(offsets[e + 1]), tile):
            end = min(start + tile, int(offsets[e + 1]))
            for pos in [*range(start, end, group), end - 1]:
                rows.add(int(order[pos]) // k)
    return np.array(sorted(rows))


@pytest.mark.parametrize("name", ["batch_t64", "prefill_t2048", "prefill_t8192_zipf"])
def test_prefill_production_shape_every_tile(device, production_tables, name):
    """Full-size grouped path (64 tokens of 1-2 routes per expert, T=2048, T=8192
    Zipf).  Each output row depends only on its token's routes, so the oracle
    checks the rows that reach every expert, every 128 routes of every expert
    (each half of a 256-route tile) and every 16-route column group of every
    tile; the whole output is checked for finiteness and run-to-run bit
    equality."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg = S.CONFIGS[name]
    x = S.hidden_states(cfg, 5)
    ids, w = S.routes(cfg, 5)
    t = production_tables
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    out, ok = routed_experts(*args)
    assert bool(ok)
    full = host_f32(out)
    assert np.all(np.isfinite(full))
    again, _ = routed_experts(*args)
    np.testing.assert_array_equal(bf16_bits_of(again), bf16_bits_of(out))
    rows = covering_rows(ids, cfg.experts)
    assert set(np.unique(ids[rows])) == set(np.unique(ids))  # every expert with routes
    host, local_ids = _subproblem(t, ids[rows])
    ref, _, mag = O.routed_experts(x[rows], local_ids, w[rows], **host, return_route_max=True)
    # one flip of 2 ulps measured at T=8192 Zipf (in 2.3e7 elements): a route's
    # down value flipped by one ulp moves bf16(down * w) by 2 ulps of it where
    # w < 1 takes the product into the next lower binade
    print(name, f"{len(rows)} of {cfg.tokens} rows:", assert_moe_close(full[rows], ref, magnitude=mag, flip_ulps=2))


def _shared_expert_tables(cfg, seed):
    """bf16-valued shared-expert weights [I, H], [I, H], [H, I] (I = the routed
    experts' intermediate size, GLM-5's single shared expert)."""
    rng = np.random.default_rng(seed)
    return [O.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))
            for shape, std in (((cfg.intermediate, cfg.hidden), cfg.hidden ** -0.5),
                               ((cfg.intermediate, cfg.hidden), cfg.hidden ** -0.5),
                               ((cfg.hidden, cfg.intermediate), 2 * cfg.intermediate ** -0.5))]


@pytest.mark.parametrize("name", ["prefill_t2048", "prefill_t8192_zipf"])
def test_prefill_layer_production_size_matches_oracle(device, production_tables, name):
    """The whole prefill layer body at the BASELINE prefill configs, as served:
    ``prefill_moe_from_routes`` (route plan, grouped GEMMs, the bf16 shared
    expert on hipBLASLt, ``bf16(bf16(routed x bf16(2.5)) + shared)`` fused into
    the route combine, the health bit; routed_experts.py:27-128) against the
    oracle's ``moe_layer`` (tests/reference/moe.py:78-99) on the rows that reach
    every expert, every 128 routes and every 16-route column group.  The whole
    output is finite; a duplicate id or a NaN weight clears health."""
    from glm_moe import synthetic as S
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import prefill_moe_from_routes

    cfg = S.CONFIGS[name]
    contract = single_gpu_contract(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                                   num_experts=cfg.experts, top_k=cfg.top_k)
    shared_f32 = _shared_expert_tables(cfg, 41)
    shared_dev = tuple(bf16_dev(a, device) for a in shared_f32)
    x = S.hidden_states(cfg, 21)
    ids, w = S.routes(cfg, 21)
    t = production_tables
    tables = tuple(t[k] for k in TABLE_KEYS)
    xs = bf16_dev(x, device)
    out, ok = prefill_moe_from_routes(xs, dev(ids, device), dev(w, device), *tables, *shared_dev, contract=contract)
    assert bool(ok)
    full = host_f32(out)
    assert np.all(np.isfinite(full))
    rows = covering_rows(ids, cfg.experts)
    host, local_ids = _subproblem(t, ids[rows])
    ref, ref_ok, mag = O.moe_layer(x[rows], local_ids, w[rows], *(host[k] for k in TABLE_KEYS), *shared_f32,
                                   return_magnitude=True)
    assert ref_ok
    print(name, f"layer, {len(rows)} of {cfg.tokens} rows:",
          assert_moe_close(full[rows], ref, magnitude=mag, flip_ulps=closeness.LAYER_FLIP_ULPS,
                           max_flips=closeness.layer_max_flips(ref.size)))

    dup = ids.copy()
    dup[cfg.tokens // 2, 1] = dup[cfg.tokens // 2, 0]
    _, ok = prefill_moe_from_routes(xs, dev(dup, device), dev(w, device), *tables, *shared_dev, contract=contract)
    assert not bool(ok)
    nan = w.copy()
    nan[cfg.tokens - 1, 0] = float("nan")
    _, ok = prefill_moe_from_routes(xs, dev(ids, device), dev(nan, device), *tables, *shared_dev, contract=contract)
    assert not bool(ok)


@pytest.mark.parametrize("tokens,experts,top_k,zipf", [(1024, 16, 8, 1.2), (640, 32, 8, 0.0)])
def test_prefill_production_k_full_output(device, tokens, experts, top_k, zipf):
    """Every output row against the oracle at the production hidden and
    intermediate sizes (K/128 = 48 and 16) with few experts, so that multi-tile
    experts, partial tiles and every column-group count meet the real K."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg = S.MoeConfig("prod_k", tokens, experts, 6144, 2048, top_k, zipf)
    x = S.hidden_states(cfg, 12)
    ids, w = S.routes(cfg, 12)
    t = S.device_expert_tables(cfg, seed=12, device=device)
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    assert bool(ok)
    counts = np.bincount(ids.reshape(-1), minlength=experts)
    assert counts.max() > 128  # multi-tile experts are present
    host = {k: v.cpu().numpy() for k, v in t.items()}
    ref, _ = O.routed_experts(x, ids, w, **host)
    print(cfg, assert_moe_close(host_f32(out), ref))


@pytest.mark.parametrize("tokens,top_k", [(300, 6), (2048, 8)])
def test_grouped_path_invalid_routes_follow_reference(device, tokens, top_k):
    """Beyond the decode kernels' 64 routes (route plan + grouped GEMMs + combine):
    an out-of-range id is computed as expert 0, a duplicate id is computed twice,
    NaN or negative weights clear the health bit -- all with the reference's
    outputs (routed_experts.py:83, :152-164); with the ownership mask an
    out-of-range route contributes zero instead (:250-253)."""
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(tokens, 64, 512, 256, top_k, 0.0, seed=tokens + 3)
    t = _device_tables(tables, device)
    xs = bf16_dev(x, device)

    def both(route_ids, weights, **kw):
        got, ok = routed_experts(xs, dev(route_ids, device), dev(weights, device), *(t[k] for k in TABLE_KEYS),
                                 **kw)
        ref, ref_ok = O.routed_experts(x, route_ids, weights, **tables, **kw)
        assert bool(ok) == ref_ok
        assert_moe_close(host_f32(got), ref)
        return ok

    bad = ids.copy()
    bad[1, 2] = 64            # one past the last expert: safe id 0
    bad[tokens // 2, 0] = -3  # negative: safe id 0
    bad[tokens - 1, top_k - 1] = 2**31 - 1
    assert not bool(both(bad, w))
    both(bad, w, drop_unowned=True, check_weights=False, route_sum="bfloat16")
    dup = ids.copy()
    dup[3, 1] = dup[3, 0]
    dup[tokens - 2, top_k - 1] = dup[tokens - 2, 0]
    assert not bool(both(dup, w))
    for value in (float("nan"), -0.25, float("inf")):
        odd = w.copy()
        odd[tokens // 3, 1] = value
        _, ok = routed_experts(xs, dev(ids, device), dev(odd, device), *(t[k] for k in TABLE_KEYS))
        assert not bool(ok), value
    neg = w.copy()
    neg[5, 0] = -0.25
    assert bool(both(ids, neg, check_weights=False))  # computed with the negative weight


@pytest.mark.parametrize("rank", [0, 5])
def test_expert_share_at_production_size_matches_owned_partial(device, production_tables, rank):
    """One EP8 share (32 of 256 experts) of the T=2048 prefill: only the share's
    routes are computed, and its FP32 partial equals the oracle's owned-only
    partial on every row (routed_experts.py:85-112, panels.py:26-83)."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts_share

    cfg = S.CONFIGS["prefill_t2048"]
    x = S.hidden_states(cfg, 13)
    ids, w = S.routes(cfg, 13)
    lo = 32 * rank
    share = {k: v[lo:lo + 32] for k, v in production_tables.items()}
    part, ok = routed_experts_share(bf16_dev(x, device), dev(ids, device), dev(w, device),
                                    *(share[k] for k in TABLE_KEYS), num_experts=256, expert_offset=lo)
    assert bool(ok)
    host = {k: v.cpu().numpy() for k, v in share.items()}
    ref, _ = O.routed_experts(x, ids, w, **host, num_experts=256, expert_offset=lo, round_output=False)
    owned_rows = ((ids >= lo) & (ids < lo + 32)).any(axis=1)
    got = host_f32(part)
    assert np.all(got[~owned_rows] == 0.0)  # tokens with no route to the share
    print(f"share {rank}: {int(owned_rows.sum())} rows", assert_moe_close(got, ref))


@pytest.mark.parametrize("tokens,top_k", [(300, 6), (4, 8), (1, 8)])
def test_expert_shares_sum_to_the_whole_layer(device, tokens, top_k):
    """Four shares of 16 experts: each partial matches the oracle's share, the
    sum of the partials over the expert axis gives the whole layer's routed
    output, and the layer bodies with a share contract (stage_size=4,
    expert_reduce summing the shares) give the one-GPU layer's output."""
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import (moe_grouped_routes, prefill_moe_from_routes, routed_experts,
                                                   routed_experts_share)

    cfg, x, ids, w, tables = _small_case(tokens, 64, 512, 256, top_k, 0.0, seed=tokens + 17)
    ids = ids.copy()
    if tokens > 1:
        ids[1, 0] = 70  # invalid id: safe id 0 (share 0) in prefill, dropped in decode
    t = _device_tables(tables, device)
    xs, idd, wd = bf16_dev(x, device), dev(ids, device), dev(w, device)
    decode = tokens == 1
    kw = dict(route_sum="bfloat16", check_weights=False, drop_unowned=True) if decode else {}
    whole, whole_ok = routed_experts(xs, idd, wd, *(t[k] for k in TABLE_KEYS), **kw)
    partials = []
    for rank in range(4):
        lo = 16 * rank
        share = {k: v[lo:lo + 16] for k, v in t.items()}
        part, ok = routed_experts_share(xs, idd, wd, *(share[k] for k in TABLE_KEYS), num_experts=64,
                                        expert_offset=lo, **kw)
        assert bool(ok) == bool(whole_ok)
        ref, _ = O.routed_experts(x, ids, w, **{k: v[lo:lo + 16] for k, v in tables.items()}, num_experts=64,
                                  expert_offset=lo, round_output=False, **kw)
        assert_moe_close(host_f32(part), ref)
        partials.append(part)
    summed = torch.stack(partials).sum(0).to(torch.bfloat16)
    print(cfg, "sum of shares vs whole:", assert_moe_close(host_f32(summed), host_f32(whole)))

    # the layer bodies with a share contract; the expert axis is simulated by
    # summing the other shares' partials
    rng = np.random.default_rng(tokens)
    shared = tuple(bf16_dev((rng.standard_normal(shape) * 0.05).astype(np.float32), device)
                   for shape in ((256, 512), (256, 512), (512, 256)))
    one = single_gpu_contract(hidden_size=512, intermediate_size=256, num_experts=64, top_k=top_k)
    four = single_gpu_contract(hidden_size=512, intermediate_size=256, num_experts=64, top_k=top_k, stage_size=4)
    rank = 2
    share = {k: v[32:48] for k, v in t.items()}

    def expert_reduce(partial):
        return sum(p for r, p in enumerate(partials) if r != rank) + partial

    if decode:
        want = moe_grouped_routes(xs, idd, wd, *(t[k] for k in TABLE_KEYS), contract=one, shared_bf16=shared)
        got = moe_grouped_routes(xs, idd, wd, *(share[k] for k in TABLE_KEYS), contract=four, shared_bf16=shared,
                                 expert_rank=rank, expert_reduce=expert_reduce)
    else:
        want, want_ok = prefill_moe_from_routes(xs, idd, wd, *(t[k] for k in TABLE_KEYS), *shared, contract=one)
        got, got_ok = prefill_moe_from_routes(xs, idd, wd, *(share[k] for k in TABLE_KEYS), *shared,
                                              contract=four, expert_rank=rank, expert_reduce=expert_reduce)
        assert bool(got_ok) == bool(want_ok)
    print("share layer body vs one-GPU body:", assert_moe_close(host_f32(got), host_f32(want)))


def test_decode_headline_layer_matches_oracle(device, production_tables):
    """The headline decode body exactly as benchmarked: one row, E=256, top-8,
    H=6144, I=2048, the resident bf16 shared expert inside the two decode kernels
    and the per-owner bf16 route sum, through ``moe_grouped_routes`` against the
    oracle's ``moe_layer(decode=True)`` (routed_experts.py:186-304)."""
    from glm_moe import synthetic as S
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import moe_grouped_routes

    cfg = S.CONFIGS["decode_t1"]
    contract = single_gpu_contract(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                                   num_experts=cfg.experts, top_k=cfg.top_k)
    shared_f32 = _shared_expert_tables(cfg, 31)
    shared_dev = tuple(bf16_dev(a, device) for a in shared_f32)
    t = production_tables
    for seed in (8, 9, 10):
        x = S.hidden_states(cfg, seed)
        ids, w = S.routes(cfg, seed)
        got = moe_grouped_routes(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                                 contract=contract, shared_bf16=shared_dev)
        host, local_ids = _subproblem(t, ids)
        ref, _, mag = O.moe_layer(x, local_ids, w, *(host[k] for k in TABLE_KEYS), *shared_f32, decode=True,
                                  return_magnitude=True)
        print("decode headline layer", seed,
              assert_moe_close(host_f32(got), ref, magnitude=mag, label=f"seed {seed}",
                               flip_ulps=closeness.LAYER_FLIP_ULPS, max_flips=closeness.layer_max_flips(ref.size)))


# ----------------------------------------------------------------------------- native FP8 mode
# No reference counterpart: the mode is checked against its own definition in
# the oracle (quantize_rows_fp8 / block_dot_fp8) to the north-star tolerance,
# and its error against the reference numerics (the bf16 oracle) is reported.
FP8_ERROR_BOUND = 5e-2  # mean-rel against the bf16 reference numerics (e4m3 activations: 3 mantissa bits)
# Against its own definition the FP8 mode keeps the north-star mean-rel (5e-3),
# but not max-abs 2e-2: its activations are re-quantised to e4m3 per 128-wide
# block, so a one-ulp bf16 difference in a SwiGLU value (the FP32 sums of the
# gate/up projections rounding the other way) can move its block's amax, hence
# the block scale, and re-round all 128 e4m3 values of the block, which moves
# the route's whole down row.  Measured at full prefill size: T=8192 Zipf
# mean-rel 1.3e-3, max-abs 0.039, 445 of 6.8e6 elements (6.5e-5) beyond 2e-2;
# T=2048 none.
FP8_MAX_ABS = 5e-2


FP8_OVER_FRACTION = 2e-4  # elements beyond max-abs 2e-2 (measured 6.5e-5; a re-quantised block moves a route row)


def assert_fp8_close(got, ref, label="fp8 mode vs its oracle"):
    c = closeness.check(got, ref, label=label, flip_ulps=np.inf,
                        max_flips=int(FP8_OVER_FRACTION * np.size(ref)))
    assert c.max_abs <= FP8_MAX_ABS, f"max-abs {c.max_abs:.3e} > {FP8_MAX_ABS}"
    return c


def test_fp8_mode_matches_its_oracle_and_reports_its_error(device):
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg, x, ids, w, tables = _small_case(512, 16, 512, 512, 8, 0.0, seed=77)
    t = _device_tables(tables, device)
    args = (bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS))
    out, ok = routed_experts(*args, activations="float8_e4m3fn")
    assert bool(ok)
    got = host_f32(out)
    ref8, _ = O.routed_experts(x, ids, w, **tables, activations="float8_e4m3fn")
    print("fp8 mode vs fp8 oracle:", assert_fp8_close(got, ref8))
    ref16, _ = O.routed_experts(x, ids, w, **tables)
    err = np.abs(got - ref16)
    rel = err.mean() / np.abs(ref16).mean()
    print(f"fp8 mode vs reference numerics: max-abs {err.max():.3e}, mean-rel {rel:.3e}")
    assert rel <= FP8_ERROR_BOUND
    again, _ = routed_experts(*args, activations="float8_e4m3fn")
    np.testing.assert_array_equal(bf16_bits_of(again), bf16_bits_of(out))  # deterministic


@pytest.mark.parametrize("name", ["prefill_t2048", "prefill_t8192_zipf"])
def test_fp8_mode_production_shape_every_tile(device, production_tables, name):
    """FP8 mode at full size against its oracle on the rows that reach every
    expert and every 128-route tile (first and last route of each tile)."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts

    cfg = S.CONFIGS[name]
    x = S.hidden_states(cfg, 7)
    ids, w = S.routes(cfg, 7)
    t = production_tables
    out, ok = routed_experts(bf16_dev(x, device), dev(ids, device), dev(w, device), *(t[k] for k in TABLE_KEYS),
                             activations="float8_e4m3fn")
    assert bool(ok)
    full = host_f32(out)
    assert np.all(np.isfinite(full))
    rows = covering_rows(ids, cfg.experts, group=128)
    host, local_ids = _subproblem(t, ids[rows])
    ref8, _ = O.routed_experts(x[rows], local_ids, w[rows], **host, activations="float8_e4m3fn")
    print(f"{name} fp8 mode vs fp8 oracle, {len(rows)} rows:", assert_fp8_close(full[rows], ref8))
    ref16, _ = O.routed_experts(x[rows], local_ids, w[rows], **host)
    err = np.abs(full[rows] - ref16)
    rel = err.mean() / np.abs(ref16).mean()
    print(f"{name} fp8 mode vs reference numerics: max-abs {err.max():.3e}, mean-rel {rel:.3e}")
    assert rel <= FP8_ERROR_BOUND


# ----------------------------------------------------------------------------- router (route_glm_noaux_tc_logits)
def test_router_reference_known_answers(device):
    """The reference's KATs (tests/layers/moe/test_router.py:51-65), exactly."""
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    logits = dev(np.float32([[3.0, 2.0, 1.0, 0.0]]), device)
    bias = dev(np.float32([0.0, 0.0, 100.0, 99.0]), device)
    ids, w = route_glm_noaux_tc_logits(logits, bias, top_k=2)
    np.testing.assert_array_equal(ids.cpu().numpy(), [[2, 3]])
    unbiased = O.sigmoid_f32(np.float32([1.0, 0.0]))
    np.testing.assert_allclose(w.cpu().numpy()[0], unbiased / unbiased.sum(dtype=np.float32), rtol=1e-7, atol=0)
    ids, w = route_glm_noaux_tc_logits(dev(np.zeros((1, 16), np.float32), device),
                                       dev(np.zeros(16, np.float32), device), top_k=8)
    np.testing.assert_array_equal(ids.cpu().numpy(), [list(range(8))])
    np.testing.assert_array_equal(w.cpu().numpy(), np.full((1, 8), 0.125, np.float32))


@pytest.mark.parametrize("tokens,experts,top_k,zipf,biased", [
    (1, 256, 8, 0.0, False), (300, 256, 8, 0.0, True), (2048, 256, 8, 1.2, False), (64, 1024, 16, 0.0, True),
    (5, 8, 2, 0.0, False), (40, 256, 64, 0.0, True), (7, 64, 64, 0.0, False),
])
def test_router_matches_oracle(device, tokens, experts, top_k, zipf, biased):
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    rng = np.random.default_rng(tokens + experts)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    if zipf:
        r = np.arange(1, experts + 1, dtype=np.float64) ** -zipf
        logits = (logits + np.log(r / r.sum()).astype(np.float32)).astype(np.float32)
    bias = (rng.standard_normal(experts) * 0.1).astype(np.float32) if biased else np.zeros(experts, np.float32)
    ids, w = route_glm_noaux_tc_logits(dev(logits, device), dev(bias, device), top_k=top_k)
    ref_ids, ref_w = O.route_glm_noaux_tc_logits(logits, bias, top_k=top_k)
    # selection is compared exactly where the oracle's k-th and (k+1)-th biased
    # scores are separated by more than the FP32 sigmoid rounding (a near-tie is
    # decided by the last bit of exp, which the reference's XLA does not pin
    # either); every other token must still hold a valid top-k of the oracle's
    # scores up to that rounding, best first, with the oracle's weights for it
    unbiased = O.sigmoid_f32(logits)
    scores = unbiased + bias[None, :]
    srt = -np.sort(-scores, axis=1)
    clear = (srt[:, top_k - 1] - srt[:, top_k]) > 1e-6 if top_k < experts else np.ones(tokens, bool)
    assert clear.mean() > 0.9
    got_ids, got_w = ids.cpu().numpy(), w.cpu().numpy()
    np.testing.assert_array_equal(got_ids[clear], ref_ids[clear])
    for t in range(tokens):
        chosen = got_ids[t]
        assert len(set(chosen.tolist())) == top_k and chosen.min() >= 0 and chosen.max() < experts
        picked = scores[t, chosen]
        assert picked.min() >= srt[t, top_k - 1] - 1e-6  # nothing outside the top-k band
        assert np.all(np.diff(picked) <= 1e-6)            # best first
        sel = unbiased[t, chosen]
        np.testing.assert_allclose(got_w[t], sel / sel.sum(dtype=np.float32), rtol=2e-6, atol=1e-7)


# ----------------------------------------------------------------------------- routing inside the decode layer
# glm_moe_moe_layer_from_logits routes each token inside the decode gate/up
# kernel.  It must give the router kernel's ids and weights and the two-step
# layer's output (route_glm_noaux_tc_logits, then the resident layer), bit for bit.
def _router_layer_case(tokens, experts, hidden, inter, top_k, seed, device, biased=True):
    rng = np.random.default_rng(seed)
    cfg, x, _, _, tables = _small_case(tokens, experts, hidden, inter, top_k, 0.0, seed=seed)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    bias = (rng.standard_normal(experts) * 0.1).astype(np.float32) if biased else np.zeros(experts, np.float32)
    shared_f32 = [(rng.standard_normal(shape) * std).astype(np.float32)
                  for shape, std in (((inter, hidden), hidden ** -0.5), ((inter, hidden), hidden ** -0.5),
                                     ((hidden, inter), 2 * inter ** -0.5))]
    return (cfg, x, logits, bias, tables, _device_tables(tables, device), shared_f32,
            [bf16_dev(a, device) for a in shared_f32])


def _layer_from_logits_abi(x_dev, logits_dev, bias_dev, t, shared_dev, top_k, flags, device):
    from glm_moe import _lib
    from glm_moe.layers.moe.routed_experts import routed_workspace

    tokens, hidden = x_dev.shape
    experts, inter = t["gate_bits"].shape[0], t["gate_bits"].shape[1]
    ids = torch.full((tokens, top_k), -7, dtype=torch.int32, device=device)
    w = torch.full((tokens, top_k), -1.0, dtype=torch.float32, device=device)
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=device)
    valid = torch.empty((), dtype=torch.bool, device=device)
    ws = routed_workspace(tokens, top_k, experts, hidden, inter, device)
    _lib.call("glm_moe_moe_layer_from_logits", _lib.ptr(x_dev), tokens, hidden, _lib.ptr(logits_dev),
              _lib.ptr(bias_dev), top_k, experts, inter, *(_lib.ptr(t[k]) for k in TABLE_KEYS), flags,
              *(_lib.ptr(s) for s in shared_dev), inter, 2.5, _lib.ptr(ids), _lib.ptr(w), _lib.ptr(out),
              _lib.ptr(valid), _lib.ptr(ws), ws.numel(), _lib.stream_of(x_dev))
    return out, ids, w, valid


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,bf16_sum", [
    (1, 256, 512, 256, 8, True),      # the decode body (bf16 route sum)
    (4, 256, 768, 384, 8, False),     # four tokens, FP32 route sum
    (8, 64, 512, 256, 8, True),       # 64 routes, the decode kernels' limit; 64 experts
    (3, 8, 256, 256, 2, False),       # the toy geometry
])
def test_layer_from_router_logits_equals_two_steps(device, tokens, experts, hidden, inter, top_k, bf16_sum):
    from glm_moe import _lib
    from glm_moe.layers.moe.routed_experts import routed_experts
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    cfg, x, logits, bias, tables, t, shared_f32, shared_dev = _router_layer_case(
        tokens, experts, hidden, inter, top_k, tokens * 31 + experts, device)
    x_dev, logits_dev, bias_dev = bf16_dev(x, device), dev(logits, device), dev(bias, device)
    flags = _lib.ROUTE_SUM_BF16 if bf16_sum else 0
    out, ids, w, ok = _layer_from_logits_abi(x_dev, logits_dev, bias_dev, t, shared_dev, top_k, flags, device)
    ref_ids, ref_w = route_glm_noaux_tc_logits(logits_dev, bias_dev, top_k=top_k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids.cpu().numpy())
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), ref_w.cpu().numpy().view(np.uint32))
    kw = dict(route_sum="bfloat16" if bf16_sum else "float32", check_weights=False)
    ref, ref_ok = routed_experts(x_dev, ref_ids, ref_w, *(t[k] for k in TABLE_KEYS), shared_tables=tuple(shared_dev),
                                 **kw)
    assert bool(ok) and bool(ref_ok)
    np.testing.assert_array_equal(bf16_bits_of(out), bf16_bits_of(ref))
    # and against the oracle: its router, then its layer
    o_ids, o_w = O.route_glm_noaux_tc_logits(logits, bias, top_k=top_k)
    np.testing.assert_array_equal(ids.cpu().numpy(), o_ids)
    o_out, _ = O.moe_layer(x, o_ids, o_w, **tables, shared_gate=shared_f32[0], shared_up=shared_f32[1],
                           shared_down=shared_f32[2], decode=bf16_sum)
    print(cfg, "vs oracle:", assert_moe_close(host_f32(out), o_out))


def test_layer_from_router_logits_known_answers_and_python_api(device):
    """Router KATs (tests/layers/moe/test_router.py:61-65: equal logits -> ids 0..7,
    weights 1/8) through the fused layer, and the Python decode MLP body on both
    of its paths (fused on decode shapes, router kernel + moe_grouped_routes otherwise)."""
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import moe_grouped_routes, moe_mlp_from_router_logits
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    cfg, x, logits, bias, tables, t, shared_f32, shared_dev = _router_layer_case(1, 256, 512, 256, 8, 77, device)
    x_dev = bf16_dev(x, device)
    zeros = torch.zeros((1, 256), dtype=torch.float32, device=device)
    _, ids, w, ok = _layer_from_logits_abi(x_dev, zeros, None, t, shared_dev, 8, 0, device)
    assert bool(ok)
    np.testing.assert_array_equal(ids.cpu().numpy(), [list(range(8))])
    np.testing.assert_array_equal(w.cpu().numpy(), np.full((1, 8), 0.125, np.float32))
    contract = single_gpu_contract(hidden_size=512, intermediate_size=256, num_experts=256, top_k=8)
    logits_dev, bias_dev = dev(logits, device), dev(bias, device)
    tabs = [t[k] for k in TABLE_KEYS]
    update, ids, w = moe_mlp_from_router_logits(x_dev, logits_dev, bias_dev, *tabs, contract=contract,
                                                shared_bf16=tuple(shared_dev))
    ref_ids, ref_w = route_glm_noaux_tc_logits(logits_dev, bias_dev, top_k=8)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids.cpu().numpy())
    np.testing.assert_array_equal(w.cpu().numpy(), ref_w.cpu().numpy())
    ref = moe_grouped_routes(x_dev, ref_ids, ref_w, *tabs, contract=contract, shared_bf16=tuple(shared_dev))
    np.testing.assert_array_equal(bf16_bits_of(update), bf16_bits_of(ref))
    # more experts than the in-kernel router takes: router kernel, then the layer
    contract = single_gpu_contract(hidden_size=512, intermediate_size=256, num_experts=512, top_k=8)
    cfg, x, logits, bias, tables, t, shared_f32, shared_dev = _router_layer_case(1, 512, 512, 256, 8, 78, device)
    x_dev, logits_dev, bias_dev = bf16_dev(x, device), dev(logits, device), dev(bias, device)
    tabs = [t[k] for k in TABLE_KEYS]
    update, ids, w = moe_mlp_from_router_logits(x_dev, logits_dev, bias_dev, *tabs, contract=contract,
                                                shared_bf16=tuple(shared_dev))
    ref_ids, ref_w = route_glm_noaux_tc_logits(logits_dev, bias_dev, top_k=8)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids.cpu().numpy())
    ref = moe_grouped_routes(x_dev, ref_ids, ref_w, *tabs, contract=contract, shared_bf16=tuple(shared_dev))
    np.testing.assert_array_equal(bf16_bits_of(update), bf16_bits_of(ref))


# ----------------------------------------------------------------------------- layer from router logits, any T
# glm_moe_moe_layer_from_router_logits: the router kernel ahead of the plan on
# grouped shapes, routing inside the decode gate/up kernel on decode shapes.
# Its ids, weights, health and output must equal the router kernel followed by
# the layer, bit for bit.
def _two_step(x_dev, logits_dev, bias_dev, tabs, top_k, shared, **kw):
    from glm_moe.layers.moe.routed_experts import routed_experts
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    ids, w = route_glm_noaux_tc_logits(logits_dev, bias_dev, top_k=top_k)
    out, ok = routed_experts(x_dev, ids, w, *tabs, shared=shared, **kw)
    return out, ok, ids, w


def _assert_same_routing_and_layer(got, want):
    out, ok, ids, w = got
    ref, ref_ok, ref_ids, ref_w = want
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids.cpu().numpy())
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), ref_w.cpu().numpy().view(np.uint32))
    assert bool(ok) == bool(ref_ok)
    np.testing.assert_array_equal(bf16_bits_of(out), bf16_bits_of(ref))


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,zipf,shared", [
    (200, 64, 512, 256, 8, 0.0, True),     # 1600 routes: the one-workgroup plan
    (256, 256, 768, 256, 8, 1.2, False),   # exactly one chunk of 2048 routes, skewed logits
    (300, 64, 256, 512, 6, 0.0, True),     # 1800 routes, top-6
    (1536, 256, 768, 256, 8, 1.2, True),   # six chunks of the multi-workgroup plan
    (700, 128, 512, 256, 5, 0.0, False),   # chunks of 2045 routes (409 whole top-5 rows)
    (4, 256, 768, 384, 8, 0.0, True),      # decode shape: routing inside the decode gate/up kernel
    (300, 512, 512, 256, 8, 0.0, True),    # 512 experts: the router runs as its own launch first
])
def test_layer_from_router_logits_any_tokens_equals_two_steps(device, tokens, experts, hidden, inter, top_k,
                                                                    zipf, shared):
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts_from_router_logits

    cfg = S.MoeConfig("plan-router", tokens, experts, hidden, inter, top_k, zipf)
    seed = tokens + experts
    x_dev = bf16_dev(S.hidden_states(cfg, seed), device)
    logits = S.router_logits(cfg, seed)
    bias = (np.random.default_rng(seed).standard_normal(experts) * 0.1).astype(np.float32)
    logits_dev, bias_dev = dev(logits, device), dev(bias, device)
    dt = _device_tables(S.host_expert_tables(cfg, seed), device)
    tabs = [dt[k] for k in TABLE_KEYS]
    sh = bf16_dev(np.random.default_rng(seed + 1).standard_normal((tokens, hidden)).astype(np.float32) * 0.05,
                  device) if shared else None
    got = routed_experts_from_router_logits(x_dev, logits_dev, bias_dev, *tabs, top_k=top_k, shared=sh)
    _assert_same_routing_and_layer(got, _two_step(x_dev, logits_dev, bias_dev, tabs, top_k, sh))
    assert bool(got[1])
    # and the router against the oracle's (ids exact, weights to FP32 rounding)
    o_ids, o_w = O.route_glm_noaux_tc_logits(logits, bias, top_k=top_k)
    gap_ok = np.ones(tokens, bool)  # ids are compared where the k-th / (k+1)-th biased scores are apart
    sc = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias
    srt = np.sort(sc, axis=1)[:, ::-1]
    gap_ok = (srt[:, top_k - 1] - srt[:, top_k]) > 1e-6
    np.testing.assert_array_equal(got[2].cpu().numpy()[gap_ok], o_ids[gap_ok])
    np.testing.assert_allclose(got[3].cpu().numpy()[gap_ok], o_w[gap_ok], rtol=1e-6, atol=1e-7)


def test_layer_from_router_logits_health_fp8_and_production_size(device, production_tables):
    """Non-finite logits (a NaN row, an inf entry), bf16 route sum and the FP8
    mode through the one-call layer from logits; then T=2048 and T=8192 Zipf at
    production size, bit-equal to the two steps."""
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts_from_router_logits

    cfg = S.MoeConfig("plan-router-health", 512, 64, 512, 256, 8)
    x_dev = bf16_dev(S.hidden_states(cfg, 5), device)
    logits = S.router_logits(cfg, 5).copy()
    logits[7, :] = np.nan
    logits[100, 3] = np.inf
    logits_dev = dev(logits, device)
    dt = _device_tables(S.host_expert_tables(cfg, 5), device)
    tabs = [dt[k] for k in TABLE_KEYS]
    zero = torch.zeros(64, dtype=torch.float32, device=device)
    for kw in ({}, {"route_sum": "bfloat16", "check_weights": False}):
        got = routed_experts_from_router_logits(x_dev, logits_dev, None, *tabs, top_k=8, **kw)
        _assert_same_routing_and_layer(got, _two_step(x_dev, logits_dev, zero, tabs, 8, None, **kw))
        if kw == {}:
            assert not np.isfinite(got[3].cpu().numpy()[7]).any()  # the NaN row's weights
            assert not bool(got[1])  # non-finite weights clear the health byte
    cfg8 = S.MoeConfig("plan-router-fp8", 1024, 64, 512, 256, 8)
    x8 = bf16_dev(S.hidden_states(cfg8, 6), device)
    l8 = dev(S.router_logits(cfg8, 6), device)
    dt8 = _device_tables(S.host_expert_tables(cfg8, 6), device)
    t8 = [dt8[k] for k in TABLE_KEYS]
    got = routed_experts_from_router_logits(x8, l8, zero, *t8, top_k=8, activations="float8_e4m3fn")
    _assert_same_routing_and_layer(got, _two_step(x8, l8, zero, t8, 8, None, activations="float8_e4m3fn"))
    tabs = [production_tables[k] for k in TABLE_KEYS]
    for name in ("prefill_t2048", "prefill_t8192_zipf"):
        pc = S.CONFIGS[name]
        x_dev = bf16_dev(S.hidden_states(pc, 21), device)
        logits_dev = dev(S.router_logits(pc, 21), device)
        bias_dev = dev((np.random.default_rng(21).standard_normal(256) * 0.01).astype(np.float32), device)
        got = routed_experts_from_router_logits(x_dev, logits_dev, bias_dev, *tabs, top_k=8)
        _assert_same_routing_and_layer(got, _two_step(x_dev, logits_dev, bias_dev, tabs, 8, None))
        assert bool(got[1])
        print(name, "layer from logits: bit-equal to router + layer")


def test_prefill_moe_from_router_logits_composes_router_and_layer(device):
    """The Python prefill MLP from logits (decoder_layer.py:123-146 from the
    logits on): the same output as the router then prefill_moe_from_routes, and
    per-row health that is false on rows with non-finite logits."""
    from glm_moe import synthetic as S
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import prefill_moe_from_router_logits, prefill_moe_from_routes
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    for tokens in (300, 1):
        cfg = S.MoeConfig("prefill-logits", tokens, 64, 512, 256, 8)
        x_dev = bf16_dev(S.hidden_states(cfg, 9), device)
        logits = S.router_logits(cfg, 9).copy()
        if tokens > 1:
            logits[3, 5] = np.nan
        logits_dev = dev(logits, device)
        bias_dev = dev((np.random.default_rng(9).standard_normal(64) * 0.1).astype(np.float32), device)
        dt = _device_tables(S.host_expert_tables(cfg, 9), device)
        tabs = [dt[k] for k in TABLE_KEYS]
        rng = np.random.default_rng(10)
        shared = tuple(bf16_dev((rng.standard_normal(shape) * 0.05).astype(np.float32), device)
                       for shape in ((256, 512), (256, 512), (512, 256)))
        contract = single_gpu_contract(hidden_size=512, intermediate_size=256, num_experts=64, top_k=8)
        out, ids, w, ok = prefill_moe_from_router_logits(x_dev, logits_dev, bias_dev, *tabs, *shared,
                                                         contract=contract)
        ref_ids, ref_w = route_glm_noaux_tc_logits(logits_dev, bias_dev, top_k=8)
        np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids.cpu().numpy())
        ref, ref_ok = prefill_moe_from_routes(x_dev, ref_ids, ref_w, *tabs, *shared, contract=contract)
        np.testing.assert_array_equal(bf16_bits_of(out), bf16_bits_of(ref))
        ok = ok.cpu().numpy()
        assert ok.shape == (tokens,)
        if tokens > 1:
            assert not ok[3] and ok[[0, 1, 2, 4]].all() == bool(ref_ok)
        else:
            assert ok.all() == bool(ref_ok)


# ----------------------------------------------------------------------------- few-row shared expert
@pytest.mark.parametrize("tokens,hidden,inter", [(1, 512, 256), (2, 768, 384), (4, 6144, 2048), (8, 1024, 512)])
def test_shared_expert_rows_matches_oracle(device, tokens, hidden, inter):
    """glm_moe_shared_expert_rows against the oracle's shared expert
    (routed_experts.py:119-124 rounding points) and against the torch/hipBLASLt
    GEMMs it replaces (equal up to FP32 summation order)."""
    from glm_moe.layers.moe.routed_experts import _shared_swiglu, shared_expert_rows

    rng = np.random.default_rng(tokens * 7 + hidden)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    tables = [(rng.standard_normal(shape) * std).astype(np.float32)
              for shape, std in (((inter, hidden), hidden ** -0.5), ((inter, hidden), hidden ** -0.5),
                                 ((hidden, inter), 2 * inter ** -0.5))]
    x16 = O.bf16_round(x)
    t16 = [O.bf16_round(t) for t in tables]
    got = shared_expert_rows(bf16_dev(x16, device), *(bf16_dev(t, device) for t in t16))
    ref = O.shared_expert(x16, *t16)
    print("vs oracle:", assert_moe_close(host_f32(got), ref))
    other = _shared_swiglu(bf16_dev(x16, device), *(bf16_dev(t, device) for t in t16))
    print("vs hipBLASLt:", assert_moe_close(host_f32(got), host_f32(other)))
    again = shared_expert_rows(bf16_dev(x16, device), *(bf16_dev(t, device) for t in t16))
    np.testing.assert_array_equal(bf16_bits_of(again), bf16_bits_of(got))


def test_prefill_layer_few_rows_uses_the_shared_rows_kernels(device, golden):
    """prefill_moe_from_routes on 4 toy rows (few-row shared expert kernels) equals
    the golden layer within tolerance and the same layer with the torch shared expert."""
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import _shared_swiglu, prefill_moe_from_routes, routed_experts

    g = golden
    contract = single_gpu_contract(hidden_size=256, intermediate_size=256, num_experts=8, top_k=2)
    x = dev(g["hidden_bits"].view(np.int16), device).view(torch.bfloat16)
    ids, w = dev(g["route_indices"], device), dev(g["route_weights"], device)
    t = _device_tables(g, device)
    shared = [dev(g[k].view(np.int16), device).view(torch.bfloat16)
              for k in ("shared_gate_bits", "shared_up_bits", "shared_down_bits")]
    out, ok = prefill_moe_from_routes(x, ids, w, *(t[k] for k in TABLE_KEYS), *shared, contract=contract)
    assert bool(ok)
    print("toy layer, few-row shared expert:", assert_moe_close(host_f32(out), O.bf16_from_bits(g["layer_bits"])))
    other, _ = routed_experts(x, ids, w, *(t[k] for k in TABLE_KEYS), shared=_shared_swiglu(x, *shared),
                              routed_scale=2.5, check_weights=True)
    print("vs torch shared expert:", assert_moe_close(host_f32(out), host_f32(other)))


def test_workspace_cache_keeps_small_and_releases_large(device):
    """Small (decode) workspaces come from the per-stream cache; workspaces above
    WORKSPACE_CACHE_MAX (long prefills) are torch allocations of the call alone
    and are not held by the module."""
    import importlib

    from glm_moe import _lib

    R = importlib.import_module("glm_moe.layers.moe.routed_experts")  # the module, not the function
    R.release_workspaces()
    small = R.routed_workspace(4, 8, 256, 6144, 2048, device)
    again = R.routed_workspace(1, 8, 256, 6144, 2048, device)
    assert again.data_ptr() == small.data_ptr() and len(R._WORKSPACES) == 1
    big_bytes = int(_lib.lib().glm_moe_routed_experts_workspace_bytes(8192, 8, 256, 6144, 2048))
    assert big_bytes > R.WORKSPACE_CACHE_MAX
    big = R.routed_workspace(8192, 8, 256, 6144, 2048, device)
    assert big.numel() == big_bytes and len(R._WORKSPACES) == 1
    assert R._WORKSPACES[next(iter(R._WORKSPACES))].numel() < R.WORKSPACE_CACHE_MAX
    del big
    R.release_workspaces()
    assert not R._WORKSPACES
