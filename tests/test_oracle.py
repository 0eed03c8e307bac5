"""Pins of the CPU oracle (oracle/moe_oracle.py) against the reference's own
known answers, independent libraries, closed forms and brute force.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong index or sign, a transposed operand) fails it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O


# ----------------------------------------------------------------------------- scalar formats
def test_e4m3fn_table_matches_torch_for_every_bit_pattern():
    ours = O.fp8_e4m3fn_table()
    theirs = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(theirs)
    np.testing.assert_array_equal(np.isnan(ours), nan)
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])


def test_e4m3fn_known_answers():
    t = O.fp8_e4m3fn_table()
    # 0x38 = 1.0 (reference tests/layers/test_fp8.py:115-119), max finite 448, NaN codes
    assert t[0x38] == 1.0 and t[0xB8] == -1.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0x01] == 2.0**-9 and t[0x07] == 7 * 2.0**-9  # subnormals m * 2^-9
    assert t[0x08] == 2.0**-6  # smallest normal
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert int(np.isnan(t).sum()) == 2


def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        # exact ties: bf16 mantissa + half an ulp, both parities
        np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8), 3.0e38, -3.39e38, 1e-40, 0.0, -0.0],
                 np.float32),
        np.array([np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    ours = O.bf16_round(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, theirs)
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]
    # tie to even: 1 + 2^-8 lies between 1 and 1 + 2^-7 and rounds to 1
    assert O.bf16_round(np.float32(1.0 + 2**-8))[()] == 1.0
    assert O.bf16_round(np.float32(1.0 + 3 * 2**-8))[()] == 1.0 + 2**-6


def test_decode_uses_checkpoint_out_in_blocks():
    # reference tests/layers/moe/test_router.py:84-97: block (r, c) scales rows r and columns c
    bits = np.full((4, 6), 0x38, np.uint8)  # all 1.0
    scale = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    got = O.decode_fp8_table(bits, scale, block_shape=(2, 3))
    expected = np.array([[1, 1, 1, 2, 2, 2], [1, 1, 1, 2, 2, 2], [3, 3, 3, 4, 4, 4], [3, 3, 3, 4, 4, 4]],
                        np.float32)
    np.testing.assert_array_equal(got, expected)


def test_decode_is_one_f32_product_then_one_bf16_rounding():
    # independent of the oracle: FP64 product (exact: 4 + 24 bits) -> f32 -> bf16 via torch
    # (tests/reference/independent.py:78-88 double rounding argument)
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 256, (256, 384), dtype=np.uint8)
    bits[(bits & 0x7F) == 0x7F] = 0x3C
    scale = rng.uniform(0.01, 7.0, (2, 3)).astype(np.float32)
    values = torch.from_numpy(bits).view(torch.float8_e4m3fn).double().numpy()
    expanded = np.repeat(np.repeat(scale.astype(np.float64), 128, 0), 128, 1)
    expected = torch.from_numpy((values * expanded).astype(np.float32)).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.decode_fp8_table(bits, scale), expected)
    # ragged edges (partial last blocks) take the other code path of the decode
    ragged = np.ascontiguousarray(bits[:200, :300])
    np.testing.assert_array_equal(O.decode_fp8_table(ragged, scale), expected[:200, :300])


# ----------------------------------------------------------------------------- route grouping
def _brute_stable_sort(keys: list[int]) -> list[int]:
    order: list[int] = []
    for i, key in enumerate(keys):  # insertion sort: stable by construction
        j = len(order)
        while j > 0 and keys[order[j - 1]] > key:
            j -= 1
        order.insert(j, i)
    return order


@pytest.mark.parametrize("rows", [1, 17, 128])
@pytest.mark.parametrize("concentrated", [False, True])
def test_group_routes_is_the_stable_counting_sort(rows, concentrated):
    rng = np.random.default_rng(183)  # reference tests/layers/moe/test_routed_experts.py:15-37
    count = 32 if concentrated else 256
    ids = np.stack([rng.choice(count, 8, replace=False) for _ in range(rows)]).astype(np.int32)
    r = O.group_prefill_routes(ids)
    assert r.valid
    flat = ids.reshape(-1).tolist()
    assert r.sorted_flat_ids.tolist() == _brute_stable_sort(flat)
    counts = [0] * 256
    for e in flat:
        counts[e] += 1
    assert r.group_sizes.tolist() == counts
    assert all(r.sorted_flat_ids[r.inverse_permutation[i]] == i for i in range(len(flat)))
    if concentrated:
        assert int(r.group_sizes[32:].sum()) == 0
    values = np.arange(rows * 8 * 3, dtype=np.float32).reshape(rows * 8, 3)
    restored = O.restore_prefill_route_rows(values[r.sorted_flat_ids], r, top_k=8)
    np.testing.assert_array_equal(restored, values.reshape(rows, 8, 3))
    hidden = np.arange(rows * 4, dtype=np.float32).reshape(rows, 4)
    np.testing.assert_array_equal(O.gather_prefill_route_rows(hidden, r, top_k=8),
                                  hidden[np.asarray(_brute_stable_sort(flat)) // 8])


@pytest.mark.parametrize("bad", [-1, 256, 0])
def test_invalid_or_duplicate_routes_are_not_admitted(bad):
    # reference tests/layers/moe/test_routed_experts.py:40-44; invalid ids count as expert 0
    ids = np.arange(8, dtype=np.int32)[None, :].copy()
    ids[0, 7] = bad
    r = O.group_prefill_routes(ids)
    assert not r.valid
    assert int(r.group_sizes.sum()) == 8
    if bad != 0:
        assert r.group_sizes[0] == 2 and r.sorted_flat_ids.tolist()[:2] == [0, 7]


def test_wrong_route_dtype_is_rejected():
    with pytest.raises(ValueError, match="int32"):
        O.group_prefill_routes(np.zeros((2, 8), np.float32))


# ----------------------------------------------------------------------------- panels
@pytest.mark.parametrize("offset", [0, 2, 4])
def test_panels_restore_every_owned_row_once(offset):
    # reference tests/kernels/test_fp8_panel_matmul.py:31-50
    counts = np.array([1, 31, 32, 33, 0, 7], np.int32)
    m = int(counts.sum())
    x = np.arange(m * 3, dtype=np.float32).reshape(m, 3)
    plan = O.build_expert_panels(counts, offset, rows=m, local_groups=2)
    assert plan.valid
    assert plan.active_panels == sum((int(c) + 31) // 32 for c in counts[offset:offset + 2])
    packed = O.pack_expert_panel_rows(x, plan)
    live = np.arange(32)[None, :] < plan.live_counts[:, None]
    np.testing.assert_array_equal(packed[~live], 0)
    group = np.repeat(np.arange(6), counts)
    owned = (group >= offset) & (group < offset + 2)
    indices = plan.restore_indices[owned]
    assert len(np.unique(indices)) == int(counts[offset:offset + 2].sum())
    assert live.reshape(-1)[indices].all()
    poisoned = np.where(live[..., None], packed, np.nan)
    np.testing.assert_array_equal(O.unpack_expert_panel_rows(poisoned, plan), np.where(owned[:, None], x, 0))


@pytest.mark.parametrize("counts,offset", [
    ([19, 0, 0, 0], -1), ([19, 0, 0, 0], 3), ([19, 0, 0, 0], 2147483647),
    ([19, -1, 0, 0], 0), ([18, 0, 0, 0], 0), ([2147483647, 0, 0, 0], 0),
])
def test_invalid_panel_metadata_gives_no_work(counts, offset):
    # reference tests/kernels/test_fp8_panel_matmul.py:53-78
    plan = O.build_expert_panels(np.array(counts, np.int32), offset, rows=19, local_groups=2)
    assert not plan.valid and plan.active_panels == 0
    assert not plan.owned_rows.any()


def test_panel_capacity_closed_form_and_scale_zero():
    # reference tests/kernels/test_fp8_panel_matmul.py:140-151
    plan = O.build_expert_panels(np.array([0, 129, 0, 0], np.int32), 0, rows=129, local_groups=4)
    assert plan.active_panels == 5
    np.testing.assert_array_equal(plan.live_counts[:5], [32, 32, 32, 32, 1])
    x = np.ones((129, 128), np.float32)
    w = np.full((4, 256, 128), 0x38, np.uint8)
    s = np.ones((4, 2, 1), np.float32)
    s[1, 1, 0] = 0
    value, ok = O.panel_fp8_matmul(x, w, s, plan)
    assert ok
    np.testing.assert_array_equal(value[:, :128], 128)
    np.testing.assert_array_equal(value[:, 128:], 0)


def _fp64_dequant_dot(x, bits, scales):
    """FP64 brute force: whole-K contraction (a different order from the oracle's blocks)."""
    w = torch.from_numpy(bits).view(torch.float8_e4m3fn).double().numpy()
    expanded = np.repeat(np.repeat(scales.astype(np.float64), 128, -2), 128, -1)
    wq = torch.from_numpy((w * expanded).astype(np.float32)).to(torch.bfloat16).double().numpy()
    return x.astype(np.float64) @ wq.T


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_panel_matmul_matches_fp64_brute_force(dtype):
    # the reference's random case (tests/kernels/test_fp8_panel_matmul.py:105-137)
    rng = np.random.default_rng(911)
    counts = np.array([1, 33, 7, 0], np.int32)
    m, k, n = 41, 1152, 512
    x = O.bf16_round(rng.normal(0, 0.2, (m, k)).astype(np.float32))
    bits = torch.from_numpy(rng.normal(0, 0.15, (2, n, k)).astype(np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    scales = rng.uniform(0.1, 2.0, (2, 4, 9)).astype(np.float32)
    scales[0, 1, 8] = 0
    scales[1, 3, 8] = 3.25
    plan = O.build_expert_panels(counts, 1, rows=m, local_groups=2)
    value, ok = O.panel_fp8_matmul(x, bits, scales, plan, result_dtype=dtype)
    assert ok
    group = np.repeat(np.arange(4), counts) - 1
    owned = (group >= 0) & (group < 2)
    assert int(owned.sum()) == 40
    np.testing.assert_array_equal(value[~owned], 0)
    expected = np.zeros((m, n))
    for row in np.nonzero(owned)[0]:
        expected[row] = _fp64_dequant_dot(x[row:row + 1], bits[group[row]], scales[group[row]])[0]
    if dtype == "float32":
        np.testing.assert_allclose(value, expected, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_allclose(value, expected, rtol=2**-7, atol=2**-9)
    # a transposed scale table must be caught by the same check
    wrong = _fp64_dequant_dot(x[1:2], bits[0], scales[0][::-1].copy())[0]
    assert np.max(np.abs(wrong - expected[1])) > 1e-2


def test_routed_projection_clips_ids_and_zeroes_unowned_slots():
    rng = np.random.default_rng(3)
    e, n, k = 4, 256, 384
    x = O.bf16_round(rng.standard_normal((5, k)).astype(np.float32))
    tables = []
    for _ in range(2):
        bits = rng.integers(0, 0x7E, (e, n, k), dtype=np.uint8)
        scales = rng.uniform(0.001, 0.01, (e, n // 128, k // 128)).astype(np.float32)
        tables.append((bits, scales))
    ids = np.array([3, -2, 9, 1, 0], np.int32)
    owned = np.array([True, True, True, False, True])
    out = O.routed_projection(x, tuple(tables), ids, owned)
    assert out.shape == (5, 2, n)
    np.testing.assert_array_equal(out[3], 0)
    for s, expert in ((0, 3), (1, 0), (2, 3), (4, 0)):
        for t in range(2):
            ref = _fp64_dequant_dot(x[s:s + 1], tables[t][0][expert], tables[t][1][expert])[0]
            np.testing.assert_allclose(out[s, t], ref, rtol=1e-5, atol=1e-4)


# ----------------------------------------------------------------------------- SwiGLU and routed experts
def _swiglu_torch_stepwise(g, u):
    """tests/reference/linear.py:71-73 in torch bf16, one op at a time: each
    bf16 op computes in FP32 and rounds once."""
    gb = torch.from_numpy(np.asarray(g, np.float32)).to(torch.bfloat16)
    ub = torch.from_numpy(np.asarray(u, np.float32)).to(torch.bfloat16)
    s = torch.sigmoid(gb)
    gs = gb * s
    return (gs * ub).float().numpy()


def test_swiglu_rounds_after_every_op():
    g = O.bf16_round(np.linspace(-8, 8, 4097).astype(np.float32))
    u = O.bf16_round(np.float32(1.0) + np.zeros_like(g))
    np.testing.assert_array_equal(O.swiglu_bf16(g, np.zeros_like(g)), 0)
    np.testing.assert_array_equal(O.swiglu_bf16(g, u), _swiglu_torch_stepwise(g, u))
    # u != 1: the last product's rounding (and the rounding of g * sigmoid(g) before it)
    rng = np.random.default_rng(4)
    g = O.bf16_round((rng.standard_normal(1 << 16) * 4).astype(np.float32))
    u = O.bf16_round((rng.standard_normal(1 << 16) * 3).astype(np.float32))
    want = _swiglu_torch_stepwise(g, u)
    np.testing.assert_array_equal(O.swiglu_bf16(g, u), want)
    # planted mistakes the comparison must catch: g * sigmoid(g) not rounded
    # before the product with u, and the sigmoid not rounded before g * s
    s = O.bf16_round(O.sigmoid_f32(g))
    assert not np.array_equal(O.bf16_round(g * s * u), want)
    assert not np.array_equal(O.bf16_round(O.bf16_round(g * O.sigmoid_f32(g)) * u), want)


def _fp64_routed_slots(x, ids, w, tables, route_sum_scale=1.0):
    """tests/reference/independent.py:257-287 form: FP64 everywhere after the
    bf16 weight decode; every route's weighted down row, ``[T, k, H]``."""
    def dq(bits, scales):
        v = torch.from_numpy(bits).view(torch.float8_e4m3fn).double().numpy()
        ex = np.repeat(np.repeat(scales.astype(np.float64), 128, -2), 128, -1)
        return torch.from_numpy((v * ex).astype(np.float32)).to(torch.bfloat16).double().numpy()
    out = np.zeros((ids.shape[0], ids.shape[1], x.shape[1]))
    for t in range(ids.shape[0]):
        for s in range(ids.shape[1]):
            e = ids[t, s]
            gate = dq(tables["gate_bits"][e], tables["gate_scale"][e]) @ x[t]
            up = dq(tables["up_bits"][e], tables["up_scale"][e]) @ x[t]
            act = gate / (1 + np.exp(-gate)) * up
            out[t, s] = w[t, s] * route_sum_scale * (dq(tables["down_bits"][e], tables["down_scale"][e]) @ act)
    return out


def _fp64_routed(x, ids, w, tables, route_sum_scale=1.0):
    return _fp64_routed_slots(x, ids, w, tables, route_sum_scale).sum(axis=1)


def test_routed_experts_matches_fp64_restatement_and_catches_planted_mistakes():
    from glm_moe import synthetic as S

    cfg = S.CONFIGS["toy"]
    x = S.hidden_states(cfg, 0).astype(np.float64)
    ids, w = S.routes(cfg, 0)
    tables = S.host_expert_tables(cfg, 0)
    got, ok = O.routed_experts(x, ids, w, **tables)
    assert ok
    ref = _fp64_routed(x, ids, w, tables)
    bound = 0.015 * np.abs(ref).max()  # tests/reference/test_reference_consistency.py:659-742
    assert np.abs(got - ref).max() <= bound
    # planted mistakes in the oracle's arithmetic must exceed the same bound
    dropped_weight = _fp64_routed(x, ids, np.ones_like(w), tables)
    assert np.abs(dropped_weight - ref).max() > bound
    swapped = dict(tables, gate_bits=tables["up_bits"], up_bits=tables["gate_bits"],
                   gate_scale=tables["up_scale"], up_scale=tables["gate_scale"])
    assert np.abs(_fp64_routed(x, ids, w, swapped) - ref).max() > bound
    # the bf16 route sum stays within the same bound
    got_bf16, _ = O.routed_experts(x, ids, w, **tables, route_sum="bfloat16")
    assert np.abs(got_bf16 - ref).max() <= bound


def test_routed_experts_invalid_routes_follow_the_reference():
    from glm_moe import synthetic as S

    cfg = S.CONFIGS["toy"]
    x = S.hidden_states(cfg, 1)
    ids, w = S.routes(cfg, 1)
    tables = S.host_expert_tables(cfg, 1)
    bad = ids.copy()
    bad[2, 1] = 99  # out of range: computed as expert 0, health false
    out, ok = O.routed_experts(x, bad, w, **tables)
    assert not ok
    safe = bad.copy()
    safe[2, 1] = 0
    ref, _ = O.routed_experts(x, safe, w, **tables)
    np.testing.assert_array_equal(out, ref)
    dropped, _ = O.routed_experts(x, bad, w, **tables, drop_unowned=True)
    zero_w = w.copy()
    zero_w[2, 1] = 0.0
    ref_drop, _ = O.routed_experts(x, ids, zero_w, **tables)
    np.testing.assert_array_equal(dropped[[0, 1, 3]], ref_drop[[0, 1, 3]])
    neg = w.copy()
    neg[0, 0] = -0.5
    assert not O.routed_experts(x, ids, neg, **tables)[1]
    assert O.routed_experts(x, ids, neg, **tables, check_weights=False)[1]


def test_route_sum_rounds_the_fp32_sum_once():
    """The decode body's bf16 route sum ``jnp.sum(weighted, axis=0, dtype=bfloat16)``
    (routed_experts.py:293) is computed by JAX in FP32 and rounded once, so with
    every route on one owner it equals the prefill body's FP32 sum
    (tests/reference/moe.py:17-21).  Each slot's weighted row is isolated through
    the ownership mask (the other slots' ids out of range contribute zero); the
    oracle's output must be their FP32 slot-order sum rounded once, not a running
    bf16 sum -- which this top-8 case tells apart on many elements."""
    from glm_moe import synthetic as S

    cfg = S.MoeConfig("sum8", 3, 16, 256, 256, 8)
    x = S.hidden_states(cfg, 4)
    ids, w = S.routes(cfg, 4)
    tables = S.host_expert_tables(cfg, 4)
    per_slot = []
    for s in range(cfg.top_k):
        only = np.full_like(ids, cfg.experts + 5)
        only[:, s] = ids[:, s]
        part, _ = O.routed_experts(x, only, w, **tables, drop_unowned=True, check_weights=False)
        per_slot.append(part)  # bf16(down * bf16(w)) of slot s: already a bf16 value
    once = np.zeros_like(per_slot[0])
    running = np.zeros_like(per_slot[0])
    for part in per_slot:
        once += part
        running = O.bf16_round(running + part)
    once = O.bf16_round(once)
    decode, _ = O.routed_experts(x, ids, w, **tables, route_sum="bfloat16", drop_unowned=True, check_weights=False)
    prefill, _ = O.routed_experts(x, ids, w, **tables)
    np.testing.assert_array_equal(decode, once)
    np.testing.assert_array_equal(prefill, once)
    assert np.mean(running != once) > 0.05  # the running sum is a different (wrong) rule here


@pytest.mark.parametrize("drop_unowned", [False, True])
def test_expert_share_partial_is_the_layer_with_other_shares_weighted_zero(drop_unowned):
    """A share (tables of experts [offset, offset + E_local) of E, global ids)
    computes its owned routes only (routed_experts.py:85-93, panels.py:26-83):
    its FP32 partial equals the whole layer's FP32 route sum with every other
    share's route weights set to zero, bit for bit (adding zeros in slot order
    changes no FP32 sum), and the shares' partials add up to the whole layer."""
    from glm_moe import synthetic as S

    cfg = S.MoeConfig("share", 6, 8, 256, 256, 3)
    x = S.hidden_states(cfg, 6)
    ids, w = S.routes(cfg, 6)
    ids = ids.copy()
    ids[4, 2] = 9  # invalid: safe id 0 (owned by the share at offset 0), or dropped
    tables = S.host_expert_tables(cfg, 6)
    kw = dict(drop_unowned=drop_unowned, check_weights=False)
    whole, whole_ok = O.routed_experts(x, ids, w, **tables, round_output=False, **kw)
    assert not whole_ok
    safe = np.where((ids >= 0) & (ids < 8), ids, -1 if drop_unowned else 0)
    total = np.zeros_like(whole)
    for rank in range(4):  # four shares of two experts
        lo = 2 * rank
        share_tables = {k: v[lo:lo + 2] for k, v in tables.items()}
        part, ok = O.routed_experts(x, ids, w, **share_tables, num_experts=8, expert_offset=lo, round_output=False,
                                    **kw)
        assert ok == whole_ok
        masked = np.where((safe >= lo) & (safe < lo + 2), w, np.float32(0.0)).astype(np.float32)
        ref, _ = O.routed_experts(x, ids, masked, **tables, round_output=False, **kw)
        np.testing.assert_array_equal(part, ref)
        total += part
    np.testing.assert_allclose(total, whole, rtol=1e-6, atol=1e-6)


def _fp64_shared(x, shared):
    g = x @ shared[0].astype(np.float64).T
    u = x @ shared[1].astype(np.float64).T
    return (g / (1 + np.exp(-g)) * u) @ shared[2].astype(np.float64).T


def test_moe_layer_matches_fp64_restatement_and_catches_planted_mistakes():
    """Whole layer ``bf16(bf16(routed) * bf16(2.5) + shared)`` (routed_experts.py:
    119-127 / :297-304) against an FP64 restatement (tests/reference/independent.py:
    257-287 form) within 1.5 % of max (tests/reference/test_reference_consistency.py:
    659-742); dropping the routed scale or swapping the shared gate and up tables
    must exceed that bound."""
    from glm_moe import synthetic as S

    cfg = S.CONFIGS["toy"]
    x = S.hidden_states(cfg, 2).astype(np.float64)
    ids, w = S.routes(cfg, 2)
    tables = S.host_expert_tables(cfg, 2)
    rng = np.random.default_rng(21)
    # shared weights scaled so that the shared output is as large as the routed one
    shared = [O.bf16_round((rng.standard_normal(s) * std).astype(np.float32))
              for s, std in (((256, 256), 0.0625), ((256, 256), 0.0625), ((256, 256), 0.005))]
    got, ok = O.moe_layer(x, ids, w, *tables.values(), *shared)
    assert ok
    routed = _fp64_routed(x, ids, w, tables)
    shared_out = _fp64_shared(x, shared)
    assert np.abs(shared_out).max() > 0.3 * np.abs(2.5 * routed).max()  # both halves matter
    ref = 2.5 * routed + shared_out
    bound = 0.015 * np.abs(ref).max()
    assert np.abs(got - ref).max() <= bound
    assert np.abs((routed + shared_out) - ref).max() > bound  # the x2.5 dropped
    swapped = _fp64_shared(x, [shared[1], shared[0], shared[2]])
    assert np.abs((2.5 * routed + swapped) - ref).max() > bound  # shared gate / up swapped
    # the decode body (unowned dropped, per-owner bf16 sum) on all-owned routes: the same bits
    dec, _ = O.moe_layer(x, ids, w, *tables.values(), *shared, decode=True)
    np.testing.assert_array_equal(dec, got)
    # the magnitude the parity checks scale rounding flips by: the same output,
    # and per element at least |output|, |2.5 x routed|, |shared| and every
    # route's 2.5 x |bf16(down * w)| (FP64 restatement, so within its tolerance)
    same, _, mag = O.moe_layer(x, ids, w, *tables.values(), *shared, return_magnitude=True)
    np.testing.assert_array_equal(same, got)
    assert np.all(mag >= np.abs(got))
    assert np.all(mag >= 2.5 * np.abs(routed) - bound) and np.all(mag >= np.abs(shared_out) - bound)
    _, _, route_max = O.routed_experts(x, ids, w, **tables, return_route_max=True)
    per_route = np.abs(_fp64_routed_slots(x, ids, w, tables)).max(axis=1)
    assert np.abs(route_max - per_route).max() <= 0.015 * per_route.max()


# ----------------------------------------------------------------------------- router
def test_noaux_bias_selects_but_does_not_weight():
    # reference tests/layers/moe/test_router.py:100-107
    logits = np.array([[3.0, 2.0, 1.0, 0.0]], np.float32)
    bias = np.array([0.0, 0.0, 100.0, 99.0], np.float32)
    idx, w = O.route_glm_noaux_tc_logits(logits, bias, top_k=2)
    np.testing.assert_array_equal(idx, [[2, 3]])
    s = 1 / (1 + np.exp(-np.array([1.0, 0.0])))
    np.testing.assert_allclose(w[0], s / s.sum(), rtol=1e-6)


def test_router_ties_choose_lowest_expert_ids():
    # reference tests/layers/moe/test_router.py:110-114
    idx, w = O.route_glm_noaux_tc_logits(np.zeros((1, 16), np.float32), np.zeros(16, np.float32), top_k=8)
    np.testing.assert_array_equal(idx, [list(range(8))])
    np.testing.assert_array_equal(w, np.full((1, 8), 0.125, np.float32))


def _brute_force_route(logits, bias, top_k):
    """An independent restatement of router.py:20-55 by brute force: each score
    is the FP64 logistic rounded to FP32, the biased score its FP32 sum with the
    bias, the selection the top_k largest (biased score, -id) pairs of a full
    Python sort (ties to the lowest id), and the weights FP64 ratios of the
    chosen unbiased scores.  Returns ids, weights and, per token, the gap between
    the k-th and (k+1)-th biased scores (where a last-bit sigmoid difference
    could swap the selection)."""
    ids, weights, gaps = [], [], []
    for row in np.asarray(logits, np.float64):
        scores = [np.float32(1.0 / (1.0 + math.exp(-v))) for v in row]
        biased = [np.float32(sc + np.float32(b)) for sc, b in zip(scores, bias)]
        pairs = sorted(((float(v), -e) for e, v in enumerate(biased)), reverse=True)
        chosen = [-e for _, e in pairs[:top_k]]
        total = math.fsum(float(scores[e]) for e in chosen)
        ids.append(chosen)
        weights.append([float(scores[e]) / total for e in chosen])
        gaps.append(pairs[top_k - 1][0] - pairs[top_k][0] if top_k < len(pairs) else np.inf)
    return np.array(ids), np.array(weights), np.array(gaps)


def _router_agrees(got, want, gaps):
    """Ids equal wherever the selection is decided by more than 1e-6; weights
    within 4e-7 relative (a few FP32 ulps)."""
    idx, w = got
    ref_idx, ref_w, _ = want
    decided = gaps > 1e-6
    return bool(np.array_equal(idx[decided], ref_idx[decided])
                and np.allclose(w[decided], ref_w[decided], rtol=4e-7, atol=0))


def test_sigmoid_is_the_fp32_logistic_within_four_ulps():
    """FP32 1 / (1 + exp(-x)) against the FP64 logistic: within 4 FP32 ulps
    (3.2 measured, at x < 0 where 1 + exp(-x) rounds), within 2 for x >= 0 (1.5);
    XLA's own last-bit rounding is not pinned (no JAX here)."""
    x = np.linspace(-30, 30, 600001).astype(np.float32)
    got = O.sigmoid_f32(x).astype(np.float64)
    exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulps = np.abs(got - exact) / np.spacing(exact.astype(np.float32)).astype(np.float64)
    assert ulps.max() <= 4
    assert ulps[x >= 0].max() <= 2


@pytest.mark.parametrize("experts,top_k,zipf,biased", [(16, 4, 0.0, False), (64, 8, 0.0, True), (256, 8, 1.2, True)])
def test_router_matches_brute_force_and_catches_planted_mistakes(experts, top_k, zipf, biased):
    """The oracle router against the brute force above on seeded logits, and
    three mistakes planted in copies of the oracle that the comparison must
    catch: weights from the biased scores, selection on the unbiased scores,
    and the selection order without the bias's effect on ties."""
    from glm_moe import synthetic as S

    cfg = S.MoeConfig("router", 96, experts, 128, 128, top_k, zipf)
    logits = S.router_logits(cfg, 3)
    rng = np.random.default_rng(experts)
    bias = (rng.standard_normal(experts) * 0.05).astype(np.float32) if biased else np.zeros(experts, np.float32)
    want = _brute_force_route(logits, bias, top_k)
    assert np.mean(want[2] > 1e-6) > 0.95
    got = O.route_glm_noaux_tc_logits(logits, bias, top_k)
    assert _router_agrees(got, want, want[2])
    if biased:
        # planted: the weights normalise the biased scores
        scores = O.sigmoid_f32(logits)
        b = (scores + bias[None, :]).astype(np.float32)
        chosen = np.take_along_axis(b, got[0], axis=-1)
        assert not _router_agrees((got[0], chosen / chosen.sum(-1, keepdims=True)), want, want[2])
        # planted: the selection ignores the bias
        assert not _router_agrees(O.route_glm_noaux_tc_logits(logits, np.zeros_like(bias), top_k), want, want[2])


def test_router_ties_brute_force_and_planted_highest_id():
    """Exact ties (integer logits, zero bias): the brute force and the oracle take
    the lowest ids; a copy of the oracle that breaks ties to the highest id
    (run on the experts in reverse order) is caught."""
    rng = np.random.default_rng(11)
    logits = rng.integers(-2, 3, (64, 32)).astype(np.float32)
    bias = np.zeros(32, np.float32)
    want = _brute_force_route(logits, bias, 6)
    got = O.route_glm_noaux_tc_logits(logits, bias, 6)
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_allclose(got[1], want[1], rtol=4e-7, atol=0)
    rev_idx, rev_w = O.route_glm_noaux_tc_logits(logits[:, ::-1].copy(), bias, 6)
    assert not np.array_equal(31 - rev_idx, want[0])


def test_synthetic_router_agrees_with_oracle_router():
    """The bench's input generator routes as the oracle does (both are checked
    against the brute force above, not against each other alone)."""
    from glm_moe import synthetic as S

    for name in ("toy", "decode_t4", "prefill_t8192_zipf"):
        cfg = S.CONFIGS[name]
        if cfg.tokens > 64:
            cfg = S.MoeConfig(cfg.name, 64, cfg.experts, cfg.hidden, cfg.intermediate, cfg.top_k, cfg.zipf)
        logits = S.router_logits(cfg, 7)
        a = S.noaux_tc_route(logits, None, cfg.top_k)
        b = O.route_glm_noaux_tc_logits(logits, np.zeros(cfg.experts, np.float32), cfg.top_k)
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1], b[1])
        want = _brute_force_route(logits, np.zeros(cfg.experts, np.float32), cfg.top_k)
        assert _router_agrees(a, want, want[2])


# ----------------------------------------------------------------------------- native FP8 mode (no reference counterpart)
def test_fp8_activation_quantization_known_answers():
    # block 0: amax 448 -> scale 1, values already on the e4m3 grid stay exact;
    # block 1: all zero -> scale 1, zeros; block 2: amax 2 -> scale 2/448, its
    # largest value maps to exactly 448 and the rest round to nearest even
    x = np.zeros((1, 3 * 128), np.float32)
    grid = O.fp8_e4m3fn_table()[np.arange(0, 127, dtype=np.uint8)]  # positive finite codes 0..126
    x[0, :127] = grid
    x[0, 127] = -448.0
    x[0, 256] = 2.0
    x[0, 257] = -1.0
    x[0, 258] = 2.0 * 17.0 / 448.0  # 17 lies between e4m3 16 and 18: a tie, rounds to even (16)
    q, s = O.quantize_rows_fp8(x)
    np.testing.assert_array_equal(s[0], np.float32([1.0, 1.0, 2.0 / 448.0]))
    np.testing.assert_array_equal(q[0, :127], grid)
    assert q[0, 127] == -448.0
    assert not np.any(q[0, 128:256])
    assert q[0, 256] == 448.0 and q[0, 257] == -224.0 and q[0, 258] == 16.0


def test_block_dot_fp8_is_exact_block_products_times_scales():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 126, (256, 256), dtype=np.uint8)  # finite codes only
    bits[bits == 0x7F] = 0
    wscale = rng.uniform(0.5, 2.0, (2, 2)).astype(np.float32)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    xq, xs = O.quantize_rows_fp8(x)
    got = O.block_dot_fp8(xq, xs, bits, wscale)
    # closed form in FP64: sum over blocks of (exact block dot) * w scale * x scale
    w = O.fp8_e4m3fn_table()[bits].astype(np.float64)
    ref = np.zeros((3, 256))
    for kb in range(2):
        sl = slice(128 * kb, 128 * kb + 128)
        ref += (xq[:, sl].astype(np.float64) @ w[:, sl].T) * np.repeat(wscale[:, kb], 128)[None, :] * xs[:, kb:kb + 1]
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # and it approximates the dequantised FP32 product to e4m3 precision
    dense = x @ (O.fp8_e4m3fn_table()[bits] * np.repeat(np.repeat(wscale, 128, 0), 128, 1)).T
    assert np.abs(got - dense).max() < 0.1 * np.abs(dense).max()
