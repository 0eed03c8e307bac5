"""CPU restatement (numpy) of glm-tpu's routed-expert MoE path.

TEST INFRASTRUCTURE ONLY.  This module is the parity checker for the HIP
implementation in ``glm-tpu_amd``.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker (or the timed CPU baseline), never as a code path of the product.

Every function restates one function of the reference (``/root/reference``,
GianluigiVitale/glm-tpu) and cites the file:line it follows.  The reference is
JAX/Pallas; JAX, jaxlib and ml_dtypes are not installed here, so nothing of it
is imported or executed.  Numerics follow the reference's arithmetic boundaries:

* e4m3fn bits decode exactly, are multiplied by the FP32 block scale in FP32 and
  rounded once (RNE) to bf16 (``glm_tpu/layers/fp8.py:113-126``);
* projections multiply bf16-valued operands exactly and accumulate in FP32 in
  ascending 128-wide K blocks (``kernel.py:209-235``, ``panel_kernel.py:83-99``);
* the SwiGLU rounds to bf16 after each elementwise op
  (``tests/reference/linear.py:71-73``);
* routed outputs are weighted in bf16 and summed over the top-k slots in FP32,
  rounded once (``routed_experts.py:104-117``, ``tests/reference/moe.py:95-99``).

How each function is pinned (checked by ``tests/test_oracle.py``):

* ``fp8_e4m3fn_table`` / ``decode_fp8_table``: the closed form of the table is
  checked against torch's independent ``float8_e4m3fn`` decoder for all 256 bit
  patterns, the KATs 0x38 = 1.0, 0x7E = 448, 0x7F/0xFF = NaN, and bf16 rounding
  against torch's ``bfloat16`` cast on random and tie-case inputs.
* ``group_prefill_routes``: brute force (np.argsort stable, np.bincount, inverse
  by scatter) is the reference's own test oracle
  (``tests/layers/moe/test_routed_experts.py:23-25``); invalid-id and
  duplicate-id KATs (``:40-44``).
* ``build_expert_panels`` / pack / unpack: the reference's invariant tests
  (``tests/kernels/test_fp8_panel_matmul.py:31-78,140-151``): restore-once,
  zero padding, NaN-poisoned padding does not leak, active = sum ceil(c/32),
  invalid metadata gives no panels, the 129-row closed form.
* ``panel_fp8_matmul`` / ``routed_projection``: the closed forms (all 0x38 bits x
  ones = K exactly; scale 0 gives 0), and an FP64 brute-force restatement with a
  different contraction order (tolerances of ``test_fp8_panel_matmul.py:131-137``).
* ``routed_experts`` / the layer compositions: an independent FP64 restatement
  (``tests/reference/independent.py:257-287`` form) within the 1.5 %-of-max bound
  of ``tests/reference/test_reference_consistency.py:659-742``, plus a planted
  mistake (dropped route weight, swapped gate/up) that the check must catch.
* ``route_glm_noaux_tc_logits``: the reference KATs
  (``tests/layers/moe/test_router.py:51-65``): bias selects but does not weight,
  ties choose the lowest ids with weights 0.125.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from typing import NamedTuple

import numpy as np

BLOCK = 128


# ----------------------------------------------------------------------------- scalar formats
def fp8_e4m3fn_table() -> np.ndarray:
    """The exact 256-entry E4M3FN decode table (``glm_tpu/layers/fp8.py:18-34``)."""
    values = np.empty(256, np.float64)
    for bits in range(256):
        sign = -1.0 if bits & 0x80 else 1.0
        exponent = (bits >> 3) & 0xF
        mantissa = bits & 0x7
        if exponent == 0:
            value = mantissa * 2.0**-9
        elif exponent == 15 and mantissa == 7:
            value = float("nan")
        else:
            value = (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
        values[bits] = sign * value
    return values.astype(np.float32)  # every entry is exact in FP32


_E4M3 = fp8_e4m3fn_table()


def bf16_round(x) -> np.ndarray:
    """Round FP32 values to bf16 (RNE), returned as FP32 holding bf16 values.

    The ``.astype(jnp.bfloat16)`` of the reference (e.g. ``fp8.py:126``).
    NaN stays NaN; +-inf stay infinite; overflow past bf16's max rounds to inf.
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    # uint32 arithmetic wraps only for NaN patterns (>= 0xFFFF8000), restored below
    rounded = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)
    out = rounded.view(np.float32)
    nan = np.isnan(f)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def bf16_bits(x) -> np.ndarray:
    """bf16 bit patterns (uint16) of FP32 values, after RNE rounding."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    """FP32 values of bf16 bit patterns (uint16)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def sigmoid_f32(x) -> np.ndarray:
    """FP32 logistic ``1 / (1 + exp(-x))`` (``jax.nn.sigmoid`` call sites, ``router.py:40``)."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


# ----------------------------------------------------------------------------- FP8 block decode
def decode_fp8_table(bits, scale, block_shape=(BLOCK, BLOCK)) -> np.ndarray:
    """``bf16(f32(e4m3(bits)) * scale[n // bn, k // bk])`` as FP32 values.

    ``glm_tpu/layers/fp8.py:113-126`` (and ``dequantize_fp8_bits_block_weight``
    ``:37-72`` for leading expert dimensions).
    """
    bits = np.asarray(bits, np.uint8)
    scale = np.asarray(scale, np.float32)
    bn, bk = block_shape
    n, k = bits.shape[-2:]
    if bits.ndim == 2 and n % bn == 0 and k % bk == 0 and scale.shape == (n // bn, k // bk):
        # whole blocks: broadcast each block's scale over its bn x bk values
        values = _E4M3[bits].reshape(n // bn, bn, k // bk, bk)
        values *= scale[:, None, :, None]
        return bf16_round(values.reshape(n, k))
    expanded = np.repeat(np.repeat(scale, bn, axis=-2), bk, axis=-1)[..., :n, :k]
    return bf16_round(_E4M3[bits] * expanded)


# ----------------------------------------------------------------------------- route grouping
class PrefillRoutes(NamedTuple):
    """``routed_experts.py:130-136``."""

    sorted_flat_ids: np.ndarray
    inverse_permutation: np.ndarray
    group_sizes: np.ndarray
    valid: bool


def group_prefill_routes(route_indices, num_experts: int = 256) -> PrefillRoutes:
    """Stable grouping of the flat routes by expert (``routed_experts.py:139-164``).

    ``flat = ids.reshape(-1)`` (index ``t * k + slot``); invalid ids become 0 for
    the metadata only; ``valid`` requires every id in range and no duplicate id
    within one token's row.
    """
    ids = np.asarray(route_indices)
    if ids.ndim != 2 or min(ids.shape) <= 0:
        raise ValueError("routes must be nonempty [tokens,top_k]")
    if ids.dtype != np.int32:
        raise ValueError("routes must be int32")
    if ids.shape[1] > num_experts:
        raise ValueError("top_k exceeds expert count")
    flat = ids.reshape(-1)
    valid_ids = (flat >= 0) & (flat < num_experts)
    ordered = np.sort(ids, axis=1)
    unique = bool(np.all(ordered[:, 1:] != ordered[:, :-1]))
    valid = bool(np.all(valid_ids)) and unique
    safe = np.where(valid_ids, flat, 0)
    order = np.argsort(safe, kind="stable").astype(np.int32)
    inverse = np.zeros_like(order)
    inverse[order] = np.arange(flat.size, dtype=np.int32)
    counts = np.bincount(safe, minlength=num_experts).astype(np.int32)
    return PrefillRoutes(order, inverse, counts, valid)


def gather_prefill_route_rows(hidden, routes: PrefillRoutes, top_k: int) -> np.ndarray:
    """``routed_experts.py:167-171``."""
    return np.asarray(hidden)[routes.sorted_flat_ids // top_k]


def restore_prefill_route_rows(sorted_values, routes: PrefillRoutes, top_k: int) -> np.ndarray:
    """``routed_experts.py:174-183``."""
    values = np.asarray(sorted_values)
    return values[routes.inverse_permutation].reshape(-1, top_k, values.shape[-1])


# ----------------------------------------------------------------------------- panels
class ExpertPanels(NamedTuple):
    """``kernels/fp8_grouped_matmul/panels.py:14-23``."""

    expert_ids: np.ndarray
    row_starts: np.ndarray
    live_counts: np.ndarray
    active_panels: int
    restore_indices: np.ndarray
    owned_rows: np.ndarray
    valid: bool


def build_expert_panels(group_sizes, group_offset: int, rows: int, local_groups: int, panel_rows: int = 32) -> ExpertPanels:
    """Expert-relative panels of ``panel_rows`` sorted rows (``panels.py:26-83``).

    The reference fixes ``panel_rows = 32``; capacity is
    ``ceil(rows / panel_rows) + local_groups - 1``.
    """
    sizes = np.asarray(group_sizes)
    if (
        type(rows) is not int
        or type(local_groups) is not int
        or min(rows, local_groups) <= 0
        or sizes.ndim != 1
        or sizes.size < local_groups
        or sizes.dtype != np.int32
        or (rows + panel_rows - 1) * sizes.size > 2147483647
    ):
        raise ValueError("expert panels require bounded rows and int32 group counts")
    g = sizes.size
    offset_raw = int(group_offset)
    valid = bool(
        np.all((sizes >= 0) & (sizes <= rows))
        and int(sizes.astype(np.int64).sum()) == rows
        and offset_raw >= 0
        and offset_raw <= g - local_groups
    )
    counts = np.where(valid, sizes, 0).astype(np.int64)
    offset = min(max(offset_raw, 0), g - local_groups)
    ends = np.cumsum(counts)
    starts = ends - counts
    local_ids = offset + np.arange(local_groups)
    local_counts = counts[local_ids]
    panel_counts = (local_counts + panel_rows - 1) // panel_rows
    panel_ends = np.cumsum(panel_counts)
    panel_starts = panel_ends - panel_counts
    capacity = (rows + panel_rows - 1) // panel_rows + local_groups - 1
    panel = np.arange(capacity)
    expert = np.clip(np.searchsorted(panel_ends, panel, side="right"), 0, local_groups - 1)
    within = (panel - panel_starts[expert]) * panel_rows
    active = panel < panel_ends[-1]
    row_starts = np.where(active, starts[local_ids[expert]] + within, 0)
    live = np.where(active, np.clip(local_counts[expert] - within, 0, panel_rows), 0)
    row = np.arange(rows)
    row_expert = np.clip(np.searchsorted(ends, row, side="right"), 0, g - 1)
    owned = valid & (row_expert >= offset) & (row_expert < offset + local_groups)
    local_row_expert = np.clip(row_expert - offset, 0, local_groups - 1)
    relative_row = row - starts[row_expert]
    restore = panel_starts[local_row_expert] * panel_rows + relative_row
    return ExpertPanels(
        np.where(active, expert, 0).astype(np.int32),
        row_starts.astype(np.int32),
        live.astype(np.int32),
        int(panel_ends[-1]),
        np.where(owned, restore, 0).astype(np.int32),
        owned.astype(bool),
        valid,
    )


def pack_expert_panel_rows(values, panels: ExpertPanels, panel_rows: int = 32) -> np.ndarray:
    """``panels.py:86-95``: gather ``[panel, panel_rows, feature]``, padding rows zero."""
    values = np.asarray(values)
    lane = np.arange(panel_rows)
    source = panels.row_starts[:, None] + lane[None, :]
    mask = lane[None, :] < panels.live_counts[:, None]
    gathered = values[np.clip(source, 0, values.shape[0] - 1)]
    return np.where(mask[..., None], gathered, np.zeros((), values.dtype))


def unpack_expert_panel_rows(values, panels: ExpertPanels) -> np.ndarray:
    """``panels.py:98-104``: restore sorted rows, zeros for unowned rows."""
    values = np.asarray(values)
    flat = values.reshape(-1, values.shape[-1])
    restored = flat[np.clip(panels.restore_indices, 0, flat.shape[0] - 1)]
    return np.where(panels.owned_rows[:, None], restored, np.zeros((), values.dtype))


# ----------------------------------------------------------------------------- projections
def block_dot_f32(x_bf16, w_bf16) -> np.ndarray:
    """``x @ w.T`` with FP32 accumulation in ascending 128-wide K blocks.

    The per-block update of ``kernel.py:214-235`` / ``panel_kernel.py:83-99``:
    operands are bf16-valued FP32 arrays, each block's dot is exact products
    accumulated in FP32, blocks are added in increasing K order.
    """
    x = np.asarray(x_bf16, np.float32)
    w = np.asarray(w_bf16, np.float32)
    k = x.shape[-1]
    acc = np.zeros((x.shape[0], w.shape[0]), np.float32)
    for kb in range(0, k, BLOCK):
        acc += x[:, kb : kb + BLOCK] @ w[:, kb : kb + BLOCK].T
    return acc


def _cast(value_f32, result_dtype: str) -> np.ndarray:
    if result_dtype == "float32":
        return np.asarray(value_f32, np.float32)
    if result_dtype == "bfloat16":
        return bf16_round(value_f32)
    raise ValueError("result must be float32 or bfloat16")


def panel_fp8_matmul(lhs, weight_bits, scale, panels: ExpertPanels, result_dtype: str = "float32"):
    """``prefill_panel_fp8_matmul`` (``panel_kernel.py:31-153``).

    Sorted bf16 rows ``[M, K]`` against their local expert's decoded weights;
    rows of unowned experts and every row of an invalid plan are zero.
    Returns ``(out [M, N], valid)``.
    """
    lhs = np.asarray(lhs, np.float32)
    bits = np.asarray(weight_bits, np.uint8)
    m = lhs.shape[0]
    n = bits.shape[1]
    out = np.zeros((m, n), np.float32)
    if not (panels.valid and panels.active_panels > 0):
        return _cast(out, result_dtype), panels.valid
    for p in range(panels.active_panels):
        e = int(panels.expert_ids[p])
        r0, live = int(panels.row_starts[p]), int(panels.live_counts[p])
        if live == 0:
            continue
        w = decode_fp8_table(bits[e], scale[e])
        out[r0 : r0 + live] = block_dot_f32(lhs[r0 : r0 + live], w)
    out = np.where(panels.owned_rows[:, None], out, np.float32(0))
    return _cast(out, result_dtype), panels.valid


def routed_projection(lhs, weights, local_expert_ids, owned, result_dtype: str = "float32") -> np.ndarray:
    """``fp8_routed_projection`` (``kernel.py:125-299``).

    ``lhs [slots, K]`` bf16 values, ``weights`` a tuple of one or two
    ``(bits [E, N, K], scale [E, N/128, K/128])`` pairs.  Ids are clipped to
    ``[0, E)`` (``:185``); unowned slots are exact zeros (``:237-240,280``).
    Returns ``[slots, tables, N]``.
    """
    lhs = np.asarray(lhs, np.float32)
    slots = lhs.shape[0]
    experts, n, _ = weights[0][0].shape
    ids = np.clip(np.asarray(local_expert_ids).astype(np.int64), 0, experts - 1)
    out = np.zeros((slots, len(weights), n), np.float32)
    for s in range(slots):
        if not owned[s]:
            continue
        for t, (bits, scale) in enumerate(weights):
            w = decode_fp8_table(bits[ids[s]], scale[ids[s]])
            out[s, t] = block_dot_f32(lhs[s : s + 1], w)[0]
    return _cast(out, result_dtype)


# ----------------------------------------------------------------------------- native FP8 mode
# The optional e4m3 x e4m3 mode of this library has no counterpart in the
# reference: activations are quantised per (row, 128-wide K block) and the
# block products are scaled in FP32.  These functions define it for its parity
# test; its error against the reference numerics is reported separately.
def quantize_rows_fp8(x) -> tuple[np.ndarray, np.ndarray]:
    """``(e4m3 values as f32 [rows, K], f32 scales [rows, K/128])``.

    scale = amax / 448 per block (1 for an all-zero block); q =
    e4m3fn(clamp(x / scale, +-448)) rounded to nearest even (torch's
    ``float8_e4m3fn`` cast, the independent decoder the table is pinned to).
    """
    import torch

    x = np.asarray(x, np.float32)
    rows, k = x.shape
    blocks = x.reshape(rows, k // BLOCK, BLOCK)
    amax = np.abs(blocks).max(axis=2)
    scale = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    v = np.clip(blocks / scale[:, :, None], np.float32(-448.0), np.float32(448.0)).astype(np.float32)
    q = torch.from_numpy(np.ascontiguousarray(v)).to(torch.float8_e4m3fn).to(torch.float32).numpy()
    return q.reshape(rows, k), scale


def block_dot_fp8(xq, xscale, bits, wscale) -> np.ndarray:
    """FP8-mode projection: per K block the exact e4m3 dot (FP64, one rounding to
    FP32) times ``wscale[n/128, kb] * xscale[row, kb]``, accumulated in FP32 in
    ascending K blocks.  ``bits`` are one expert's ``[N, K]`` e4m3 bytes."""
    xq = np.asarray(xq, np.float64)
    wq = _E4M3[np.asarray(bits, np.uint8)].astype(np.float64)
    n, k = wq.shape
    acc = np.zeros((xq.shape[0], n), np.float32)
    for kb in range(k // BLOCK):
        sl = slice(kb * BLOCK, (kb + 1) * BLOCK)
        p = (xq[:, sl] @ wq[:, sl].T).astype(np.float32)
        f = (np.repeat(np.asarray(wscale, np.float32)[:, kb], BLOCK)[None, :] *
             np.asarray(xscale, np.float32)[:, kb : kb + 1]).astype(np.float32)
        acc = (acc + p * f).astype(np.float32)
    return acc


def swiglu_bf16(gate_bf16, up_bf16) -> np.ndarray:
    """``(g * sigmoid(g) * u).astype(bf16)`` with a bf16 rounding after each op.

    ``routed_experts.py:102,280``; op-by-op rounding as in
    ``tests/reference/linear.py:71-73``.
    """
    g = bf16_round(gate_bf16)
    u = bf16_round(up_bf16)
    s = bf16_round(sigmoid_f32(g))
    return bf16_round(bf16_round(g * s) * u)


# ----------------------------------------------------------------------------- routed experts
def _blas_threads(n: int):
    """Context limiting the BLAS thread pool to n threads (no-op without threadpoolctl)."""
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        from contextlib import nullcontext

        return nullcontext()
    return threadpool_limits(limits=n, user_api="blas")


def routed_experts(hidden, route_indices, route_weights, gate_bits, gate_scale, up_bits, up_scale,
                   down_bits, down_scale, route_sum: str = "float32", check_weights: bool = True,
                   drop_unowned: bool = False, activations: str = "bfloat16", workers: int | None = None,
                   num_experts: int | None = None, expert_offset: int = 0, round_output: bool = True,
                   return_route_max: bool = False):
    """The routed half of the MoE layer, returned as ``(bf16 [T, H] values, valid)``.

    ``prefill_moe_from_routes`` (``routed_experts.py:82-117``) on one device
    (every mesh axis of size 1, so both ``psum`` are the identity): group the
    routes, FP32 gate/up projections, bf16 SwiGLU, bf16 down projection, bf16
    route weighting, restore, FP32 sum over the top-k slots, one bf16 rounding.
    ``route_sum="bfloat16"`` is the decode body's per-owner sum
    (``routed_experts.py:293``, ``jnp.sum(weighted, axis=0, dtype=bfloat16)``):
    JAX computes a bf16 ``sum`` in FP32 and rounds the result once (jax 0.10.1,
    ``jax/_src/numpy/reductions.py``: ``sum`` is a reduction with
    ``upcast_f16_for_computation=True``), so one owner's partial is the FP32
    sum rounded once.  On one device every route has the same owner and the
    two modes agree bit for bit, as ``tests/reference/moe.py:17-21`` states
    (they differ only when a row's routes are split over owners).

    ``valid`` is ``routes.valid`` (ids in range, no duplicate id in a row) and,
    with ``check_weights``, finite non-negative weights (``:83``).  As in the
    reference the output is computed for an invalid set too, with the safe ids
    of ``group_prefill_routes`` (an out-of-range id counts as expert 0).  With
    ``drop_unowned`` a route whose id is outside ``[0, E)`` contributes zero
    instead: the decode body's ownership mask (``routed_experts.py:250-253``)
    on one device.

    Each selected expert is decoded once, by one of ``workers`` threads (default:
    the usable cores, at most 16), so memory stays bounded at full shapes.

    ``activations="float8_e4m3fn"`` is this library's native FP8 mode (no
    reference counterpart): token rows and SwiGLU activations are quantised by
    ``quantize_rows_fp8`` and every projection is ``block_dot_fp8``.

    An expert-parallel share: the tables hold the experts ``[expert_offset,
    expert_offset + E_local)`` of ``num_experts`` and the ids are global.  The
    routes are grouped over every expert (validity and safe ids as above); only
    the owned experts' routes are computed (the owned panels of
    ``build_expert_panels`` with ``offset = axis_index("expert") * local_experts``,
    ``routed_experts.py:85-93``, ``panels.py:26-83``), the others contribute zero.
    ``round_output=False`` returns the share's partial before the sum over the
    expert axis: the FP32 route sum, or with ``route_sum="bfloat16"`` that sum
    rounded to bf16 (the decode body's per-owner sum, ``:293-295``).

    ``return_route_max=True`` appends ``max over slots |bf16(down * w)|`` per
    output element (FP32 ``[T, H]``): the largest bf16-rounded value the
    element's sum passes through, the scale of a one-ulp rounding difference
    in any of its routes.
    """
    x = bf16_round(np.asarray(hidden, np.float32))
    ids = np.asarray(route_indices, np.int32)
    w = np.asarray(route_weights, np.float32)
    t, k = ids.shape
    local = np.asarray(gate_bits).shape[0]
    experts = local if num_experts is None else int(num_experts)
    if not 0 <= expert_offset <= experts - local:
        raise ValueError("the share's experts lie outside [0, num_experts)")
    routes = group_prefill_routes(ids, num_experts=experts)
    valid = routes.valid
    if check_weights:
        valid = valid and bool(np.all(np.isfinite(w) & (w >= 0)))
    h = x.shape[1]
    sorted_ids = routes.sorted_flat_ids
    offsets = np.concatenate([[0], np.cumsum(routes.group_sizes)])
    weighted = np.zeros((t * k, h), np.float32)  # flat (token, slot) order
    wr = bf16_round(w.reshape(-1))
    if activations not in ("bfloat16", "float8_e4m3fn"):
        raise ValueError("activations must be bfloat16 or float8_e4m3fn")
    if route_sum not in ("float32", "bfloat16"):
        raise ValueError("route_sum must be float32 or bfloat16")
    fp8 = activations == "float8_e4m3fn"
    if fp8:
        xq, xs = quantize_rows_fp8(x)

    def expert_rows(e: int) -> None:
        # every route of global expert e (table e - expert_offset); routes of
        # different experts fill disjoint rows
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        flat = sorted_ids[r0:r1]
        e = e - expert_offset
        if fp8:
            tok = flat // k
            gate = bf16_round(block_dot_fp8(xq[tok], xs[tok], gate_bits[e], gate_scale[e]))
            up = bf16_round(block_dot_fp8(xq[tok], xs[tok], up_bits[e], up_scale[e]))
            act = swiglu_bf16(gate, up)
            aq, ascale = quantize_rows_fp8(act)
            down = bf16_round(block_dot_fp8(aq, ascale, down_bits[e], down_scale[e]))
        else:
            rows = x[flat // k]
            gate = bf16_round(block_dot_f32(rows, decode_fp8_table(gate_bits[e], gate_scale[e])))
            up = bf16_round(block_dot_f32(rows, decode_fp8_table(up_bits[e], up_scale[e])))
            act = swiglu_bf16(gate, up)
            down = bf16_round(block_dot_f32(act, decode_fp8_table(down_bits[e], down_scale[e])))
        weighted[flat] = bf16_round(down * wr[flat][:, None])

    used = [e for e in range(expert_offset, expert_offset + local) if offsets[e + 1] > offsets[e]]
    if workers is None:
        workers = min(16, len(os.sched_getaffinity(0)))
    if workers > 1 and len(used) > 1:
        # numpy releases the GIL in the decode and the BLAS calls; one BLAS thread
        # per worker (nested BLAS thread pools oversubscribe the cores)
        with _blas_threads(1), ThreadPoolExecutor(max_workers=min(workers, len(used))) as pool:
            list(pool.map(expert_rows, used))
    else:
        for e in used:
            expert_rows(e)
    if drop_unowned:
        owned = ((ids >= 0) & (ids < experts)).reshape(-1)
        weighted[~owned] = 0.0
    per_slot = weighted.reshape(t, k, h)
    # both route sums: FP32 in slot order, one bf16 rounding (see above)
    total = np.zeros((t, h), np.float32)
    for s in range(k):
        total += per_slot[:, s]
    out = total if not round_output and route_sum == "float32" else bf16_round(total)
    if return_route_max:
        return out, valid, np.abs(per_slot).max(axis=1)
    return out, valid


def shared_expert(hidden, shared_gate, shared_up, shared_down) -> np.ndarray:
    """The bf16-resident shared expert (``routed_experts.py:119-124`` / ``:269-302``)."""
    x = bf16_round(np.asarray(hidden, np.float32))
    gate = bf16_round(block_dot_f32(x, bf16_round(shared_gate)))
    up = bf16_round(block_dot_f32(x, bf16_round(shared_up)))
    act = swiglu_bf16(gate, up)
    return bf16_round(block_dot_f32(act, bf16_round(shared_down)))


def moe_layer(hidden, route_indices, route_weights, gate_bits, gate_scale, up_bits, up_scale,
              down_bits, down_scale, shared_gate, shared_up, shared_down,
              routed_scaling_factor: float = 2.5, route_sum: str = "float32", decode: bool = False,
              return_magnitude: bool = False):
    """Whole layer ``bf16(bf16(routed) * bf16(2.5) + shared)`` (``routed_experts.py:125,303-304``).

    Returns ``(bf16 [T, H] values, valid)``; ``valid`` also requires a finite
    output (``:126``).  ``decode=True`` is ``moe_grouped_routes``: the
    per-owner bf16 route sum (one rounding of the FP32 sum, as in
    ``routed_experts``), unowned routes dropped, no health checks on the weights.

    ``return_magnitude=True`` appends, per output element, the largest
    magnitude among the bf16-rounded values it passes through (every route's
    ``bf16(down * w)`` scaled by 2.5, ``bf16(routed * 2.5)``, the shared
    expert's output, the output): the scale of a one-ulp rounding difference
    upstream.
    """
    routed, valid, route_max = routed_experts(hidden, route_indices, route_weights, gate_bits, gate_scale,
                                              up_bits, up_scale, down_bits, down_scale,
                                              route_sum="bfloat16" if decode else route_sum,
                                              check_weights=not decode, drop_unowned=decode,
                                              return_route_max=True)
    shared = shared_expert(hidden, shared_gate, shared_up, shared_down)
    scale = bf16_round(np.float32(routed_scaling_factor))
    scaled = bf16_round(routed * scale)
    out = bf16_round(scaled + shared)
    valid = bool(valid and np.all(np.isfinite(out)))
    if return_magnitude:
        return out, valid, np.maximum.reduce([route_max * scale, np.abs(scaled), np.abs(shared), np.abs(out)])
    return out, valid


# ----------------------------------------------------------------------------- router
def route_glm_noaux_tc_logits(router_logits, correction_bias, top_k: int = 8):
    """GLM ``noaux_tc`` selection (``glm_tpu/layers/moe/router.py:20-55``).

    FP32 sigmoid scores; the top-k of ``scores + bias`` with ties to the lowest
    id (``lax.top_k``); weights are the unbiased scores of the chosen experts
    normalised in FP32.
    """
    logits = np.asarray(router_logits, np.float32)
    scores = sigmoid_f32(logits)
    biased = (scores + np.asarray(correction_bias, np.float32)[None, :]).astype(np.float32)
    idx = np.argsort(-biased, axis=-1, kind="stable")[:, :top_k].astype(np.int32)
    chosen = np.take_along_axis(scores, idx, axis=-1)
    weights = (chosen / chosen.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return idx, weights
