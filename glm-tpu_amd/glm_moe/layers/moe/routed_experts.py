"""The routed-expert MoE layer bodies on one MI355X, backed by libglm_moe.

Mirrors ``glm_tpu/layers/moe/routed_experts.py`` of the reference with the same
names, parameter lists and arithmetic boundaries:

* ``prefill_moe_from_routes`` (``:27-128``): rows ``[T, H]`` -> (bf16 output, health);
* ``moe_grouped_routes`` (``:186-304``): the one-row decode body;
* ``PrefillRoutes`` / ``group_prefill_routes`` / ``gather_prefill_route_rows`` /
  ``restore_prefill_route_rows`` (``:130-183``).

The routed half runs as one HIP pipeline (``routed_experts`` below): a stable
counting-sort route plan, the fused gate/up FP8 projection with bf16 SwiGLU,
the down FP8 projection with bf16 route weighting, and the route combine.
Work is launched only for the experts the routes select.  On one GPU every
mesh axis has size 1: ``hidden_local`` is the full hidden state, every expert
is local and both ``psum`` of the reference are the identity.

The shared expert runs inside the two decode kernels for decode shapes
(``glm_moe_moe_layer_resident``: one pass over HBM for routed and shared
weights), else as torch bf16 GEMMs on the same GPU (hipBLASLt), at the
reference's rounding points; the epilogue ``routed * 2.5 + shared`` is always
fused into the library's route-sum kernel.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable
from typing import Any, NamedTuple

import torch

from glm_moe import _lib
from glm_moe.contracts import GlmMoeNumericalContract, single_gpu_contract
from glm_moe.kernels.fp8_grouped_matmul.kernel import RoutedProjectionConfig


class PrefillRoutes(NamedTuple):
    """Permutation metadata; ``valid`` MUST join the caller's serving health."""

    sorted_flat_ids: torch.Tensor
    inverse_permutation: torch.Tensor
    group_sizes: torch.Tensor
    valid: torch.Tensor


def group_prefill_routes(route_indices: torch.Tensor, *, num_experts: int = 256) -> PrefillRoutes:
    """Group by expert, preserving original token/slot order inside each group.

    Invalid dynamic ids or duplicate experts produce ``valid=False``; they are
    not silently admitted (``routed_experts.py:139-164``).
    """
    if route_indices.ndim != 2 or min(route_indices.shape) <= 0:
        raise ValueError("routes must be nonempty [tokens,top_k]")
    if route_indices.dtype != torch.int32:
        raise ValueError("routes must be int32")
    if not isinstance(num_experts, int) or isinstance(num_experts, bool) or num_experts <= 0:
        raise ValueError("num_experts must be a positive integer")
    if route_indices.shape[1] > num_experts:
        raise ValueError("top_k exceeds expert count")
    _lib.require_device(route_indices)
    tokens, top_k = route_indices.shape
    device = route_indices.device
    n = tokens * top_k
    order = torch.empty(n, dtype=torch.int32, device=device)
    inverse = torch.empty(n, dtype=torch.int32, device=device)
    counts = torch.empty(num_experts, dtype=torch.int32, device=device)
    valid = torch.empty((), dtype=torch.bool, device=device)
    scratch_bytes = int(_lib.lib().glm_moe_group_routes_workspace_bytes(tokens, top_k, num_experts))
    scratch = torch.empty(max(scratch_bytes, 1), dtype=torch.uint8, device=device)
    _lib.call(
        "glm_moe_group_routes",
        _lib.ptr(route_indices), tokens, top_k, num_experts, _lib.ptr(order), _lib.ptr(inverse),
        _lib.ptr(counts), _lib.ptr(valid), _lib.ptr(scratch), scratch.numel(), _lib.stream_of(route_indices),
    )
    return PrefillRoutes(order, inverse, counts, valid)


def _gather(values: torch.Tensor, index: torch.Tensor, div: int, rows: int) -> torch.Tensor:
    _lib.require_device(values, index)
    flat = values.reshape(values.shape[0], -1)
    row_bytes = flat.shape[1] * flat.element_size()
    if row_bytes % 4:
        raise ValueError("gathered rows must be a multiple of 4 bytes")
    out = torch.empty((rows, *values.shape[1:]), dtype=values.dtype, device=values.device)
    _lib.call("glm_moe_gather_rows", _lib.ptr(flat), flat.shape[0], row_bytes, _lib.ptr(index), div,
              _lib.ptr(None), rows, _lib.ptr(out), _lib.stream_of(values))
    return out


def gather_prefill_route_rows(hidden: torch.Tensor, routes: PrefillRoutes, *, top_k: int) -> torch.Tensor:
    """``hidden[sorted_flat_ids // top_k]`` (``routed_experts.py:167-171``)."""
    if hidden.ndim != 2 or top_k <= 0 or tuple(routes.sorted_flat_ids.shape) != (hidden.shape[0] * top_k,):
        raise ValueError("hidden and route geometry disagree")
    return _gather(hidden, routes.sorted_flat_ids, top_k, routes.sorted_flat_ids.numel())


def restore_prefill_route_rows(sorted_values: torch.Tensor, routes: PrefillRoutes, *, top_k: int) -> torch.Tensor:
    """``sorted_values[inverse].reshape(T, top_k, F)`` (``routed_experts.py:174-183``)."""
    if (
        sorted_values.ndim != 2
        or top_k <= 0
        or sorted_values.shape[0] != routes.inverse_permutation.numel()
        or sorted_values.shape[0] % top_k
    ):
        raise ValueError("sorted output and route geometry disagree")
    restored = _gather(sorted_values, routes.inverse_permutation, 1, sorted_values.shape[0])
    return restored.reshape(-1, top_k, sorted_values.shape[-1])


class RoutedTimings(NamedTuple):
    """Kernel times (ms) of one ``routed_experts`` call per stage, from HIP events
    the kernels record at their own start and end; a stage that ran no kernel
    (the decode path has no separate plan or combine) is 0."""

    plan: float
    gate_up: float
    down: float
    combine: float

    @property
    def total(self) -> float:
        return self.plan + self.gate_up + self.down + self.combine


class StageEvents:
    """A start and a stop HIP event for each of the four stages of ``routed_experts``."""

    STAGES = 4

    def __init__(self) -> None:
        import ctypes

        self._handles = []
        for _ in range(2 * self.STAGES):
            slot = ctypes.c_void_p()
            _lib.call("glm_moe_event_create", ctypes.byref(slot))
            self._handles.append(slot.value)
        self.array = (ctypes.c_void_p * (2 * self.STAGES))(*self._handles)
        self.timed = ctypes.c_uint32(0)

    def elapsed(self) -> RoutedTimings:
        import ctypes

        ms = []
        for i in range(self.STAGES):
            if not (self.timed.value >> i) & 1:
                ms.append(0.0)
                continue
            value = ctypes.c_float()
            _lib.call("glm_moe_event_elapsed_ms", ctypes.c_void_p(self._handles[2 * i]),
                      ctypes.c_void_p(self._handles[2 * i + 1]), ctypes.byref(value))
            ms.append(value.value)
        return RoutedTimings(*ms)

    def close(self) -> None:
        import ctypes

        for handle in self._handles:
            _lib.call("glm_moe_event_destroy", ctypes.c_void_p(handle))
        self._handles = []


# One growable workspace buffer per (device, stream) for the small (decode and
# short-prefill) calls: calls enqueued on one stream run in order, so they can
# share it; calls on different streams get different buffers and never race.
# A buffer grows to the largest such call seen on its stream and is kept until
# release_workspaces().  Workspaces above WORKSPACE_CACHE_MAX (long prefills:
# ~270 MB at T=2048, ~1.3 GB at T=8192) are taken from torch's caching
# allocator for the one call instead, so the memory goes back to torch's pool
# (stream-ordered, for any tensor) when the call has been enqueued, rather than
# staying held by this module; calls captured into a HIP graph take their own
# buffer from the graph's memory pool.
WORKSPACE_CACHE_MAX = 256 << 20
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def routed_workspace(tokens: int, top_k: int, num_experts: int, hidden: int, intermediate: int,
                     device: torch.device) -> torch.Tensor:
    """The workspace of ``routed_experts`` for a call on the current stream of
    ``device``: a slice of that stream's buffer, grown when a call needs more."""
    nbytes = max(int(_lib.lib().glm_moe_routed_experts_workspace_bytes(
        tokens, top_k, num_experts, hidden, intermediate)), 1)
    device = torch.device(device)
    if torch.cuda.is_current_stream_capturing() or nbytes > WORKSPACE_CACHE_MAX:
        # under HIP graph capture: a buffer of the graph's private memory pool,
        # which stays valid for every replay (a cached buffer could be regrown,
        # and so freed, while the graph still uses it); above the cache's limit:
        # torch's allocator, which reuses the block only for later work on this
        # stream once the caller drops it
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # the old buffer returns to torch's allocator in the order of its stream
        _WORKSPACES.pop(key, None)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws[:nbytes]


def release_workspaces() -> None:
    """Drop every cached workspace buffer (they return to torch's allocator)."""
    _WORKSPACES.clear()


def routed_experts(
    hidden: torch.Tensor,
    route_indices: torch.Tensor,
    route_weights: torch.Tensor,
    gate_bits: torch.Tensor,
    gate_scale: torch.Tensor,
    up_bits: torch.Tensor,
    up_scale: torch.Tensor,
    down_bits: torch.Tensor,
    down_scale: torch.Tensor,
    *,
    route_sum: str = "float32",
    check_weights: bool = True,
    drop_unowned: bool = False,
    activations: str = "bfloat16",
    out: torch.Tensor | None = None,
    events: StageEvents | None = None,
    shared: torch.Tensor | None = None,
    shared_tables: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    routed_scale: float = 2.5,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Routed experts of ``[T, H]`` bf16 rows: ``(bf16 [T, H], valid)``.

    The routed half of ``prefill_moe_from_routes`` (``routed_experts.py:82-117``):
    FP32 gate/up projections, bf16 SwiGLU, bf16 down projection, bf16 route
    weighting and the sum over the top-k slots in FP32 with one rounding
    (``route_sum="bfloat16"``, the decode body's per-owner bf16 sum, ``:293``,
    is computed by JAX in FP32 and rounded once, so on one device it gives the
    same output).

    ``activations="float8_e4m3fn"`` selects the native FP8 MFMA mode (no
    reference counterpart; prefill shapes only): token rows and SwiGLU
    activations are quantised per (row, 128-wide block) to e4m3 with an FP32
    scale, and the e4m3 x e4m3 block products are scaled in FP32.

    With ``shared`` (the shared expert's bf16 ``[T, H]`` output) the layer
    epilogue is fused into the kernel that finishes the route sum:
    ``bf16(bf16(routed * bf16(routed_scale)) + shared)`` (``:125``, ``:303``),
    and ``valid`` also requires a finite output (``:126``).  ``shared_tables``
    (its resident bf16 gate, up, down tables) instead computes the shared
    expert inside the same two decode kernels (decode shapes only:
    ``uses_decode_kernels``); it streams the shared weights once per row, so
    the layer bodies use it for a single row.
    """
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise ValueError("routed experts take bf16 [tokens, hidden] rows")
    tokens, h = hidden.shape
    if route_indices.ndim != 2 or route_indices.shape[0] != tokens or route_indices.dtype != torch.int32:
        raise ValueError("route indices must be int32 [tokens, top_k]")
    top_k = route_indices.shape[1]
    if tuple(route_weights.shape) != (tokens, top_k) or route_weights.dtype != torch.float32:
        raise ValueError("route weights must be float32 [tokens, top_k]")
    if gate_bits.ndim != 3 or gate_bits.dtype != torch.uint8:
        raise ValueError("expert gate bits must be uint8 [E, I, H]")
    experts, inter, gh = gate_bits.shape
    if gh != h or tuple(up_bits.shape) != (experts, inter, h) or tuple(down_bits.shape) != (experts, h, inter):
        raise ValueError("expert table geometry disagrees with the hidden size")
    if up_bits.dtype != torch.uint8 or down_bits.dtype != torch.uint8:
        raise ValueError("expert tables must be uint8 e4m3fn bits")
    for scale, rows, cols in ((gate_scale, inter, h), (up_scale, inter, h), (down_scale, h, inter)):
        if scale.dtype != torch.float32 or tuple(scale.shape) != (experts, rows // 128, cols // 128):
            raise ValueError("expert scales must be float32 [E, N/128, K/128]")
    if route_sum not in ("float32", "bfloat16"):
        raise ValueError("route_sum must be float32 or bfloat16")
    if activations not in ("bfloat16", "float8_e4m3fn"):
        raise ValueError("activations must be bfloat16 or float8_e4m3fn")
    if shared is not None:
        if tuple(shared.shape) != (tokens, h) or shared.dtype != torch.bfloat16 or not shared.is_contiguous():
            raise ValueError("shared expert rows must be contiguous bf16 [tokens, hidden]")
        if events is not None:
            raise ValueError("stage events time the routed experts alone")
    if shared_tables is not None:
        if shared is not None:
            raise ValueError("pass the shared expert's output or its tables, not both")
        if events is not None:
            raise ValueError("stage events time the routed experts alone")
        if (
            len(shared_tables) != 3
            or any(t.dtype != torch.bfloat16 or not t.is_contiguous() for t in shared_tables)
            or tuple(shared_tables[0].shape) != (inter, h)
            or tuple(shared_tables[1].shape) != (inter, h)
            or tuple(shared_tables[2].shape) != (h, inter)
        ):
            raise ValueError("resident shared expert tables must be contiguous bf16 [I, H], [I, H], [H, I]")
    _lib.require_device(hidden, route_indices, route_weights, gate_bits, gate_scale, up_bits, up_scale,
                        down_bits, down_scale, out, shared, *(shared_tables or ()))
    device = hidden.device
    if out is None:
        out = torch.empty((tokens, h), dtype=torch.bfloat16, device=device)
    elif tuple(out.shape) != (tokens, h) or out.dtype != torch.bfloat16:
        raise ValueError("out must be bf16 [tokens, hidden]")
    valid = torch.empty((), dtype=torch.bool, device=device)
    ws = routed_workspace(tokens, top_k, experts, h, inter, device)
    flags = 0
    if route_sum == "bfloat16":
        flags |= _lib.ROUTE_SUM_BF16
    if check_weights:
        flags |= _lib.CHECK_WEIGHTS
    if drop_unowned:
        flags |= _lib.DROP_UNOWNED
    if activations == "float8_e4m3fn":
        flags |= _lib.FP8_ACTIVATIONS
    args = [
        _lib.ptr(hidden), tokens, h, _lib.ptr(route_indices), _lib.ptr(route_weights), top_k, experts, inter,
        _lib.ptr(gate_bits), _lib.ptr(gate_scale), _lib.ptr(up_bits), _lib.ptr(up_scale), _lib.ptr(down_bits),
        _lib.ptr(down_scale), flags, _lib.ptr(out), _lib.ptr(valid), _lib.ptr(ws), ws.numel(),
    ]
    if shared_tables is not None:
        args[15:15] = [*(_lib.ptr(t) for t in shared_tables), inter, float(routed_scale)]
        _lib.call("glm_moe_moe_layer_resident", *args, _lib.stream_of(hidden))
    elif shared is not None:
        args[15:15] = [_lib.ptr(shared), float(routed_scale)]
        _lib.call("glm_moe_moe_layer", *args, _lib.stream_of(hidden))
    elif events is None:
        _lib.call("glm_moe_routed_experts", *args, _lib.stream_of(hidden))
    else:
        _lib.call("glm_moe_routed_experts_timed", *args, events.array, ctypes.byref(events.timed),
                  _lib.stream_of(hidden))
    return out, valid


def routed_experts_from_router_logits(
    hidden: torch.Tensor,
    router_logits: torch.Tensor,
    correction_bias: torch.Tensor | None,
    gate_bits: torch.Tensor,
    gate_scale: torch.Tensor,
    up_bits: torch.Tensor,
    up_scale: torch.Tensor,
    down_bits: torch.Tensor,
    down_scale: torch.Tensor,
    *,
    top_k: int = 8,
    route_sum: str = "float32",
    check_weights: bool = True,
    activations: str = "bfloat16",
    shared: torch.Tensor | None = None,
    routed_scale: float = 2.5,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Routing from the router logits, then the routed experts (and, with
    ``shared``, the fused layer epilogue): ``(bf16 [T, H], valid, route_indices,
    route_weights)``.

    Bit for bit ``route_glm_noaux_tc_logits`` (``router.py:20-55``) followed by
    ``routed_experts`` with its outputs, in one library call: on decode shapes
    with up to 256 experts the decode gate/up kernel routes its own token (no
    launch of its own); on the multi-workgroup prefill plan the router counts
    the plan's histogram rows on the way (router, then the plan's scatter);
    otherwise the router kernel runs ahead of the one-workgroup plan.
    """
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise ValueError("routed experts take bf16 [tokens, hidden] rows")
    tokens, h = hidden.shape
    if gate_bits.ndim != 3 or gate_bits.dtype != torch.uint8:
        raise ValueError("expert gate bits must be uint8 [E, I, H]")
    experts, inter, gh = gate_bits.shape
    if gh != h or tuple(up_bits.shape) != (experts, inter, h) or tuple(down_bits.shape) != (experts, h, inter):
        raise ValueError("expert table geometry disagrees with the hidden size")
    for scale, rows, cols in ((gate_scale, inter, h), (up_scale, inter, h), (down_scale, h, inter)):
        if scale.dtype != torch.float32 or tuple(scale.shape) != (experts, rows // 128, cols // 128):
            raise ValueError("expert scales must be float32 [E, N/128, K/128]")
    if router_logits.ndim != 2 or tuple(router_logits.shape) != (tokens, experts):
        raise ValueError(f"router_logits must have shape {(tokens, experts)}")
    if correction_bias is not None and tuple(correction_bias.shape) != (experts,):
        raise ValueError(f"correction_bias must have shape {(experts,)}")
    if not isinstance(top_k, int) or isinstance(top_k, bool) or not 0 < top_k <= min(experts, 64):
        raise ValueError("top_k must be in [1, min(num_experts, 64)]")
    if route_sum not in ("float32", "bfloat16") or activations not in ("bfloat16", "float8_e4m3fn"):
        raise ValueError("route_sum must be float32 or bfloat16; activations bfloat16 or float8_e4m3fn")
    if shared is not None and (tuple(shared.shape) != (tokens, h) or shared.dtype != torch.bfloat16
                               or not shared.is_contiguous()):
        raise ValueError("shared expert rows must be contiguous bf16 [tokens, hidden]")
    _lib.require_device(hidden, router_logits, correction_bias, gate_bits, gate_scale, up_bits, up_scale,
                        down_bits, down_scale, shared, out)
    device = hidden.device
    logits = router_logits.float().contiguous()
    bias = None if correction_bias is None else correction_bias.float().contiguous()
    if out is None:
        out = torch.empty((tokens, h), dtype=torch.bfloat16, device=device)
    elif tuple(out.shape) != (tokens, h) or out.dtype != torch.bfloat16:
        raise ValueError("out must be bf16 [tokens, hidden]")
    ids = torch.empty((tokens, top_k), dtype=torch.int32, device=device)
    weights = torch.empty((tokens, top_k), dtype=torch.float32, device=device)
    valid = torch.empty((), dtype=torch.bool, device=device)
    ws = routed_workspace(tokens, top_k, experts, h, inter, device)
    flags = ((_lib.ROUTE_SUM_BF16 if route_sum == "bfloat16" else 0) | (_lib.CHECK_WEIGHTS if check_weights else 0)
             | (_lib.FP8_ACTIVATIONS if activations == "float8_e4m3fn" else 0))
    _lib.call("glm_moe_moe_layer_from_router_logits", _lib.ptr(hidden), tokens, h, _lib.ptr(logits),
              _lib.ptr(bias), top_k, experts, inter, _lib.ptr(gate_bits), _lib.ptr(gate_scale), _lib.ptr(up_bits),
              _lib.ptr(up_scale), _lib.ptr(down_bits), _lib.ptr(down_scale), flags, _lib.ptr(shared),
              float(routed_scale), _lib.ptr(ids), _lib.ptr(weights), _lib.ptr(out), _lib.ptr(valid), _lib.ptr(ws),
              ws.numel(), _lib.stream_of(hidden))
    return out, valid, ids, weights


def routed_experts_share(
    hidden: torch.Tensor,
    route_indices: torch.Tensor,
    route_weights: torch.Tensor,
    gate_bits: torch.Tensor,
    gate_scale: torch.Tensor,
    up_bits: torch.Tensor,
    up_scale: torch.Tensor,
    down_bits: torch.Tensor,
    down_scale: torch.Tensor,
    *,
    num_experts: int,
    expert_offset: int,
    route_sum: str = "float32",
    check_weights: bool = True,
    drop_unowned: bool = False,
    activations: str = "bfloat16",
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """One expert-parallel share of the routed experts: ``(f32 [T, H] partial, valid)``.

    The tables hold the experts ``[expert_offset, expert_offset + E_local)`` of
    ``num_experts``; ``route_indices`` are global ids.  Only owned routes are
    computed.  The partial is the share's FP32 route sum (``route_sum="bfloat16"``:
    rounded to bf16 values, the decode body's per-owner sum,
    ``routed_experts.py:293``), to be summed over the expert axis (the
    reference's ``psum``, ``:113-117`` / ``:294-295``) and finished by
    ``moe_layer_epilogue``.  Owned panels follow ``panels.py:26-83`` with
    ``offset = axis_index("expert") * local_experts`` (``routed_experts.py:85-93``).
    """
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise ValueError("routed experts take bf16 [tokens, hidden] rows")
    tokens, h = hidden.shape
    if route_indices.ndim != 2 or route_indices.shape[0] != tokens or route_indices.dtype != torch.int32:
        raise ValueError("route indices must be int32 [tokens, top_k]")
    top_k = route_indices.shape[1]
    if tuple(route_weights.shape) != (tokens, top_k) or route_weights.dtype != torch.float32:
        raise ValueError("route weights must be float32 [tokens, top_k]")
    if gate_bits.ndim != 3 or gate_bits.dtype != torch.uint8:
        raise ValueError("expert gate bits must be uint8 [E_local, I, H]")
    local, inter, gh = gate_bits.shape
    if gh != h or tuple(up_bits.shape) != (local, inter, h) or tuple(down_bits.shape) != (local, h, inter):
        raise ValueError("expert table geometry disagrees with the hidden size")
    for scale, rows, cols in ((gate_scale, inter, h), (up_scale, inter, h), (down_scale, h, inter)):
        if scale.dtype != torch.float32 or tuple(scale.shape) != (local, rows // 128, cols // 128):
            raise ValueError("expert scales must be float32 [E_local, N/128, K/128]")
    if not 0 <= expert_offset <= num_experts - local:
        raise ValueError(f"the share's experts [{expert_offset}, {expert_offset + local}) lie outside "
                         f"[0, {num_experts})")
    if route_sum not in ("float32", "bfloat16") or activations not in ("bfloat16", "float8_e4m3fn"):
        raise ValueError("route_sum must be float32 or bfloat16; activations bfloat16 or float8_e4m3fn")
    _lib.require_device(hidden, route_indices, route_weights, gate_bits, gate_scale, up_bits, up_scale,
                        down_bits, down_scale, out)
    if out is None:
        out = torch.empty((tokens, h), dtype=torch.float32, device=hidden.device)
    elif tuple(out.shape) != (tokens, h) or out.dtype != torch.float32:
        raise ValueError("out must be float32 [tokens, hidden]")
    valid = torch.empty((), dtype=torch.bool, device=hidden.device)
    ws = routed_workspace(tokens, top_k, local, h, inter, hidden.device)
    flags = ((_lib.ROUTE_SUM_BF16 if route_sum == "bfloat16" else 0) | (_lib.CHECK_WEIGHTS if check_weights else 0)
             | (_lib.DROP_UNOWNED if drop_unowned else 0)
             | (_lib.FP8_ACTIVATIONS if activations == "float8_e4m3fn" else 0))
    _lib.call("glm_moe_routed_experts_share", _lib.ptr(hidden), tokens, h, _lib.ptr(route_indices),
              _lib.ptr(route_weights), top_k, num_experts, expert_offset, local, inter, _lib.ptr(gate_bits),
              _lib.ptr(gate_scale), _lib.ptr(up_bits), _lib.ptr(up_scale), _lib.ptr(down_bits),
              _lib.ptr(down_scale), flags, _lib.ptr(out), _lib.ptr(valid), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(hidden))
    return out, valid


def moe_layer_epilogue(routed: torch.Tensor, shared: torch.Tensor, valid: torch.Tensor, *,
                       routed_scale: float = 2.5) -> torch.Tensor:
    """``bf16(bf16(bf16(routed) * bf16(routed_scale)) + shared)`` of the FP32 routed
    sum over the expert axis (``routed_experts.py:113-127`` / ``:294-304``); a
    non-finite output clears ``valid`` in place (``:126``)."""
    if routed.ndim != 2 or routed.dtype != torch.float32:
        raise ValueError("the routed sum must be float32 [tokens, hidden]")
    if tuple(shared.shape) != tuple(routed.shape) or shared.dtype != torch.bfloat16:
        raise ValueError("shared expert rows must be bf16 [tokens, hidden]")
    if valid.dtype != torch.bool or valid.numel() != 1:
        raise ValueError("valid must be a one-element bool tensor")
    _lib.require_device(routed, shared, valid)
    out = torch.empty(routed.shape, dtype=torch.bfloat16, device=routed.device)
    _lib.call("glm_moe_moe_layer_epilogue", _lib.ptr(routed), routed.shape[0], routed.shape[1], _lib.ptr(shared),
              float(routed_scale), _lib.ptr(out), _lib.ptr(valid), _lib.stream_of(routed))
    return out


def swiglu_bf16(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The expert activation ``(g * sigmoid(g) * u).astype(bf16)`` on bf16 tensors,
    one bf16 rounding per op (``routed_experts.py:102,280``): the device function
    the library's gate/up kernels fuse into their epilogues."""
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16 or gate.shape != up.shape:
        raise ValueError("swiglu_bf16 takes two bf16 tensors of one shape")
    _lib.require_device(gate, up)
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    _lib.call("glm_moe_swiglu_bf16", _lib.ptr(gate), _lib.ptr(up), gate.numel(), _lib.ptr(out), _lib.stream_of(gate))
    return out


def uses_decode_kernels(tokens: int, top_k: int, hidden: int, intermediate: int) -> bool:
    """Whether a layer of this geometry runs on the two decode kernels (where the
    shared expert can run inside them)."""
    return bool(_lib.lib().glm_moe_uses_decode_kernels(tokens, top_k, hidden, intermediate))


def _shared_swiglu(hidden: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """The bf16-resident shared expert at the reference's rounding points.

    FP32-accumulated gate/up rounded to bf16 (``routed_experts.py:119-122`` /
    ``:269-279``) on hipBLASLt, bf16 SwiGLU one op at a time (``:123`` / ``:280``)
    in the library's one-pass kernel (the routed epilogues' device function), bf16
    down projection with FP32 accumulation and one rounding (``:124`` /
    ``:297-302``) on hipBLASLt.
    """
    g = hidden @ gate.t()
    u = hidden @ up.t()
    return swiglu_bf16(g, u) @ down.t()


SHARED_ROWS_MAX = 8  # rows the few-row shared-expert kernels take (glm_moe_shared_expert_rows)
RESIDENT_ROWS_MAX = 8  # rows whose layer runs the shared expert inside the decode kernels


def shared_expert_rows_fit(tokens: int, hidden: int, intermediate: int) -> bool:
    """Whether glm_moe_shared_expert_rows takes this geometry (1..8 rows, sizes
    multiples of 128 and at most 8192)."""
    return (1 <= tokens <= SHARED_ROWS_MAX and hidden % 128 == 0 and intermediate % 128 == 0
            and 0 < hidden <= 8192 and 0 < intermediate <= 8192)


def shared_expert_rows(hidden: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
                       down: torch.Tensor) -> torch.Tensor:
    """The bf16 shared expert of a few rows on the library's kernels: ``bf16 [T, H]``.

    Same rounding points as ``_shared_swiglu`` (``routed_experts.py:119-124`` /
    ``:269-302``), with every weight byte read once for all ``T <= 8`` rows in
    two launches instead of three GEMMs and the elementwise SwiGLU.
    """
    tokens, h = hidden.shape
    inter = gate.shape[0]
    if not shared_expert_rows_fit(tokens, h, inter):
        raise ValueError("the few-row shared expert takes 1..8 rows and sizes that are multiples of 128, <= 8192")
    if (tuple(gate.shape) != (inter, h) or tuple(up.shape) != (inter, h) or tuple(down.shape) != (h, inter)
            or any(t.dtype != torch.bfloat16 for t in (hidden, gate, up, down))):
        raise ValueError("shared expert tables must be bf16 [I, H], [I, H], [H, I] for bf16 [T, H] rows")
    x, g, u, d = (t.contiguous() for t in (hidden, gate, up, down))
    _lib.require_device(x, g, u, d)
    out = torch.empty((tokens, h), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(int(_lib.lib().glm_moe_shared_expert_rows_workspace_bytes(tokens, inter)),
                     dtype=torch.uint8, device=x.device)
    _lib.call("glm_moe_shared_expert_rows", _lib.ptr(x), tokens, h, _lib.ptr(g), _lib.ptr(u), _lib.ptr(d), inter,
              _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return out


def _shared_expert(hidden: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """The shared expert's bf16 output rows: the few-row kernels for up to 8
    rows, torch GEMMs on hipBLASLt (which read the weights once per call) above."""
    if shared_expert_rows_fit(hidden.shape[0], hidden.shape[1], gate.shape[0]):
        return shared_expert_rows(hidden, gate, up, down)
    return _shared_swiglu(hidden, gate, up, down)


def _check_layer_shapes(hidden_local, route_indices, route_weights, gate_bits, up_bits, down_bits,
                        contract: GlmMoeNumericalContract, *, rows_exact: int | None) -> None:
    if hidden_local.ndim != 2 or hidden_local.shape[0] <= 0 or hidden_local.dtype != torch.bfloat16:
        raise ValueError("MoE requires BF16 live rows")
    if rows_exact is not None and hidden_local.shape[0] != rows_exact:
        raise ValueError("grouped MoE input must contain one live row")
    if hidden_local.shape[1] != contract.hidden_size:
        raise ValueError("MoE hidden size differs from contract")
    expected = (hidden_local.shape[0], contract.top_k)
    if tuple(route_indices.shape) != expected or tuple(route_weights.shape) != expected:
        raise ValueError("routing geometry differs from contract")
    if route_indices.dtype != torch.int32:
        raise ValueError("routes must be int32")
    if route_weights.dtype != torch.float32:
        raise ValueError("route weights must be FP32")
    gate_shape = (contract.local_experts, contract.intermediate_size, contract.hidden_size)
    if tuple(gate_bits.shape) != gate_shape or tuple(up_bits.shape) != gate_shape:
        raise ValueError("expert gate/up geometry differs from contract")
    if tuple(down_bits.shape) != (contract.local_experts, contract.hidden_size, contract.intermediate_size):
        raise ValueError("expert down geometry differs from contract")


def _share_of(contract: GlmMoeNumericalContract, expert_rank: int | None, expert_reduce) -> int:
    """The first global expert of this device's share (``axis_index("expert") *
    local_experts``, ``routed_experts.py:85``, ``:250``); 0 on one GPU."""
    if contract.stage_size == 1:
        if expert_rank not in (None, 0) or expert_reduce is not None:
            raise ValueError("a one-GPU contract (stage_size=1) holds every expert: no expert_rank / expert_reduce")
        return 0
    if expert_reduce is None or expert_rank is None:
        raise ValueError("an expert-parallel share (stage_size > 1) needs expert_rank and expert_reduce, the sum "
                         "of the shares' FP32 partials over the expert axis")
    if not 0 <= expert_rank < contract.stage_size:
        raise ValueError("expert_rank must lie in [0, stage_size)")
    return expert_rank * contract.local_experts


def prefill_moe_from_routes(
    hidden_local: torch.Tensor,
    route_indices: torch.Tensor,
    route_weights: torch.Tensor,
    expert_gate_bits_local: torch.Tensor,
    expert_gate_scale_local: torch.Tensor,
    expert_up_bits_local: torch.Tensor,
    expert_up_scale_local: torch.Tensor,
    expert_down_bits_local: torch.Tensor,
    expert_down_scale_local: torch.Tensor,
    shared_gate_local: torch.Tensor,
    shared_up_local: torch.Tensor,
    shared_down_local: torch.Tensor,
    *,
    contract: GlmMoeNumericalContract = single_gpu_contract(),
    interpret: bool = False,
    expert_rank: int | None = None,
    expert_reduce: Callable[[torch.Tensor], torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return (hidden ``[T, H]`` bf16, health) of one prefill MoE layer.

    ``routed_experts.py:27-128``.  A false health bit forbids serving; it must
    not be discarded by a caller.

    With ``contract.stage_size > 1`` the tables are this device's expert share,
    ``expert_rank`` its position on the expert axis, and ``expert_reduce`` the
    sum over that axis of the shares' FP32 ``[T, H]`` partials (the reference's
    ``lax.psum(..., "expert")``, ``:113-117``; e.g. an all-reduce): only the
    share's own routes are computed, and the shared expert and the epilogue
    follow the sum.
    """
    del interpret
    _check_layer_shapes(hidden_local, route_indices, route_weights, expert_gate_bits_local,
                        expert_up_bits_local, expert_down_bits_local, contract, rows_exact=None)
    offset = _share_of(contract, expert_rank, expert_reduce)
    if contract.fp8_block_shape != (128, 128):
        raise ValueError("expert panels require checkpoint scale blocks128x128")
    inter, h = contract.intermediate_size, contract.hidden_size
    if (
        tuple(shared_gate_local.shape) != (inter, h)
        or tuple(shared_up_local.shape) != (inter, h)
        or tuple(shared_down_local.shape) != (h, inter)
    ):
        raise ValueError("prefill shared expert geometry differs from contract")
    tables = (shared_gate_local, shared_up_local, shared_down_local)
    if contract.stage_size > 1:
        partial, valid = routed_experts_share(
            hidden_local, route_indices, route_weights, expert_gate_bits_local, expert_gate_scale_local,
            expert_up_bits_local, expert_up_scale_local, expert_down_bits_local, expert_down_scale_local,
            num_experts=contract.num_experts, expert_offset=offset, route_sum="float32", check_weights=True)
        routed = expert_reduce(partial)
        out = moe_layer_epilogue(routed, _shared_expert(hidden_local, *tables), valid,
                                 routed_scale=contract.routed_scaling_factor)
        return out, valid
    rows = hidden_local.shape[0]
    if rows <= RESIDENT_ROWS_MAX and uses_decode_kernels(rows, contract.top_k, h, inter):
        # up to 8 rows on the decode kernels: the shared expert runs inside the same
        # two launches (its weights streamed once per group of up to 4 rows for
        # gate/up, once for down)
        shared_kw = {"shared_tables": tuple(t.contiguous() for t in tables)}
    else:
        shared_kw = {"shared": _shared_expert(hidden_local, *tables)}
    return routed_experts(
        hidden_local, route_indices, route_weights, expert_gate_bits_local, expert_gate_scale_local,
        expert_up_bits_local, expert_up_scale_local, expert_down_bits_local, expert_down_scale_local,
        route_sum="float32", check_weights=True, routed_scale=contract.routed_scaling_factor, **shared_kw,
    )


def prefill_moe_from_router_logits(
    hidden_local: torch.Tensor,
    router_logits: torch.Tensor,
    correction_bias: torch.Tensor | None,
    expert_gate_bits_local: torch.Tensor,
    expert_gate_scale_local: torch.Tensor,
    expert_up_bits_local: torch.Tensor,
    expert_up_scale_local: torch.Tensor,
    expert_down_bits_local: torch.Tensor,
    expert_down_scale_local: torch.Tensor,
    shared_gate_local: torch.Tensor,
    shared_up_local: torch.Tensor,
    shared_down_local: torch.Tensor,
    *,
    contract: GlmMoeNumericalContract = single_gpu_contract(),
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The prefill MoE MLP of ``[T, H]`` rows from their router logits:
    ``(output, route_indices, route_weights, valid)``.

    The reference's prefill MLP from the logits on (``decoder_layer.py:123-146``):
    the noaux_tc selection of ``prefill_router`` (``router.py:146``, i.e.
    ``route_glm_noaux_tc_logits``) feeding ``prefill_moe_from_routes``, in one
    library call (``glm_moe_moe_layer_from_router_logits``; one row: the decode
    kernels with the resident shared expert, routing inside the gate/up
    kernel).  ``valid`` is per row, as the
    reference's ``router_valid & grouped_valid``: the layer's health and, per
    row, finite logits, bias and route weights (``router.py:161-166``; the
    hidden rows' own finiteness check belongs to the router's matmul, before
    these logits).  One device (``stage_size == 1``): an expert-parallel share
    routes first and calls ``prefill_moe_from_routes``.
    """
    if contract.stage_size != 1:
        raise ValueError("routing inside the layer takes a one-GPU contract; for an expert-parallel share route "
                         "with route_glm_noaux_tc_logits and call prefill_moe_from_routes")
    if router_logits.ndim != 2 or tuple(router_logits.shape) != (hidden_local.shape[0], contract.num_experts):
        raise ValueError(f"router_logits must have shape {(hidden_local.shape[0], contract.num_experts)}")
    top_k = contract.top_k
    inter, h = contract.intermediate_size, contract.hidden_size
    ids_probe = torch.zeros((hidden_local.shape[0], top_k), dtype=torch.int32, device=hidden_local.device)
    _check_layer_shapes(hidden_local, ids_probe, ids_probe.float(), expert_gate_bits_local, expert_up_bits_local,
                        expert_down_bits_local, contract, rows_exact=None)
    if contract.fp8_block_shape != (128, 128):
        raise ValueError("expert panels require checkpoint scale blocks128x128")
    tables = (shared_gate_local, shared_up_local, shared_down_local)
    if (tuple(tables[0].shape) != (inter, h) or tuple(tables[1].shape) != (inter, h)
            or tuple(tables[2].shape) != (h, inter)):
        raise ValueError("prefill shared expert geometry differs from contract")
    bias = (torch.zeros(contract.num_experts, dtype=torch.float32, device=hidden_local.device)
            if correction_bias is None else correction_bias)
    if hidden_local.shape[0] == 1 and contract.num_experts <= 256 and uses_decode_kernels(1, top_k, h, inter):
        # one row: the resident shared expert inside the two decode kernels, which also route
        experts = contract.num_experts
        resident = tuple(t.contiguous() for t in tables)
        logits = router_logits.float().contiguous()
        bias = bias.float().contiguous()
        _lib.require_device(hidden_local, logits, bias, expert_gate_bits_local, expert_gate_scale_local,
                            expert_up_bits_local, expert_up_scale_local, expert_down_bits_local,
                            expert_down_scale_local, *resident)
        out = torch.empty((1, h), dtype=torch.bfloat16, device=hidden_local.device)
        layer_valid = torch.empty((), dtype=torch.bool, device=hidden_local.device)
        ids = torch.empty((1, top_k), dtype=torch.int32, device=hidden_local.device)
        weights = torch.empty((1, top_k), dtype=torch.float32, device=hidden_local.device)
        ws = routed_workspace(1, top_k, experts, h, inter, hidden_local.device)
        _lib.call(
            "glm_moe_moe_layer_from_logits", _lib.ptr(hidden_local.contiguous()), 1, h, _lib.ptr(logits),
            _lib.ptr(bias), top_k, experts, inter, _lib.ptr(expert_gate_bits_local),
            _lib.ptr(expert_gate_scale_local), _lib.ptr(expert_up_bits_local), _lib.ptr(expert_up_scale_local),
            _lib.ptr(expert_down_bits_local), _lib.ptr(expert_down_scale_local), _lib.CHECK_WEIGHTS,
            *(_lib.ptr(t) for t in resident), inter, float(contract.routed_scaling_factor), _lib.ptr(ids),
            _lib.ptr(weights), _lib.ptr(out), _lib.ptr(layer_valid), _lib.ptr(ws), ws.numel(),
            _lib.stream_of(hidden_local))
    else:
        out, layer_valid, ids, weights = routed_experts_from_router_logits(
            hidden_local, router_logits, bias, expert_gate_bits_local, expert_gate_scale_local,
            expert_up_bits_local, expert_up_scale_local, expert_down_bits_local, expert_down_scale_local,
            top_k=top_k, route_sum="float32", check_weights=True, shared=_shared_expert(hidden_local, *tables),
            routed_scale=contract.routed_scaling_factor)
    row_valid = (torch.isfinite(router_logits).all(dim=1) & torch.isfinite(bias).all()
                 & torch.isfinite(weights).all(dim=1))
    return out, ids, weights, row_valid & layer_valid


def moe_grouped_routes(
    hidden_local: torch.Tensor,
    route_indices: torch.Tensor,
    route_weights: torch.Tensor,
    expert_gate_bits_local: torch.Tensor,
    expert_gate_scale_local: torch.Tensor,
    expert_up_bits_local: torch.Tensor,
    expert_up_scale_local: torch.Tensor,
    expert_down_bits_local: torch.Tensor,
    expert_down_scale_local: torch.Tensor,
    *,
    contract: GlmMoeNumericalContract = single_gpu_contract(),
    config: RoutedProjectionConfig = RoutedProjectionConfig(),
    expert_axis: str = "expert",
    feature_axis: str = "feature",
    interpret: bool = False,
    shared_bf16: tuple[Any, Any, Any],
    expert_rank: int | None = None,
    expert_reduce: Callable[[torch.Tensor], torch.Tensor] | None = None,
) -> torch.Tensor:
    """The decode MoE of one row with route-grouped routed experts (``routed_experts.py:186-304``).

    Routes whose expert this device does not hold contribute zero (``:250-253``);
    the weighted routes of the share are summed in bf16 (``:293``).  With
    ``contract.stage_size > 1`` the tables are the share of ``expert_rank`` and
    ``expert_reduce`` sums the shares' partials over the expert axis (``:294-295``),
    as for ``prefill_moe_from_routes``.
    """
    del expert_axis, feature_axis, interpret
    _check_layer_shapes(hidden_local, route_indices, route_weights, expert_gate_bits_local,
                        expert_up_bits_local, expert_down_bits_local, contract, rows_exact=1)
    offset = _share_of(contract, expert_rank, expert_reduce)
    if tuple(config.block_shape) != tuple(contract.fp8_block_shape):
        raise ValueError("grouped MoE tile config block differs from the contract")
    inter, h = contract.intermediate_size, contract.hidden_size
    if (
        len(shared_bf16) != 3
        or any(t.dtype != torch.bfloat16 for t in shared_bf16)
        or tuple(shared_bf16[0].shape) != (inter, h)
        or tuple(shared_bf16[1].shape) != (inter, h)
        or tuple(shared_bf16[2].shape) != (h, inter)
    ):
        raise ValueError("grouped MoE BF16 shared tables drifted")
    if contract.stage_size > 1:
        partial, valid = routed_experts_share(
            hidden_local, route_indices, route_weights, expert_gate_bits_local, expert_gate_scale_local,
            expert_up_bits_local, expert_up_scale_local, expert_down_bits_local, expert_down_scale_local,
            num_experts=contract.num_experts, expert_offset=offset, route_sum="bfloat16", check_weights=False,
            drop_unowned=True)
        routed = expert_reduce(partial)
        return moe_layer_epilogue(routed, _shared_expert(hidden_local, *shared_bf16), valid,
                                  routed_scale=contract.routed_scaling_factor)
    if uses_decode_kernels(1, contract.top_k, h, inter):
        shared_kw = {"shared_tables": tuple(t.contiguous() for t in shared_bf16)}
    else:
        shared_kw = {"shared": _shared_expert(hidden_local, *shared_bf16)}
    output, _ = routed_experts(
        hidden_local, route_indices, route_weights, expert_gate_bits_local, expert_gate_scale_local,
        expert_up_bits_local, expert_up_scale_local, expert_down_bits_local, expert_down_scale_local,
        route_sum="bfloat16", check_weights=False, drop_unowned=True,
        routed_scale=contract.routed_scaling_factor, **shared_kw,
    )
    return output


def moe_mlp_from_router_logits(
    hidden_local: torch.Tensor,
    router_logits: torch.Tensor,
    correction_bias: torch.Tensor | None,
    expert_gate_bits_local: torch.Tensor,
    expert_gate_scale_local: torch.Tensor,
    expert_up_bits_local: torch.Tensor,
    expert_up_scale_local: torch.Tensor,
    expert_down_bits_local: torch.Tensor,
    expert_down_scale_local: torch.Tensor,
    *,
    contract: GlmMoeNumericalContract = single_gpu_contract(),
    shared_bf16: tuple[Any, Any, Any],
    expert_rank: int | None = None,
    expert_reduce: Callable[[torch.Tensor], torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The decode MoE MLP body of one row from its router logits:
    ``(update, route_indices, route_weights)``.

    The reference's decode MLP (``glm_tpu/models/glm_moe_dsa/decoder_layer.py:636-656``)
    routes the row (``route_glm_noaux_tc_logits``, ``router.py:20-55``, the last
    step of ``router_from_shards``) and runs ``moe_grouped_routes`` on the
    selection, returning both.  Here, on the shapes the decode kernels take
    (``uses_decode_kernels``, at most 256 experts), the gate/up kernel routes its
    token itself (``glm_moe_moe_layer_from_logits``: one launch fewer, ids and
    weights bit-equal to the router kernel's); otherwise the router kernel runs
    first, then ``moe_grouped_routes``.
    """
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    experts, top_k = contract.num_experts, contract.top_k  # the router scores every expert
    if router_logits.ndim != 2 or tuple(router_logits.shape) != (hidden_local.shape[0], experts):
        raise ValueError(f"router_logits must have shape {(hidden_local.shape[0], experts)}")
    if correction_bias is not None and tuple(correction_bias.shape) != (experts,):
        raise ValueError(f"correction_bias must have shape {(experts,)}")
    inter, h = contract.intermediate_size, contract.hidden_size
    fused = (
        contract.stage_size == 1 and hidden_local.ndim == 2 and hidden_local.shape[0] == 1 and experts <= 256
        and uses_decode_kernels(1, top_k, h, inter)
    )
    if not fused:
        bias = correction_bias if correction_bias is not None else torch.zeros(
            experts, dtype=torch.float32, device=router_logits.device)
        ids, weights = route_glm_noaux_tc_logits(router_logits, bias, top_k=top_k)
        update = moe_grouped_routes(
            hidden_local, ids, weights, expert_gate_bits_local, expert_gate_scale_local, expert_up_bits_local,
            expert_up_scale_local, expert_down_bits_local, expert_down_scale_local, contract=contract,
            shared_bf16=shared_bf16, expert_rank=expert_rank, expert_reduce=expert_reduce)
        return update, ids, weights
    ids = torch.empty((1, top_k), dtype=torch.int32, device=hidden_local.device)
    weights = torch.empty((1, top_k), dtype=torch.float32, device=hidden_local.device)
    _check_layer_shapes(hidden_local, ids, weights, expert_gate_bits_local, expert_up_bits_local,
                        expert_down_bits_local, contract, rows_exact=1)
    if (
        len(shared_bf16) != 3
        or any(t.dtype != torch.bfloat16 for t in shared_bf16)
        or tuple(shared_bf16[0].shape) != (inter, h)
        or tuple(shared_bf16[1].shape) != (inter, h)
        or tuple(shared_bf16[2].shape) != (h, inter)
    ):
        raise ValueError("grouped MoE BF16 shared tables drifted")
    for scale, rows, cols in ((expert_gate_scale_local, inter, h), (expert_up_scale_local, inter, h),
                              (expert_down_scale_local, h, inter)):
        if scale.dtype != torch.float32 or tuple(scale.shape) != (experts, rows // 128, cols // 128):
            raise ValueError("expert scales must be float32 [E, N/128, K/128]")
    tables = tuple(t.contiguous() for t in shared_bf16)
    logits = router_logits.float().contiguous()
    bias = None if correction_bias is None else correction_bias.float().contiguous()
    _lib.require_device(hidden_local, logits, bias, expert_gate_bits_local, expert_gate_scale_local,
                        expert_up_bits_local, expert_up_scale_local, expert_down_bits_local,
                        expert_down_scale_local, *tables)
    out = torch.empty((1, h), dtype=torch.bfloat16, device=hidden_local.device)
    valid = torch.empty((), dtype=torch.bool, device=hidden_local.device)
    ws = routed_workspace(1, top_k, experts, h, inter, hidden_local.device)
    flags = _lib.ROUTE_SUM_BF16 | _lib.DROP_UNOWNED  # moe_grouped_routes' body (routed_experts.py:250-253, :293)
    _lib.call(
        "glm_moe_moe_layer_from_logits", _lib.ptr(hidden_local.contiguous()), 1, h, _lib.ptr(logits),
        _lib.ptr(bias), top_k, experts, inter, _lib.ptr(expert_gate_bits_local), _lib.ptr(expert_gate_scale_local),
        _lib.ptr(expert_up_bits_local), _lib.ptr(expert_up_scale_local), _lib.ptr(expert_down_bits_local),
        _lib.ptr(expert_down_scale_local), flags, *(_lib.ptr(t) for t in tables), inter,
        float(contract.routed_scaling_factor), _lib.ptr(ids), _lib.ptr(weights), _lib.ptr(out), _lib.ptr(valid),
        _lib.ptr(ws), ws.numel(), _lib.stream_of(hidden_local),
    )
    return out, ids, weights
