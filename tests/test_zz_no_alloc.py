"""The allocation-free decode layer, glm_moe_moe_layer_resident_noalloc, through
the C ABI: its output and health must equal glm_moe_moe_layer_resident's (same
kernels, caller workspace) bit for bit, on calls in a row whose last is
smaller -- the static scratch keeps the previous call's contents, which the
next must not depend on -- including the shape that fills the scratch exactly,
and replayed from a HIP graph."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from glm_moe import _lib
from glm_moe import synthetic as S

pytestmark = pytest.mark.gpu

TABLE_KEYS = ("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale")


def _case(tokens, experts, hidden, inter, top_k, seed, device):
    cfg = S.MoeConfig("noalloc", tokens, experts, hidden, inter, top_k)
    x = torch.from_numpy(S.hidden_states(cfg, seed)).to(torch.bfloat16).to(device)
    ids, w = S.routes(cfg, seed)
    tables = S.device_expert_tables(cfg, seed, device)
    g = torch.Generator(device=device).manual_seed(seed)
    shared = tuple((torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)
                   for shape, std in (((inter, hidden), hidden ** -0.5), ((inter, hidden), hidden ** -0.5),
                                      ((hidden, inter), 2 * inter ** -0.5)))
    return x, torch.from_numpy(ids).to(device), torch.from_numpy(w).to(device), tables, shared


def _launch(case, flags, out, valid, workspace=None):
    x, ids, w, tables, shared = case
    tokens, hidden = x.shape
    top_k = ids.shape[1]
    experts, inter, _ = tables["gate_bits"].shape
    args = [_lib.ptr(x), tokens, hidden, _lib.ptr(ids), _lib.ptr(w), top_k, experts, inter,
            *(_lib.ptr(tables[k]) for k in TABLE_KEYS), flags, *(_lib.ptr(t) for t in shared), inter, 2.5,
            _lib.ptr(out), _lib.ptr(valid)]
    if workspace is None:
        _lib.call("glm_moe_moe_layer_resident_noalloc", *args, _lib.stream_of(x))
    else:
        _lib.call("glm_moe_moe_layer_resident", *args, _lib.ptr(workspace), workspace.numel(), _lib.stream_of(x))


def _outputs(case):
    x = case[0]
    out = torch.full(tuple(x.shape), float("nan"), dtype=torch.bfloat16, device=x.device)
    return out, torch.zeros((), dtype=torch.bool, device=x.device)


def _run(case, flags, workspace=None):
    out, valid = _outputs(case)
    _launch(case, flags, out, valid, workspace)
    torch.cuda.synchronize()
    return out, valid


def _workspace(case):
    x, ids, _, tables, _ = case
    experts, inter, hidden = tables["gate_bits"].shape
    nbytes = int(_lib.lib().glm_moe_routed_experts_workspace_bytes(x.shape[0], ids.shape[1], experts, hidden, inter))
    return torch.empty(nbytes, dtype=torch.uint8, device=x.device)


def _bits(t):
    return t.cpu().view(torch.int16).numpy()


def test_noalloc_layer_equals_the_workspace_layer():
    device = torch.device("cuda:0")
    flags = _lib.ROUTE_SUM_BF16 | _lib.DROP_UNOWNED
    # 64 routes x I = 2048 (288 KiB of the scratch), then the shape that fills it
    # to the last byte (64 tokens of one route: 64 x 2048 routed + 64 x 2048
    # shared bf16 activations = 512 KiB), then a smaller call
    for tokens, experts, hidden, inter, top_k, seed in ((8, 32, 768, 2048, 8, 1), (64, 32, 768, 2048, 1, 4),
                                                        (1, 16, 512, 256, 4, 2)):
        case = _case(tokens, experts, hidden, inter, top_k, seed, device)
        want, want_ok = _run(case, flags, _workspace(case))
        got, ok = _run(case, flags)
        assert bool(want_ok) and bool(ok)
        assert torch.isfinite(got.float()).all()
        np.testing.assert_array_equal(_bits(got), _bits(want))
        again, _ = _run(case, 0)  # prefill-body flags on the same inputs: same kernels, same result here
        np.testing.assert_array_equal(_bits(again), _bits(want))


def test_noalloc_layer_replays_in_a_graph():
    """Captured in a HIP graph (the callers it is for), replays equal the
    workspace layer's eager result, replay after replay, with eager calls on
    other inputs -- which overwrite the shared static scratch -- between them."""
    device = torch.device("cuda:0")
    flags = _lib.ROUTE_SUM_BF16 | _lib.DROP_UNOWNED
    case = _case(4, 32, 768, 2048, 8, 5, device)
    other_case = _case(4, 32, 768, 2048, 8, 6, device)
    want, want_ok = _run(case, flags, _workspace(case))
    other, _ = _run(other_case, flags, _workspace(other_case))
    assert bool(want_ok) and not torch.equal(want, other)
    out, valid = _outputs(case)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch(case, flags, out, valid)
    for replay in range(3):
        again, _ = _run(other_case, flags)  # eager call: the scratch now holds other inputs' rows
        np.testing.assert_array_equal(_bits(again), _bits(other))
        out.fill_(float("nan"))
        valid.zero_()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(out), _bits(want), err_msg=f"replay {replay}")
        assert bool(valid)


def test_noalloc_layer_refuses_shapes_beyond_its_scratch():
    device = torch.device("cuda:0")
    x, ids, w, tables, shared = _case(9, 16, 512, 256, 8, 3, device)  # 72 routes: not a decode shape
    out = torch.empty((9, 512), dtype=torch.bfloat16, device=device)
    valid = torch.empty((), dtype=torch.bool, device=device)
    with pytest.raises(ValueError, match="allocation-free"):
        _lib.call("glm_moe_moe_layer_resident_noalloc", _lib.ptr(x), 9, 512, _lib.ptr(ids), _lib.ptr(w), 8, 16, 256,
                  *(_lib.ptr(tables[k]) for k in TABLE_KEYS), 0, *(_lib.ptr(t) for t in shared), 256, 2.5,
                  _lib.ptr(out), _lib.ptr(valid), _lib.stream_of(x))
