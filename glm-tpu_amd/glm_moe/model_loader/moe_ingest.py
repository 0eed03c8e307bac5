"""One MoE layer's tables from safetensors checkpoint files onto the GPU.

The reference loads routed experts into final-owner tensors named
``model.layers.L.mlp.experts.{gate,up,down}_proj.{weight_bits,scale_inv}`` with
a leading expert axis (``glm_tpu/models/glm_moe_dsa/weights.py:334-335,
393-398``), from per-expert source tensors
``model.layers.L.mlp.experts.e.{proj}.{weight,weight_scale_inv}``
(``glm_tpu/model_loader/placement.py:24-27``), and refuses FP8 payloads holding
NaN encodings and non-finite FP32 payloads (``sharded_state/format.py:307-324``).

Here the stacked tables are exactly what the kernels read: uint8 e4m3fn
``[E, N, K]`` (N = output rows, K contiguous) and FP32 block scales
``[E, N/128, K/128]``, so ingest is a copy per expert and no repacking.  The
finite-bit gate runs on the GPU over the tables once they are in HBM
(``glm_moe_count_nonfinite_fp8``).  The shared expert is dequantised to the
bf16 resident tables the layer bodies take, with the library's decode
(``glm_tpu/layers/fp8.py:37-72``).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Iterable

import numpy as np
import torch

from glm_moe import _lib
from glm_moe.model_loader.placement import (
    PROJECTIONS,
    expert_coordinate,
    router_source_names,
    routed_source,
    shared_source_names,
    source_names,
)
from glm_moe.model_loader.safetensors_io import SafetensorsFile, TensorInfo


class CheckpointValidationError(ValueError):
    """A checkpoint that must not be served (the reference's ``glm_tpu.exceptions``)."""


@dataclass
class MoeLayerTables:
    """One layer's expert tables on the GPU, for ``num_local`` experts starting
    at global id ``first_expert`` (all of them when ``ep_size == 1``)."""

    layer: int
    num_experts: int
    first_expert: int
    gate_bits: torch.Tensor
    gate_scale: torch.Tensor
    up_bits: torch.Tensor
    up_scale: torch.Tensor
    down_bits: torch.Tensor
    down_scale: torch.Tensor
    shared_gate: torch.Tensor | None = None  # bf16 [I_shared, H]
    shared_up: torch.Tensor | None = None
    shared_down: torch.Tensor | None = None  # bf16 [H, I_shared]
    router_weight: torch.Tensor | None = None  # [E, H] as stored
    correction_bias: torch.Tensor | None = None  # FP32 [E]

    @property
    def num_local(self) -> int:
        return int(self.gate_bits.shape[0])

    def expert_tables(self) -> tuple[torch.Tensor, ...]:
        """The six tables in the order the routed-expert entry points take them."""
        return (self.gate_bits, self.gate_scale, self.up_bits, self.up_scale, self.down_bits, self.down_scale)

    def local_route_indices(self, route_indices: torch.Tensor) -> torch.Tensor:
        """Global expert ids -> this share's local ids; ids of other shares fall
        outside ``[0, num_local)`` and are dropped by ``drop_unowned`` (the
        reference's owned mask, ``routed_experts.py:250-253``)."""
        return route_indices - self.first_expert


def _index(paths: Iterable[str | Path]) -> dict[str, SafetensorsFile]:
    where: dict[str, SafetensorsFile] = {}
    for path in paths:
        f = SafetensorsFile(path)
        for name in f.tensors:
            if name in where:
                raise CheckpointValidationError(f"tensor {name!r} appears in more than one file")
            where[name] = f
    return where


def _info(where: dict[str, SafetensorsFile], name: str, dtype: str, shape: tuple[int, ...]) -> TensorInfo:
    if name not in where:
        raise CheckpointValidationError(f"checkpoint lacks {name!r}")
    info = where[name].info(name)
    if info.dtype != dtype:
        raise CheckpointValidationError(f"{name!r} is {info.dtype}, expected {dtype}")
    if info.shape != shape:
        raise CheckpointValidationError(f"{name!r} has shape {info.shape}, expected {shape}")
    return info


class _Uploader:
    """Host bytes -> device through one reusable pinned staging buffer."""

    def __init__(self, device: torch.device):
        self.device = device
        self.stage: torch.Tensor | None = None

    def copy(self, src: np.ndarray, dst: torch.Tensor) -> None:
        raw = np.ascontiguousarray(src).reshape(-1).view(np.uint8)
        if self.stage is None or self.stage.numel() < raw.size:
            self.stage = torch.empty(max(raw.size, 1 << 20), dtype=torch.uint8, pin_memory=True)
        host = self.stage[: raw.size]
        host.numpy()[:] = raw
        dst.view(-1).view(torch.uint8).copy_(host, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()  # the staging buffer is reused next


def validate_finite_fp8(bits: torch.Tensor, what: str) -> None:
    """The finite-bit gate of FP8 payloads (``format.py:307-315``), on the GPU."""
    count = torch.zeros(1, dtype=torch.int64, device=bits.device)
    _lib.call("glm_moe_count_nonfinite_fp8", _lib.ptr(bits), bits.numel(), _lib.ptr(count), _lib.stream_of(bits))
    bad = int(count.item())
    if bad:
        raise CheckpointValidationError(f"FP8 payload contains non-finite bits ({what}: {bad} bytes)")


def _validate_finite(t: torch.Tensor, what: str) -> None:
    if not bool(torch.isfinite(t.float()).all()):
        raise CheckpointValidationError(f"checkpoint {what} payload is non-finite")


def load_moe_layer(
    paths: Iterable[str | Path],
    layer: int,
    *,
    device: torch.device | str,
    num_experts: int,
    hidden_size: int,
    intermediate_size: int,
    ep_rank: int = 0,
    ep_size: int = 1,
    shared: bool = True,
    router: bool = True,
) -> MoeLayerTables:
    """Stack one layer's routed experts (this rank's share), and optionally its
    shared expert (as bf16) and router, from safetensors files onto ``device``."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("the tables are loaded onto a GPU (there is no CPU path)")
    if not 0 <= ep_rank < ep_size:
        raise ValueError("ep_rank must lie in [0, ep_size)")
    expert_coordinate(0, num_experts, ep_size)  # E must divide over the ranks
    local = num_experts // ep_size
    first = ep_rank * local
    where = _index(paths)
    extra = sorted({r.expert for n in where if (r := routed_source(n)) and r.layer == layer and r.expert >= num_experts})
    if extra:
        raise CheckpointValidationError(f"layer {layer} holds experts beyond {num_experts}: {extra[:4]}")
    h, inter = hidden_size, intermediate_size
    geometry = {"gate_proj": (inter, h), "up_proj": (inter, h), "down_proj": (h, inter)}
    up = _Uploader(device)
    tables: dict[str, torch.Tensor] = {}
    for proj in PROJECTIONS:
        n, k = geometry[proj]
        sshape = (-(-n // 128), -(-k // 128))
        bits = torch.empty((local, n, k), dtype=torch.uint8, device=device)
        scale = torch.empty((local, *sshape), dtype=torch.float32, device=device)
        for e in range(local):
            wname, sname = source_names(layer, first + e, proj)
            winfo = _info(where, wname, "F8_E4M3", (n, k))
            sinfo = _info(where, sname, "F32", sshape)
            up.copy(where[wname].raw(winfo.name), bits[e])
            up.copy(where[sname].raw(sinfo.name), scale[e])
        short = proj.split("_")[0]
        validate_finite_fp8(bits, f"layer {layer} experts {short}_proj")
        _validate_finite(scale, f"F32 (layer {layer} experts {short}_proj scale_inv)")
        tables[f"{short}_bits"] = bits
        tables[f"{short}_scale"] = scale
    out = MoeLayerTables(layer=layer, num_experts=num_experts, first_expert=first, **tables)
    if shared:
        from glm_moe.layers.fp8 import dequantize_fp8_bits_block_weight

        sh = {}
        for proj in PROJECTIONS:
            wname, sname = shared_source_names(layer, proj)
            if wname not in where:
                raise CheckpointValidationError(f"checkpoint lacks {wname!r}")
            winfo = where[wname].info(wname)
            if winfo.dtype != "F8_E4M3" or len(winfo.shape) != 2:
                raise CheckpointValidationError(f"{wname!r} must be a 2-D F8_E4M3 tensor")
            n, k = winfo.shape
            if (proj == "down_proj" and n != h) or (proj != "down_proj" and k != h):
                raise CheckpointValidationError(f"{wname!r} has shape {winfo.shape}, not against hidden size {h}")
            sinfo = _info(where, sname, "F32", (-(-n // 128), -(-k // 128)))
            bits = torch.empty((n, k), dtype=torch.uint8, device=device)
            scale = torch.empty(sinfo.shape, dtype=torch.float32, device=device)
            up.copy(where[wname].raw(wname), bits)
            up.copy(where[sname].raw(sname), scale)
            validate_finite_fp8(bits, f"layer {layer} shared {proj}")
            _validate_finite(scale, f"F32 (layer {layer} shared {proj} scale_inv)")
            sh[proj] = dequantize_fp8_bits_block_weight(bits, scale)
        out.shared_gate, out.shared_up, out.shared_down = sh["gate_proj"], sh["up_proj"], sh["down_proj"]
    if router:
        wname, bname = router_source_names(layer)
        if wname not in where:
            raise CheckpointValidationError(f"checkpoint lacks {wname!r}")
        winfo = where[wname].info(wname)
        if winfo.dtype not in ("BF16", "F32") or winfo.shape != (num_experts, h):
            raise CheckpointValidationError(f"{wname!r} must be BF16/F32 [{num_experts}, {h}]")
        binfo = _info(where, bname, "F32", (num_experts,))
        wdtype = torch.bfloat16 if winfo.dtype == "BF16" else torch.float32
        out.router_weight = torch.empty(winfo.shape, dtype=wdtype, device=device)
        out.correction_bias = torch.empty(binfo.shape, dtype=torch.float32, device=device)
        up.copy(where[wname].raw(wname), out.router_weight)
        up.copy(where[bname].raw(bname), out.correction_bias)
        _validate_finite(out.router_weight, f"{winfo.dtype} (layer {layer} router)")
        _validate_finite(out.correction_bias, f"F32 (layer {layer} correction bias)")
    return out
