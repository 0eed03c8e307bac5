"""Seeded synthetic inputs of the benchmark / parity configurations.

The five configurations of the benchmark (toy, decode T=1, batched decode
T=4, prefill T=2048 uniform, prefill T=8192 Zipf s=1.2):

* activations bf16 ~ N(0, 1);
* router logits ~ N(0, 1) (plus ``log(zipf weight)`` for the Zipf config),
  routed with GLM ``noaux_tc`` semantics (sigmoid scores, top-k of the scores
  with ties to the lowest id, FP32 renormalised weights; reference
  ``glm_tpu/layers/moe/router.py:20-55``) with zero correction bias;
* expert weights N(0, 0.02) per 128x128 block quantised to e4m3fn with an FP32
  scale ``amax / 448`` -- on the host with numpy + torch's e4m3fn cast for the
  small configs, on the GPU with ``glm_moe_synthesize_fp8_weights`` for the
  production shapes (9.7 GB per layer).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from glm_moe import _lib


@dataclass(frozen=True)
class MoeConfig:
    name: str
    tokens: int
    experts: int
    hidden: int
    intermediate: int
    top_k: int
    zipf: float = 0.0  # Zipf exponent added to the router logits (0: uniform)

    @property
    def routes(self) -> int:
        return self.tokens * self.top_k


CONFIGS: dict[str, MoeConfig] = {
    "toy": MoeConfig("toy", 4, 8, 256, 256, 2),
    "decode_t1": MoeConfig("decode_t1", 1, 256, 6144, 2048, 8),
    "decode_t4": MoeConfig("decode_t4", 4, 256, 6144, 2048, 8),
    # 64 concurrent chats: 512 routes over ~218 experts, past the decode kernels
    "batch_t64": MoeConfig("batch_t64", 64, 256, 6144, 2048, 8),
    # the reference engine's prefill block (llm_engine.py:56-62): 128 rows, 1,024 routes
    "prefill_t128": MoeConfig("prefill_t128", 128, 256, 6144, 2048, 8),
    "prefill_t2048": MoeConfig("prefill_t2048", 2048, 256, 6144, 2048, 8),
    "prefill_t8192_zipf": MoeConfig("prefill_t8192_zipf", 8192, 256, 6144, 2048, 8, zipf=1.2),
}


def noaux_tc_route(logits: np.ndarray, bias: np.ndarray | None, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """GLM noaux_tc selection on the host (input generation only)."""
    logits = np.asarray(logits, np.float32)
    scores = (np.float32(1.0) / (np.float32(1.0) + np.exp(-logits))).astype(np.float32)
    biased = scores if bias is None else (scores + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    idx = np.argsort(-biased, axis=-1, kind="stable")[:, :top_k].astype(np.int32)
    chosen = np.take_along_axis(scores, idx, axis=-1)
    weights = (chosen / chosen.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return idx, weights


def router_logits(cfg: MoeConfig, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((cfg.tokens, cfg.experts), dtype=np.float32)
    if cfg.zipf:
        ranks = np.arange(1, cfg.experts + 1, dtype=np.float64)
        weights = ranks ** (-cfg.zipf)
        logits = (logits + np.log(weights / weights.sum()).astype(np.float32)[None, :]).astype(np.float32)
    return logits


def routes(cfg: MoeConfig, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """(ids int32 [T, k], weights f32 [T, k]) for one seed."""
    return noaux_tc_route(router_logits(cfg, seed), None, cfg.top_k)


def hidden_states(cfg: MoeConfig, seed: int) -> np.ndarray:
    """bf16-valued FP32 activations ~ N(0, 1), as a float32 numpy array."""
    rng = np.random.default_rng(seed + 1_000_003)
    x = rng.standard_normal((cfg.tokens, cfg.hidden), dtype=np.float32)
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def host_fp8_weights(rng: np.random.Generator, experts: int, n: int, k: int, sigma: float = 0.02):
    """(bits uint8 [E, N, K], scales f32 [E, N/128, K/128]) quantised on the host."""
    w = rng.normal(0.0, sigma, (experts, n, k)).astype(np.float32)
    blocks = w.reshape(experts, n // 128, 128, k // 128, 128)
    amax = np.abs(blocks).max(axis=(2, 4)).astype(np.float32)
    scale = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(blocks / scale[:, :, None, :, None], -448.0, 448.0).astype(np.float32)
    bits = torch.from_numpy(q.reshape(experts, n, k)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return np.ascontiguousarray(bits), scale


def host_expert_tables(cfg: MoeConfig, seed: int):
    """Host gate/up/down tables of a small config: dict of numpy arrays."""
    rng = np.random.default_rng(seed + 2_000_029)
    gb, gs = host_fp8_weights(rng, cfg.experts, cfg.intermediate, cfg.hidden)
    ub, us = host_fp8_weights(rng, cfg.experts, cfg.intermediate, cfg.hidden)
    db, ds = host_fp8_weights(rng, cfg.experts, cfg.hidden, cfg.intermediate)
    return {"gate_bits": gb, "gate_scale": gs, "up_bits": ub, "up_scale": us, "down_bits": db, "down_scale": ds}


def device_fp8_weights(experts: int, n: int, k: int, seed: int, device, sigma: float = 0.02):
    """(bits, scales) generated on the GPU by ``glm_moe_synthesize_fp8_weights``."""
    bits = torch.empty((experts, n, k), dtype=torch.uint8, device=device)
    scales = torch.empty((experts, n // 128, k // 128), dtype=torch.float32, device=device)
    _lib.call("glm_moe_synthesize_fp8_weights", ctypes.c_uint64(seed), experts, n, k, ctypes.c_float(sigma),
              _lib.ptr(bits), _lib.ptr(scales), _lib.stream_of(bits))
    return bits, scales


def device_expert_tables(cfg: MoeConfig, seed: int, device) -> dict[str, torch.Tensor]:
    """GPU gate/up/down tables of a config (the production shapes fit one GPU)."""
    base = (seed & 0xFFFFFFFF) << 8
    gb, gs = device_fp8_weights(cfg.experts, cfg.intermediate, cfg.hidden, base + 1, device)
    ub, us = device_fp8_weights(cfg.experts, cfg.intermediate, cfg.hidden, base + 2, device)
    db, ds = device_fp8_weights(cfg.experts, cfg.hidden, cfg.intermediate, base + 3, device)
    return {"gate_bits": gb, "gate_scale": gs, "up_bits": ub, "up_scale": us, "down_bits": db, "down_scale": ds}


def distinct_experts(ids: np.ndarray, experts: int) -> int:
    flat = np.asarray(ids).reshape(-1)
    flat = flat[(flat >= 0) & (flat < experts)]
    return int(np.unique(flat).size)


def algorithmic_bytes(cfg: MoeConfig, ids: np.ndarray) -> dict[str, int]:
    """HBM bytes the routed path must move at minimum, per stage.

    Per distinct selected expert: its e4m3 gate/up/down bytes and FP32 block
    scales; plus the activations in and the output out, ids and weights.
    """
    d = distinct_experts(ids, cfg.experts)
    h, i, t, k = cfg.hidden, cfg.intermediate, cfg.tokens, cfg.top_k
    scale = lambda n, kk: (n // 128) * (kk // 128) * 4  # noqa: E731
    gate_up = d * 2 * (i * h + scale(i, h)) + t * h * 2 + t * k * i * 2
    down = d * (h * i + scale(h, i)) + t * k * i * 2 + t * k * h * 2
    total = d * (3 * h * i + 2 * scale(i, h) + scale(h, i)) + 2 * t * h * 2 + t * k * 8
    return {"gate_up": gate_up, "down": down, "total": total, "distinct_experts": d}


def algorithmic_flops(cfg: MoeConfig) -> dict[str, int]:
    """Routed GEMM flops: 2 * T * k * (2 * H * I) gate/up and 2 * T * k * H * I down."""
    tk = cfg.tokens * cfg.top_k
    hi = cfg.hidden * cfg.intermediate
    return {"gate_up": 4 * tk * hi, "down": 2 * tk * hi, "total": 6 * tk * hi}
