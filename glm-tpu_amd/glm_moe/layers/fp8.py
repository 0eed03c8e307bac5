"""FP8 E4M3FN bit decoding and block-scale application on the GPU.

Mirrors ``glm_tpu/layers/fp8.py`` of the reference: ``fp8_e4m3fn_lookup``
(``:18-34``), ``dequantize_fp8_bits_block_weight`` (``:37-72``) and
``decode_fp8_table`` (``:113-126``).  The decode runs in libglm_moe's HIP
kernel (``v_cvt_pk_f32_fp8``, one FP32 multiply, RNE to bf16).
"""

from __future__ import annotations

from functools import lru_cache

import torch

from glm_moe import _lib


@lru_cache(maxsize=1)
def fp8_e4m3fn_lookup() -> tuple[float, ...]:
    """The exact 256-entry E4M3FN decode table as host literals (``fp8.py:18-34``)."""
    values = []
    for bits in range(256):
        sign = -1.0 if bits & 0x80 else 1.0
        exponent = (bits >> 3) & 0xF
        mantissa = bits & 0x7
        if exponent == 0:
            value = mantissa * (2.0**-9)
        elif exponent == 15 and mantissa == 7:
            value = float("nan")
        else:
            value = (1.0 + mantissa / 8.0) * (2.0 ** (exponent - 7))
        values.append(sign * value)
    return tuple(values)


def decode_fp8_table(bits: torch.Tensor, scale: torch.Tensor, *, block_shape: tuple[int, int] = (128, 128)) -> torch.Tensor:
    """``bf16(f32(bits) * scale_block)`` for uint8 ``[N, K]`` bits (``fp8.py:113-126``)."""
    if bits.ndim != 2 or scale.ndim != 2 or bits.dtype != torch.uint8 or scale.dtype != torch.float32:
        raise ValueError("decode_fp8_table takes uint8 [N,K] bits and float32 [N/bn,K/bk] scales")
    n, k = bits.shape
    bn, bk = block_shape
    if tuple(scale.shape) != ((n + bn - 1) // bn, (k + bk - 1) // bk):
        raise ValueError("decode_fp8_table scale geometry disagrees with the bits")
    _lib.require_device(bits, scale)
    out = torch.empty((n, k), dtype=torch.bfloat16, device=bits.device)
    _lib.call("glm_moe_decode_fp8_table", _lib.ptr(bits), _lib.ptr(scale), n, k, bn, bk, _lib.ptr(out),
              _lib.stream_of(bits))
    return out


def dequantize_fp8_bits_block_weight(
    weight_bits: torch.Tensor,
    scale: torch.Tensor,
    *,
    block_shape: tuple[int, int] = (128, 128),
    output_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Decode raw checkpoint U8 bits with colocated FP32 block scales (``fp8.py:37-72``).

    Leading dimensions are preserved; only the final ``[out, in]`` dimensions
    are block-scaled.  The value is always the bf16 decode; ``output_dtype``
    only widens it.
    """
    if weight_bits.ndim < 2 or scale.ndim != weight_bits.ndim:
        raise ValueError("FP8 bits and scales must have matching rank >= 2")
    if tuple(weight_bits.shape[:-2]) != tuple(scale.shape[:-2]):
        raise ValueError("FP8 bits/scales leading dimensions disagree")
    if weight_bits.dtype != torch.uint8:
        raise ValueError(f"FP8 storage must be uint8 bits, got {weight_bits.dtype}")
    if len(block_shape) != 2 or any(not isinstance(i, int) or isinstance(i, bool) or i <= 0 for i in block_shape):
        raise ValueError("block_shape must contain two positive integers")
    expected = tuple((d + b - 1) // b for d, b in zip(weight_bits.shape[-2:], block_shape))
    if tuple(scale.shape[-2:]) != expected:
        raise ValueError(f"FP8 scale tail must be {expected}, got {tuple(scale.shape[-2:])}")
    n, k = weight_bits.shape[-2:]
    flat_bits = weight_bits.reshape(-1, n, k)
    flat_scale = scale.reshape(-1, *expected)
    out = torch.empty(flat_bits.shape, dtype=torch.bfloat16, device=weight_bits.device)
    for i in range(flat_bits.shape[0]):
        out[i] = decode_fp8_table(flat_bits[i], flat_scale[i].contiguous(), block_shape=block_shape)
    return out.reshape(weight_bits.shape).to(output_dtype)
