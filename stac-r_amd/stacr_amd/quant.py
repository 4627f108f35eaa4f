"""Residual value quantization: the container type and the public quantizer.

Mirrors stacr/quant.py (QuantizedValues :9-27, pack_int4 :30-37, unpack_int4 :40-46,
quantize_values :49-65).  quantize_values runs the HIP quantizer for bits 4/8; bits 0 is a
passthrough (no arithmetic).  pack/unpack/dequantize are the byte-format helpers callers use to
read saved tensors back; the kernels read and write the same layout.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels


@dataclass
class QuantizedValues:
    """Symmetric per-tensor quantized 1-D values: data, fp32 scale, bit width, element count."""

    data: torch.Tensor
    scale: torch.Tensor
    bits: int
    length: int

    def dequantize(self, dtype: torch.dtype) -> torch.Tensor:
        values = unpack_int4(self.data, self.length) if self.bits == 4 else self.data
        return values.to(dtype) * self.scale.to(dtype)

    def stored_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.data, self.scale))


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Two signed nibbles per byte: entry 2i in the low nibble, 2i+1 in the high; odd tail -> 0."""
    flat = values.reshape(-1).to(torch.int8)
    if flat.numel() % 2:
        flat = torch.cat([flat, flat.new_zeros(1)])
    pairs = (flat.view(-1, 2).to(torch.int16) & 0xF).to(torch.uint8)
    return (pairs[:, 0] | (pairs[:, 1] << 4)).contiguous()


def unpack_int4(packed: torch.Tensor, length: int) -> torch.Tensor:
    nibbles = torch.stack([packed & 0xF, (packed >> 4) & 0xF], dim=1).reshape(-1).to(torch.int8)
    return torch.where(nibbles > 7, nibbles - 16, nibbles)[:length]


def quantize_values(values: torch.Tensor, bits: int) -> QuantizedValues:
    """Per-tensor symmetric quantization; ``bits=0`` keeps the values and a unit fp32 scale."""
    if bits not in (0, 4, 8):
        raise ValueError("residual_bits must be 0, 4, or 8")
    flat = values.reshape(-1)
    length = int(flat.numel())
    if bits == 0 or length == 0:
        return QuantizedValues(flat, torch.ones((), dtype=torch.float32, device=flat.device), 0, length)
    data, scale = kernels.quantize(flat, bits)
    return QuantizedValues(data, scale, bits, length)
