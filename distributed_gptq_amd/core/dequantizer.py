"""GPTQDequantizer and dequantize_model (src/distributed_gptq/core/dequantizer.py:14-163).

``dequantize_weight`` computes (q - zeros) * scales in fp32 with the 4-bit
low-nibble-first unpack of ``_unpack_4bit`` (:68-89); both run in the HIP
library and are bit-exact against the torch formula.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .. import _ops


class GPTQDequantizer:
    def __init__(self, bits: int = 4, group_size: int = 128):
        self.bits = bits
        self.group_size = group_size
        self.max_val = 2 ** bits - 1

    def dequantize_weight(self, qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                          g_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
        """(q - zero[g]) * scale[g] per output row (:31-66); ``g_idx[k]`` is
        the group of input column k (default k // group_size).  4-bit weights
        are packed two per byte, low nibble first; other widths one code per
        byte."""
        N = qweight.shape[0]
        if self.bits == 4:
            K = qweight.shape[1] * 2
            bits = 4
        else:
            K = qweight.shape[1]
            bits = 0
        if scales.dim() == 1:
            scales = scales.reshape(N, -1)
            zeros = zeros.reshape(N, -1)
        return _ops.dequant(qweight, bits, scales, zeros, K, g_idx=g_idx, group_size=self.group_size)

    def _unpack_4bit(self, qweight: torch.Tensor) -> torch.Tensor:
        """uint8 (N, K/2) -> float (N, K): low nibble -> even index (:86-87)."""
        return _ops.unpack(qweight, 4, qweight.shape[1] * 2).float()

    def dequantize_layer(self, layer: nn.Module) -> nn.Module:
        from ..models.layers import QuantizedLinear
        if not isinstance(layer, QuantizedLinear):
            return layer
        out = nn.Linear(layer.in_features, layer.out_features, bias=layer.bias is not None,
                        device=layer.qweight.device)
        out.weight.data = layer.unpack_weights()
        if layer.bias is not None:
            out.bias.data = layer.bias.data.float()
        return out

    def dequantize_model(self, model: nn.Module) -> nn.Module:
        """Every QuantizedLinear of ``model`` replaced by an nn.Linear holding
        its fp32 dequantised weights (:123-142); returns ``model``."""
        for name, child in model.named_children():
            if len(list(child.children())) > 0:
                setattr(model, name, self.dequantize_model(child))
            else:
                setattr(model, name, self.dequantize_layer(child))
        return model


def dequantize_model(model: nn.Module, bits: int = 4, group_size: int = 128) -> nn.Module:
    """:145-163."""
    return GPTQDequantizer(bits=bits, group_size=group_size).dequantize_model(model)
