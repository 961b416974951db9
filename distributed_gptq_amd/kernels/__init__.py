"""Kernel entry points under the reference's names
(src/distributed_gptq/kernels/__init__.py:8-22), backed by the HIP library
instead of Triton.

``check_triton_availability()`` / ``TRITON_AVAILABLE`` keep their names for
drop-in code and report whether the accelerated kernels can run (the HIP
library loads and a GPU is present).
"""
from __future__ import annotations

import math

import torch

from .. import _lib as L
from .. import _ops


def _available() -> bool:
    try:
        L.load()
    except Exception:
        return False
    return True


TRITON_AVAILABLE = _available()


def check_triton_availability() -> bool:
    """kernels/triton_kernels.py:22-29: True when the kernels can run."""
    return TRITON_AVAILABLE and torch.cuda.is_available()


def quantize_tensor(tensor: torch.Tensor, bits: int = 4, group_size: int = 128):
    """kernels/triton_kernels.py:377-433: flat groups of ``group_size``
    elements, s = (max - min) / maxq, z = -min / s (not rounded),
    q = clamp(round(x / s + z), 0, maxq) (round half away from zero, as the
    Triton kernel's round) stored as int8.  Returns (q, scales, zeros)."""
    if not check_triton_availability():
        raise RuntimeError("HIP kernels not available")
    return _ops.quantize_tensor(tensor.cuda(), bits, group_size)


def dequantize_tensor(quantized_tensor: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                      group_size: int = 128) -> torch.Tensor:
    """kernels/triton_kernels.py:436-481: (q - z[g]) * s[g] in fp32, q read
    as int8."""
    if not check_triton_availability():
        raise RuntimeError("HIP kernels not available")
    return _ops.dequantize_tensor(quantized_tensor.cuda(), scales.cuda(), zeros.cuda(), group_size)


class TritonQuantizedLinear:
    """kernels/triton_kernels.py:225-374 with HIP kernels: int8 codes (one per
    byte), fp16 per-(row, group) scales and unrounded zeros."""

    def __init__(self, in_features: int, out_features: int, bits: int = 4, group_size: int = 128,
                 bias: bool = True):
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.use_bias = bias
        self.n_groups = math.ceil(in_features / group_size)
        self.qweight = torch.zeros((out_features, in_features), dtype=torch.int8, device="cuda")
        self.scales = torch.ones((out_features, self.n_groups), dtype=torch.float16, device="cuda")
        self.zeros = torch.zeros((out_features, self.n_groups), dtype=torch.float16, device="cuda")
        self.bias = torch.zeros(out_features, dtype=torch.float32, device="cuda") if bias else None

    def quantize_weights(self, weights: torch.Tensor):
        """:267-308: per (row, group) s = (max - min)/maxq, z = -min/s stored
        as fp16, then q = clamp(round(w/s + z), 0, maxq) with the stored
        values."""
        if not check_triton_availability():
            raise RuntimeError("Triton not available for quantization")
        w = weights.cuda().contiguous()
        N, K = w.shape
        if K % self.group_size:
            raise ValueError("in_features must be a multiple of group_size")
        _, s, z = _ops.quantize_tensor(w.float(), self.bits, self.group_size)
        self.scales = s.reshape(N, self.n_groups).to(torch.float16)
        self.zeros = z.reshape(N, self.n_groups).to(torch.float16)
        q, _, _ = _ops.quantize_tensor(w, self.bits, self.group_size, scales=self.scales.float(),
                                       zeros=self.zeros.float())
        self.qweight = q.reshape(N, K)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """:310-345: y = x @ ((q - z) * s)^T + bias, in x's dtype."""
        codes = self.qweight.view(torch.uint8)
        y = _ops.linear(x, codes, 0, self.scales, self.zeros, self.in_features, group_size=self.group_size,
                        bias=self.bias.to(x.dtype) if self.bias is not None else None)
        return y

    __call__ = forward


__all__ = ["check_triton_availability", "quantize_tensor", "dequantize_tensor", "TritonQuantizedLinear",
           "TRITON_AVAILABLE"]
