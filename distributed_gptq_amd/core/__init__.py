"""core: GPTQ, QuantizationConfig, Quantizer, GPTQDequantizer
(src/distributed_gptq/core/__init__.py:5-15)."""
from .gptq import GPTQ, GPTQMultiGPU, quantize_layer_gptq
from .quantizer import QuantizationConfig, Quantizer
from .dequantizer import GPTQDequantizer

__all__ = ["GPTQ", "GPTQMultiGPU", "quantize_layer_gptq", "QuantizationConfig", "Quantizer", "GPTQDequantizer"]
