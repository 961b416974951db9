"""core: GPTQ, QuantizationConfig, Quantizer, GPTQDequantizer
(src/distributed_gptq/core/__init__.py:5-15)."""
from .gptq import GPTQ, GPTQMultiGPU, quantize_layer_gptq
from .quantizer import (DistributedConfig, DistributedGPTQuantizer, QuantizationConfig, QuantizationMode, Quantizer,
                        create_distributed_config, quantize_model_simple)
from .dequantizer import GPTQDequantizer, dequantize_model

__all__ = ["GPTQ", "GPTQMultiGPU", "quantize_layer_gptq", "DistributedGPTQuantizer", "QuantizationConfig", "Quantizer",
           "quantize_model_simple", "GPTQDequantizer", "dequantize_model", "DistributedConfig", "QuantizationMode",
           "create_distributed_config"]
