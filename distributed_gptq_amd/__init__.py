"""MI355X-native GPTQ hot path behind the Python API of
kambojvikram/Distributed_GPTQ (src/distributed_gptq/__init__.py:11-31).

Compute runs in libgptq_hip.so (hand-written gfx950 HIP kernels behind a
C ABI, include/gptq_hip.h); this package mirrors the reference's import
paths: ``core.gptq`` (GPTQ), ``core.quantizer`` (QuantizationConfig,
Quantizer), ``core.dequantizer``, ``models.layers`` (QuantizedLinear and the
gptq::linear operator) and ``kernels``; ``core.checkpoint`` holds the
reference quantizer's save/load (safetensors + JSON sidecar).
"""
from .core.gptq import GPTQ, GPTQMultiGPU, quantize_layer_gptq
from .core.quantizer import (DistributedConfig, DistributedGPTQuantizer, QuantizationConfig, QuantizationMode,
                             Quantizer, create_distributed_config, quantize_model_simple)
from .core.dequantizer import GPTQDequantizer, dequantize_model

__version__ = "0.1.0"

__all__ = ["__version__", "GPTQ", "GPTQMultiGPU", "quantize_layer_gptq", "DistributedGPTQuantizer",
           "QuantizationConfig", "Quantizer", "quantize_model_simple", "GPTQDequantizer", "dequantize_model",
           "DistributedConfig", "QuantizationMode", "create_distributed_config",
           "QuantizedLinear", "replace_with_quantized_layers", "save_quantized_model", "load_quantized_model"]


def __getattr__(name):
    # models.layers registers the gptq::linear operator on import
    if name in ("QuantizedLinear", "replace_with_quantized_layers"):
        from .models import layers
        return getattr(layers, name)
    if name in ("save_quantized_model", "load_quantized_model"):
        from .core import checkpoint
        return getattr(checkpoint, name)
    raise AttributeError(name)
