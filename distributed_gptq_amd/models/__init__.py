"""models: QuantizedLinear and the gptq::linear operator (the reference's
models/layers.py); its model adapters are not part of this path."""
from .layers import FusedQuantizedLinear, QuantizedLinear, replace_with_quantized_layers

__all__ = ["FusedQuantizedLinear", "QuantizedLinear", "replace_with_quantized_layers"]
