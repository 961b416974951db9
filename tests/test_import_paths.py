"""The reference's import paths resolve to this package (drop-in): user code
written for src/distributed_gptq imports unchanged.  No GPU needed."""
import importlib

import pytest


@pytest.mark.parametrize("stmt", [
    "from distributed_gptq import GPTQ, DistributedGPTQuantizer, QuantizationConfig, quantize_model_simple",
    "from distributed_gptq import __version__, DistributedConfig, QuantizationMode, create_distributed_config",
    "from distributed_gptq.core import GPTQ, DistributedGPTQuantizer, QuantizationConfig, quantize_model_simple, "
    "GPTQDequantizer, dequantize_model",
    "from distributed_gptq.core.gptq import GPTQ, GPTQMultiGPU, quantize_layer_gptq",
    "from distributed_gptq.core.quantizer import DistributedGPTQuantizer, QuantizationConfig, quantize_model_simple",
    "from distributed_gptq.core.dequantizer import GPTQDequantizer, dequantize_model",
    "from distributed_gptq.models.layers import QuantizedLinear, replace_with_quantized_layers",
    "from distributed_gptq.models import QuantizedLinear, replace_with_quantized_layers",
    "from distributed_gptq.kernels import check_triton_availability, quantize_tensor, dequantize_tensor, "
    "TritonQuantizedLinear, TRITON_AVAILABLE",
    "from distributed_gptq.kernels.triton_kernels import TritonQuantizedLinear",
])
def test_reference_import_statements(stmt):
    exec(stmt, {})


def test_same_objects_under_both_names():
    import distributed_gptq
    import distributed_gptq_amd
    from distributed_gptq.core.gptq import GPTQ
    from distributed_gptq.models.layers import QuantizedLinear
    assert GPTQ is distributed_gptq_amd.GPTQ
    assert QuantizedLinear is importlib.import_module("distributed_gptq_amd.models.layers").QuantizedLinear
    assert importlib.import_module("distributed_gptq.core.quantizer") is \
        importlib.import_module("distributed_gptq_amd.core.quantizer")
    assert distributed_gptq.__version__ == "0.1.0"
    cfg = distributed_gptq.create_distributed_config()
    assert cfg.world_size >= 1 and cfg.is_main_process in (True, False)


def test_quantization_config_validation_matches_reference_tests():
    """tests/test_quantization.py:95-131 of the reference: defaults, and
    ValueError for bits=5, group_size=0, percdamp=-0.1."""
    from distributed_gptq import QuantizationConfig
    c = QuantizationConfig()
    assert (c.bits, c.group_size, c.actorder, c.percdamp, c.blocksize, c.calibration_samples, c.use_triton,
            c.save_packed) == (4, 128, False, 0.01, 128, 128, False, True)
    for kw in ({"bits": 5}, {"group_size": 0}, {"percdamp": -0.1}, {"percdamp": 1.5}, {"blocksize": 0}):
        with pytest.raises(ValueError):
            QuantizationConfig(**kw)
    assert QuantizationConfig(group_size=-1).group_size == -1
    for b in (2, 3, 4, 8):
        assert QuantizationConfig(bits=b).to_dict()["bits"] == b
