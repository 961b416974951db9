"""The reference's import path, ``distributed_gptq``, for drop-in use.

User code written against kambojvikram/Distributed_GPTQ imports
``distributed_gptq`` and its submodules (src/distributed_gptq/__init__.py:11-31,
core/__init__.py:5-15, models/layers.py, kernels/__init__.py:8-22).  Each of
those module paths is registered here as the corresponding module of
``distributed_gptq_amd`` itself (the same module objects, so classes,
isinstance checks and monkeypatching agree under both names):

    distributed_gptq                         -> distributed_gptq_amd
    distributed_gptq.core(.gptq|.quantizer|.dequantizer)
    distributed_gptq.models(.layers)
    distributed_gptq.kernels(.triton_kernels)

The reference's multi-process coordinator (``DistributedGPTQCoordinator``,
distributed/) is not part of this single-GPU build.
"""
import sys

import distributed_gptq_amd as _impl
from distributed_gptq_amd import core as _core
from distributed_gptq_amd import kernels as _kernels
from distributed_gptq_amd import models as _models
from distributed_gptq_amd.core import dequantizer as _dequantizer
from distributed_gptq_amd.core import gptq as _gptq
from distributed_gptq_amd.core import quantizer as _quantizer
from distributed_gptq_amd.models import layers as _layers

for _name, _mod in {"core": _core, "core.gptq": _gptq, "core.quantizer": _quantizer,
                    "core.dequantizer": _dequantizer, "models": _models, "models.layers": _layers,
                    "kernels": _kernels, "kernels.triton_kernels": _kernels}.items():
    sys.modules[f"{__name__}.{_name}"] = _mod

core, models, kernels = _core, _models, _kernels

from distributed_gptq_amd import *  # noqa: E402,F401,F403
from distributed_gptq_amd import __all__, __version__  # noqa: E402,F401


def __getattr__(name):
    return getattr(_impl, name)
