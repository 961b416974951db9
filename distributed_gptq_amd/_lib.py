"""ctypes binding of libgptq_hip.so (the C ABI declared in include/gptq_hip.h).

torch is imported first so that its bundled HIP runtime (soname
libamdhip64.so.7) is the one the library binds to: device pointers and
stream handles from torch are passed straight through.

There is no fallback: if the library is missing, or no GPU is present,
every compute entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see module doc)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgptq_hip.so")

# status codes (gptq_status)
OK, ERR_ARG, ERR_SHAPE, ERR_DTYPE, ERR_WORKSPACE, ERR_LAUNCH, ERR_DEVICE = range(7)
# dtypes (gptq_dtype)
F32, F16, BF16 = 0, 1, 2
# factor modes / sweep flags
FACTOR_FULL_INVERSE, FACTOR_UPPER_CHOL_INV = 0, 1
SWEEP_TRAILING, SWEEP_REF_QUANTIZER, SWEEP_GROUPS_FROM_W0, PARAMS_SYM = 1, 2, 4, 8
TENSOR_PARAMS_GIVEN = 1

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the exact list of exported entry points
SIGNATURES = {
    "gptq_last_error": (ctypes.c_char_p, []),
    "gptq_abi_version": (_i, []),
    "gptq_hessian_workspace_size": (_sz, [_i64, _i64]),
    "gptq_hessian_workspace_min": (_sz, [_i64]),
    "gptq_hessian_accumulate": (_i, [_p, _p, _i64, _i64, _i64, _i, _p, _sz, _p]),
    "gptq_factor_workspace_size": (_sz, [_i64]),
    "gptq_damp_factor": (_i, [_p, _i64, _f, _f, _p, _i, _p, _p, _p, _p, _p, _sz, _p]),
    "gptq_sweep_workspace_size": (_sz, [_i64, _i64, _i]),
    "gptq_quantize_sweep": (_i, [_p, _p, _p, _i64, _i64, _i64, _i, _i, _i, _i, _p, _p, _p, _i,
                                 _p, _p, _p, _p, _p, _sz, _p]),
    "gptq_minmax_params": (_i, [_p, _i64, _i64, _i64, _i, _i, _i, _p, _p, _p]),
    "gptq_quantize_rows": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _p, _p, _p]),
    "gptq_prepare_weight": (_i, [_p, _i, _i64, _i64, _i64, _p, _p, _i, _p, _p]),
    "gptq_pack": (_i, [_p, _i64, _i64, _i, _p, _p]),
    "gptq_unpack": (_i, [_p, _i64, _i64, _i, _p, _p]),
    "gptq_pack_reference_layout": (_i, [_p, _i64, _i64, _i, _p, _p]),
    "gptq_dequant": (_i, [_p, _i, _p, _p, _i, _p, _i, _i64, _i64, _i64, _p, _p]),
    "gptq_dequant_to": (_i, [_p, _i, _p, _p, _i, _p, _i, _i64, _i64, _i64, _p, _i, _p]),
    "gptq_linear": (_i, [_p, _i, _i64, _p, _i, _p, _p, _i, _p, _i, _i64, _p, _i, _i64, _i64, _p, _p]),
    "gptq_linear_perm_workspace_size": (_sz, [_i64, _i64, _i]),
    "gptq_linear_workspace_size": (_sz, [_i64, _i64, _i64, _i, _i, _i, _i]),
    "gptq_linear_ws": (_i, [_p, _i, _i64, _p, _p, _i, _p, _p, _i, _p, _i, _i64, _p, _i, _i64, _i64, _p, _p, _sz, _p]),
    "gptq_linear_perm": (_i, [_p, _i, _i64, _p, _p, _i, _p, _p, _i, _p, _i, _i64, _p, _i, _i64, _i64, _p, _p, _sz,
                              _p]),
    "gptq_linear_perm_noalloc_max_bytes": (_sz, []),
    "gptq_linear_perm_noalloc": (_i, [_p, _i, _i64, _p, _p, _i, _p, _p, _i, _p, _i, _i64, _p, _i, _i64, _i64, _p,
                                      _p]),
    "gptq_quantize_tensor": (_i, [_p, _i, _i64, _i, _i, _i, _p, _p, _p, _p]),
    "gptq_dequantize_tensor": (_i, [_p, _i64, _i, _p, _p, _p, _p]),
    "gptq_stream_read": (_i, [_p, _sz, _i, _i, _p, _p]),
}


class GPTQLibraryError(RuntimeError):
    """A C-ABI call returned a non-zero gptq_status."""

    def __init__(self, status, fn, msg):
        super().__init__(f"{fn} failed (status {status}): {msg}")
        self.status = status


_lock = threading.Lock()
_handle = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library (once) and declare every entry point."""
    global _handle
    with _lock:
        if _handle is None:
            if not os.path.exists(path):
                raise ImportError(
                    f"{path} is not built: run `python -m distributed_gptq_amd.build` "
                    "(this package has no CPU fallback)")
            h = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _handle = h
        return _handle


def lib() -> ctypes.CDLL:
    return load()


def check(status: int, fn: str):
    if status == OK:
        return
    msg = lib().gptq_last_error().decode(errors="replace")
    if status in (ERR_ARG, ERR_SHAPE):
        raise ValueError(f"{fn}: {msg}")
    if status == ERR_DTYPE:
        raise TypeError(f"{fn}: {msg}")
    raise GPTQLibraryError(status, fn, msg)


def call(name: str, *args):
    """Call entry point ``name`` and raise on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    check(rc, name)
    return rc


def require_gpu(t: torch.Tensor | None = None):
    """The product path runs on the GPU only; fail loudly otherwise."""
    if not torch.cuda.is_available():
        raise RuntimeError("distributed_gptq_amd needs an AMD GPU (gfx950) and has no CPU fallback")
    if t is not None and t.device.type != "cuda":
        raise RuntimeError(f"expected a GPU tensor, got one on {t.device}")
    load()
