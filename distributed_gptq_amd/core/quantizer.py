"""QuantizationConfig and the min-max Quantizer (find_params / quantize).

``QuantizationConfig`` mirrors src/distributed_gptq/core/quantizer.py:24-40
(same fields and defaults); invalid values raise ValueError at construction
(the reference's ``validate()`` asserts, :36-40, and its tests expect
ValueError, tests/test_quantization.py:119-131).  ``group_size=-1`` means one
group per output row (per-channel).

``Quantizer`` carries the find_params/quantize names of canonical GPTQ (the
reference inlines the same min-max arithmetic at core/gptq.py:159-179); its
arithmetic runs in the HIP library.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass

import torch
import torch.nn as nn

from .. import _lib as L
from .. import _ops


@dataclass
class QuantizationConfig:
    """Configuration for GPTQ quantization (core/quantizer.py:24-34)."""
    bits: int = 4
    group_size: int = 128
    actorder: bool = False
    percdamp: float = 0.01
    blocksize: int = 128
    calibration_samples: int = 128
    use_triton: bool = False
    save_packed: bool = True

    def __post_init__(self):
        self.validate()

    def validate(self):
        """core/quantizer.py:36-40, raising ValueError instead of asserting."""
        if self.bits not in (2, 3, 4, 8):
            raise ValueError(f"Bits must be 2, 3, 4, or 8, got {self.bits}")
        if not (self.group_size > 0 or self.group_size == -1):
            raise ValueError(f"Group size must be positive (or -1 for per-channel), got {self.group_size}")
        if not 0 <= self.percdamp <= 1:
            raise ValueError(f"Percdamp must be between 0 and 1, got {self.percdamp}")
        if self.blocksize <= 0:
            raise ValueError(f"Blocksize must be positive, got {self.blocksize}")

    def to_dict(self):
        return asdict(self)


class Quantizer(nn.Module):
    """Asymmetric (or symmetric) min-max quantizer.

    ``formula="canonical"``: xmin = min(x, 0), xmax = max(x, 0), an all-zero
    row gets [-1, 1]; codes = clamp(round(x / s) + z, 0, maxq).
    ``formula="reference"``: raw min/max (core/gptq.py:165-169) and
    codes = clamp(round(x / s + z), 0, maxq) (:175).
    Both: s = (xmax - xmin) / maxq, z = round(-xmin / s),
    quantize(x) = s * (codes - z) (:179).
    """

    def __init__(self, shape=1):
        super().__init__()
        self.register_buffer("maxq", torch.tensor(0))
        self.register_buffer("scale", torch.zeros(shape))
        self.register_buffer("zero", torch.zeros(shape))
        self.bits = 0
        self.perchannel = False
        self.sym = True
        self.formula = "canonical"
        self.group_size = -1

    def configure(self, bits, perchannel=False, sym=True, mse=False, norm=2.4, grid=100, maxshrink=.8,
                  trits=False, formula="canonical", group_size=-1):
        if mse or trits:
            raise NotImplementedError("mse grid search and ternary codes are not part of this path")
        if formula not in ("canonical", "reference"):
            raise ValueError("formula must be 'canonical' or 'reference'")
        if formula == "reference" and sym:
            sym = False  # the reference quantizer is asymmetric only
        self.bits = int(bits)
        self.maxq = torch.tensor(2 ** self.bits - 1)
        self.perchannel = perchannel
        self.sym = sym
        self.formula = formula
        self.group_size = group_size

    def _flags(self):
        f = L.SWEEP_REF_QUANTIZER if self.formula == "reference" else 0
        if self.sym and self.formula == "canonical":
            f |= L.PARAMS_SYM
        return f

    def _rows(self, x, weight):
        if weight:
            return x.reshape(x.shape[0], -1) if self.perchannel else x.reshape(1, -1)
        if not self.perchannel:
            return x.reshape(1, -1)
        # activations: one row per feature (last dim)
        return x.reshape(-1, x.shape[-1]).t()

    def find_params(self, x: torch.Tensor, weight: bool = False):
        if self.bits == 0:
            raise RuntimeError("call configure(bits, ...) first")
        rows = self._rows(x, weight).float().contiguous()
        gs = self.group_size if (weight and self.perchannel) else -1
        self.scale, self.zero = _ops.minmax_params(rows, self.bits, gs, self._flags())
        if not weight and self.perchannel:
            shape = [1] * (x.dim() - 1) + [-1]
            self.scale = self.scale.reshape(shape)
            self.zero = self.zero.reshape(shape)

    def codes(self, x: torch.Tensor, weight: bool = True) -> torch.Tensor:
        rows = self._rows(x, weight)
        gs = self.group_size if (weight and self.perchannel) else -1
        c, _ = _ops.quantize_rows(rows, self.scale.reshape(rows.shape[0], -1), self.zero.reshape(rows.shape[0], -1),
                                  self.bits, gs, self._flags(), True, False)
        return c.reshape(x.shape) if weight else c.t().reshape(x.shape)

    def quantize(self, x: torch.Tensor, weight: bool = True) -> torch.Tensor:
        if not self.ready():
            return x
        rows = self._rows(x, weight)
        gs = self.group_size if (weight and self.perchannel) else -1
        _, dq = _ops.quantize_rows(rows, self.scale.reshape(rows.shape[0], -1), self.zero.reshape(rows.shape[0], -1),
                                   self.bits, gs, self._flags(), False, True)
        out = dq if weight or not self.perchannel else dq.t()
        return out.reshape(x.shape).to(x.dtype)

    def enabled(self):
        return self.bits > 0

    def ready(self):
        return bool(torch.all(self.scale != 0))
