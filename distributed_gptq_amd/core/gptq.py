"""GPTQ per-layer quantization on the HIP library.

``GPTQ`` keeps the interface of src/distributed_gptq/core/gptq.py:16-266:
constructor arguments, ``add_batch(inp, out)`` (:63-89), ``quantize()``
(:91-214, reference semantics), ``pack_weights()`` (:216-266) and the
attributes H, nsamples, H_inv, scale, zero, maxq, layer.  It adds
``fasterquant()``, the canonical GPTQ sweep (upper Cholesky factor of H^-1,
lazy-batch trailing update, act-order) that the reference's class is named
after but does not implement.

Differences from the reference, all deliberate:
  * ``quantize()`` repairs the broadcast at :175 (the column is used as a
    (K, 1) vector; as written the reference raises on its first column) and
    raises ValueError for the shapes it cannot define (out_features >
    in_features or out_features % group_size != 0, :125-126, :153).
  * a constant group (max == min) uses s = 1 instead of dividing by zero.
  * ``add_batch`` stages small batches in a device buffer and accumulates
    them into H in larger launches (H is exact either way; reading ``H``
    flushes the buffer).
  * only nn.Linear layers are supported (the reference's Conv2d branch never
    reshapes its input, :76-79).
"""
from __future__ import annotations

import logging
from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn

from .. import _lib as L
from .. import _ops

logger = logging.getLogger(__name__)


class GPTQ:
    """GPTQ quantizer for one nn.Linear layer (core/gptq.py:16-61)."""

    def __init__(self, layer: nn.Module, bits: int = 4, group_size: int = 128, actorder: bool = False,
                 percdamp: float = 0.01, blocksize: int = 128, device: Optional[torch.device] = None,
                 layer_name: Optional[str] = None, token_buffer: int = 32768):
        if not isinstance(layer, nn.Linear):
            raise NotImplementedError("GPTQ here quantizes nn.Linear layers")
        if bits not in (2, 3, 4, 8):
            raise ValueError(f"bits must be 2, 3, 4 or 8, got {bits}")
        self.layer = layer
        self.layer_name = layer_name
        self.bits = bits
        self.group_size = group_size
        self.actorder = actorder
        self.percdamp = percdamp
        self.blocksize = blocksize
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda" if torch.cuda.is_available() else "cpu")
        self.maxq = 2 ** self.bits - 1
        self.scale = None
        self.zero = None
        self.g_idx = None
        self.perm = None
        self.qcodes = None
        self.H_inv = None
        self.nsamples = 0
        self._H = None
        self._buf = None
        self._buf_n = 0
        self._buf_cap = int(token_buffer)
        self._mode = None

    # ---------------------------------------------------------- Hessian --
    @property
    def H(self):
        self._flush()
        return self._H

    @H.setter
    def H(self, value):
        self._flush()
        self._H = value

    def _flush(self):
        if self._buf is not None and self._buf_n:
            _ops.hessian_accumulate(self._H, self._buf[:self._buf_n])
        self._buf_n = 0

    def add_batch(self, inp: torch.Tensor, out: Optional[torch.Tensor] = None):
        """H += X^T X over the tokens of ``inp`` (core/gptq.py:63-89).
        ``nsamples`` counts sequences (the leading dimension), as the
        reference does (:74, :81); ``out`` is accepted and ignored."""
        L.require_gpu()
        if self.device.type != "cuda":
            raise RuntimeError("GPTQ runs on the GPU; construct it with a cuda device")
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        bsz = inp.shape[0]
        K = inp.shape[-1]
        x = inp.reshape(-1, K)
        if x.device != self.device:
            x = x.to(self.device, non_blocking=True)
        if x.dtype not in _ops.DTYPES:
            x = x.float()
        self.nsamples += bsz
        if self._H is None:
            self._H = torch.zeros((K, K), dtype=torch.float32, device=self.device)
        elif self._H.shape[0] != K:
            raise ValueError(f"input has {K} features, the Hessian is {self._H.shape[0]} x {self._H.shape[0]}")
        n = x.shape[0]
        if self._buf_cap <= 0 or n >= self._buf_cap // 2:
            self._flush()
            _ops.hessian_accumulate(self._H, x)
            return
        if self._buf is None or self._buf.dtype != x.dtype or self._buf.shape[1] != K:
            self._flush()
            self._buf = torch.empty((self._buf_cap, K), dtype=x.dtype, device=self.device)
        if self._buf_n + n > self._buf_cap:
            self._flush()
        self._buf[self._buf_n:self._buf_n + n].copy_(x)
        self._buf_n += n

    def free(self):
        """Drop the Hessian, staging buffer and factors."""
        self._H = None
        self._buf = None
        self._buf_n = 0
        self.H_inv = None

    # -------------------------------------------------- reference sweep --
    def quantize(self) -> Dict[str, Any]:
        """Reference semantics (core/gptq.py:91-214): H /= nsamples, damping,
        full inverse, transposed column sweep with intra-block propagation,
        layer weight replaced by the fp32 codes."""
        H = self.H
        if H is None:
            raise RuntimeError("no calibration data: call add_batch() before quantize()")
        W = self.layer.weight.data
        N, K = W.shape
        gs = self.group_size
        if gs <= 0 or N > K or N % gs:
            raise ValueError(
                f"the reference sweep is defined for out_features <= in_features and out_features % group_size == 0"
                f" (core/gptq.py:125-126, :153); got out={N}, in={K}, group_size={gs}; use fasterquant()")
        Hinv, Hd, _, info = _ops.damp_factor(H, 1.0 / self.nsamples, self.percdamp, None,
                                             L.FACTOR_FULL_INVERSE, want_hd=True)
        A = _ops.prepare_weight(W, transpose=True)  # (K, N): W = weight.t() (:107-108)
        res = _ops.quantize_sweep(A, Hinv, self.bits, gs, self.blocksize, L.SWEEP_REF_QUANTIZER)
        if int(info.item()) != 0:
            raise torch.linalg.LinAlgError(
                "cholesky: the damped Hessian is not positive-definite (core/gptq.py:122)")
        self._H = Hd  # the reference normalises and damps self.H in place (:113-119)
        self.H_inv = Hinv
        self.scale = res["scale"]
        self.zero = res["zero"]
        self.layer.weight.data = res["codes"].t().float()
        total_error = float(res["err_sq"].double().sum().item())
        self._mode = "reference"
        return {
            "bits": self.bits,
            "group_size": self.group_size,
            "total_error": total_error,
            "compression_ratio": 32.0 / self.bits,
            "scale_shape": self.scale.shape,
            "zero_shape": self.zero.shape,
        }

    # -------------------------------------------------- canonical sweep --
    def fasterquant(self, blocksize: Optional[int] = None, percdamp: Optional[float] = None,
                    groupsize: Optional[int] = None, actorder: Optional[bool] = None,
                    static_groups: bool = False) -> Dict[str, Any]:
        """Canonical GPTQ: H = 2/nsamples * sum x x^T, dead inputs zeroed,
        optional act-order, damping, U = chol(H^-1) upper, lazy-batch sweep;
        the layer weight becomes the dequantized weights (layer dtype)."""
        if static_groups:
            raise NotImplementedError("static_groups is not part of this path")
        bs = self.blocksize if blocksize is None else blocksize
        pd = self.percdamp if percdamp is None else percdamp
        gs = self.group_size if groupsize is None else groupsize
        ao = self.actorder if actorder is None else actorder
        H = self.H
        if H is None:
            raise RuntimeError("no calibration data: call add_batch() before fasterquant()")
        W = self.layer.weight.data
        N, K = W.shape
        if gs > K:
            gs = K
        scale = zero = None
        if gs <= 0:
            # per-channel parameters from the original weights (before dead columns are zeroed)
            scale, zero = _ops.minmax_params(W.float(), self.bits, -1, 0)
        scl = 2.0 / self.nsamples
        perm = None
        if ao:
            d = torch.diagonal(H) * scl
            d = torch.where(d == 0, torch.ones_like(d), d)
            perm = torch.argsort(d, descending=True, stable=True).to(torch.int32)
        U, _, dead, info = _ops.damp_factor(H, scl, pd, perm, L.FACTOR_UPPER_CHOL_INV, want_dead=True)
        Wp = _ops.prepare_weight(W, perm=perm, dead=dead)
        res = _ops.quantize_sweep(Wp, U, self.bits, gs, bs, L.SWEEP_TRAILING, out_cols=perm,
                                  dequant_dtype=W.dtype, scale=scale, zero=zero, want_losses=True,
                                  want_err=False)
        if int(info.item()) != 0:
            raise torch.linalg.LinAlgError("cholesky: the damped Hessian is not positive-definite")
        if perm is None:
            g_idx = torch.arange(K, device=W.device, dtype=torch.int32) // max(gs, 1) if gs > 0 else \
                torch.zeros(K, device=W.device, dtype=torch.int32)
        else:
            g_idx = torch.empty(K, device=W.device, dtype=torch.int32)
            g_idx[perm.long()] = (torch.arange(K, device=W.device, dtype=torch.int32) // gs) if gs > 0 else 0
        self.layer.weight.data = res["dequant"]
        self.scale, self.zero = res["scale"], res["zero"]
        self.g_idx, self.perm = g_idx, perm
        self.qcodes = res["codes"]
        self.losses = res["losses"]
        self.H_inv = U
        self._mode = "canonical"
        self._gs_used = gs
        total = float(res["losses"].double().sum().item())
        return {
            "bits": self.bits,
            "group_size": gs,
            "total_error": total,
            "compression_ratio": 32.0 / self.bits,
            "scale_shape": self.scale.shape,
            "zero_shape": self.zero.shape,
        }

    # ------------------------------------------------------------ packing --
    def _codes_nk(self) -> torch.Tensor:
        if self._mode == "canonical":
            return self.qcodes
        if self._mode == "reference":
            return self.layer.weight.data.round().clamp(0, 255).to(torch.uint8)
        raise RuntimeError("quantize() or fasterquant() first")

    def pack_weights(self) -> Dict[str, torch.Tensor]:
        """``GPTQ.pack_weights`` layout (core/gptq.py:216-266): on W = codes^T
        (K x N), 4-bit MSB-first pairs along N, 2-bit weights 64/16/4/1,
        3-bit uint8 and 8-bit int8 unpacked."""
        codes = self._codes_nk()
        packed = _ops.pack_reference_layout(codes, self.bits)
        N, K = codes.shape
        return {
            "packed_weights": packed,
            "scale": self.scale,
            "zero": self.zero,
            "bits": self.bits,
            "group_size": self.group_size,
            "shape": torch.Size((K, N)),
        }

    def pack_native(self) -> Dict[str, torch.Tensor]:
        """Native GEMV layout: LSB-first bit stream per output row, fp16
        scales/zeros (N x groups), g_idx (K,) -- what QuantizedLinear and
        gptq::linear consume.  Canonical (fasterquant) results only."""
        if self._mode != "canonical":
            raise RuntimeError("pack_native() needs fasterquant() results (out_features x in_features codes)")
        return {
            "qweight": _ops.pack(self.qcodes, self.bits),
            "scales": self.scale.to(torch.float16),
            "zeros": self.zero.to(torch.float16),
            "g_idx": self.g_idx,
            "bits": self.bits,
            "group_size": self._gs_used,
        }


class GPTQMultiGPU:
    """core/gptq.py:269-380, re-targeted at one GPU: layers are prepared on a
    single device and quantized one after another (a sequential layer loop
    instead of ``hash(name) % n_devices`` placement, :323)."""

    def __init__(self, model: nn.Module, bits: int = 4, group_size: int = 128, actorder: bool = False,
                 percdamp: float = 0.01, blocksize: int = 128, devices: Optional[List[torch.device]] = None):
        self.model = model
        self.bits = bits
        self.group_size = group_size
        self.actorder = actorder
        self.percdamp = percdamp
        self.blocksize = blocksize
        self.devices = list(devices) if devices else [torch.device("cuda", 0)]
        self.layer_quantizers: Dict[str, GPTQ] = {}

    def prepare_layer(self, layer_name: str, layer: nn.Module) -> GPTQ:
        device = self.devices[0]
        layer = layer.to(device)
        q = GPTQ(layer, bits=self.bits, group_size=self.group_size, actorder=self.actorder,
                 percdamp=self.percdamp, blocksize=self.blocksize, device=device, layer_name=layer_name)
        self.layer_quantizers[layer_name] = q
        return q

    def add_batch_to_all(self, inputs: Dict[str, torch.Tensor]):
        for name, q in self.layer_quantizers.items():
            if name in inputs:
                q.add_batch(inputs[name])

    def quantize_all_layers(self, canonical: bool = True) -> Dict[str, Dict[str, Any]]:
        results = {}
        for name, q in self.layer_quantizers.items():
            logger.info("Quantizing layer: %s", name)
            results[name] = q.fasterquant() if canonical else q.quantize()
            q.free()
        return results

    def get_quantized_model(self) -> nn.Module:
        return self.model


def quantize_layer_gptq(layer: nn.Module, calibration_data, bits: int = 4, group_size: int = 128,
                        canonical: bool = False, **kwargs) -> Dict[str, Any]:
    """core/gptq.py:383-417: add every calibration batch, then quantize."""
    q = GPTQ(layer, bits=bits, group_size=group_size, **kwargs)
    for batch in calibration_data:
        inp = batch[0] if isinstance(batch, (tuple, list)) else batch
        q.add_batch(inp)
    return q.fasterquant() if canonical else q.quantize()


__all__ = ["GPTQ", "GPTQMultiGPU", "quantize_layer_gptq"]
