"""Sequential single-GPU layer loop over the HIP kernels.

The reference quantizes the layers of a model one after another
(core/quantizer.py:133-155 -> coordinator.py:183-235 -> GPTQ.add_batch /
quantize), and its multi-GPU variant only spreads whole layers over devices
(core/gptq.py:311-341).  Here the loop runs on one GPU, and layers that see
the same input (q/k/v, gate/up) share one Hessian and one factorisation:
their Hessians are identical, so factorising once gives bit-identical
results.

``quantize_layers`` takes, per layer, its weight and a key naming its
Hessian; every device result stays on the GPU and the only host sync is the
positive-definiteness check at the end.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import _lib as L
from . import _ops


@dataclass
class LayerResult:
    codes: torch.Tensor        # (N, K) uint8, original column order
    qweight: torch.Tensor      # (N, ceil(K*bits/8)) uint8, native packed layout
    scale: torch.Tensor        # (N, ngroups) fp32, sweep (act-order) group order
    zero: torch.Tensor         # (N, ngroups) fp32
    g_idx: torch.Tensor        # (K,) int32: group of input column k
    dequant: Optional[torch.Tensor]  # (N, K) layer dtype
    losses_sum: torch.Tensor   # () fp32 device scalar


def factorize(H: torch.Tensor, nsamples: int, percdamp: float, actorder: bool):
    """Canonical damping + act-order + upper Cholesky factor of H^-1.
    Returns (U, perm or None, dead, info)."""
    scl = 2.0 / nsamples
    perm = None
    if actorder:
        d = torch.diagonal(H) * scl
        d = torch.where(d == 0, torch.ones_like(d), d)
        perm = torch.argsort(d, descending=True, stable=True).to(torch.int32)
    U, _, dead, info = _ops.damp_factor(H, scl, percdamp, perm, L.FACTOR_UPPER_CHOL_INV, want_dead=True)
    return U, perm, dead, info


def quantize_layers(weights: Dict[str, torch.Tensor], hkeys: Dict[str, str],
                    hessians: Dict[str, Tuple[torch.Tensor, int]], bits: int = 4, group_size: int = 128,
                    blocksize: int = 128, percdamp: float = 0.01, actorder: bool = False,
                    want_dequant: bool = True, check: bool = True) -> Dict[str, LayerResult]:
    """GPTQ (canonical) on every layer in ``weights`` (name -> (N, K) weight),
    with Hessian ``hessians[hkeys[name]]`` = (sum x x^T, nsamples)."""
    factors = {}
    infos = []
    for key in dict.fromkeys(hkeys[n] for n in weights):
        H, ns = hessians[key]
        factors[key] = factorize(H, ns, percdamp, actorder)
        infos.append(factors[key][3])
    out = {}
    for name, W in weights.items():
        U, perm, dead, _ = factors[hkeys[name]]
        N, K = W.shape
        gs = group_size if 0 < group_size < K else (K if group_size > 0 else -1)
        scale = zero = None
        if gs <= 0:
            scale, zero = _ops.minmax_params(W.float(), bits, -1, 0)
        Wp = _ops.prepare_weight(W, perm=perm, dead=dead)
        res = _ops.quantize_sweep(Wp, U, bits, gs, blocksize, L.SWEEP_TRAILING, out_cols=perm,
                                  dequant_dtype=W.dtype if want_dequant else None, scale=scale, zero=zero,
                                  want_losses=True, want_err=False)
        del Wp
        ar = torch.arange(K, device=W.device, dtype=torch.int32)
        gcol = ar // gs if gs > 0 else torch.zeros_like(ar)
        if perm is None:
            g_idx = gcol
        else:
            g_idx = torch.empty_like(ar)
            g_idx[perm.long()] = gcol
        out[name] = LayerResult(codes=res["codes"], qweight=_ops.pack(res["codes"], bits), scale=res["scale"],
                                zero=res["zero"], g_idx=g_idx, dequant=res["dequant"],
                                losses_sum=res["losses"].sum())
    if check:
        bad = torch.stack([i.reshape(()) for i in infos]).cpu()
        if bool((bad != 0).any()):
            raise torch.linalg.LinAlgError("a damped Hessian is not positive-definite")
    return out
