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
positive-definiteness check at the end.  Each Hessian's chain (damping +
factorisation, then the sweeps of the layers sharing it) is independent of
the others, and every one of them is a sequence of latency-bound launches, so
the chains run on separate streams (at most ``streams``; one stream per chain
of the same device) and overlap on the GPU.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple, Union

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
    perm: Optional[torch.Tensor] = None  # (K,) int32 sweep order with act-order, else None


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


_SIDE_STREAMS: Dict[int, list] = {}


def side_streams(device: torch.device, n: int) -> list:
    """``n`` reusable streams of the default priority on ``device``.  HIP maps
    streams onto GPU_MAX_HW_QUEUES hardware queues (4 by default), so the
    caller's stream plus more than three side streams put two streams on one
    queue, whose work then runs one after the other."""
    idx = torch.device(device).index
    pool = _SIDE_STREAMS.setdefault(idx, [])
    while len(pool) < n:
        pool.append(torch.cuda.Stream(device=device))
    return pool[:n]


def _quantize_one(W, U, perm, dead, bits, group_size, blocksize, want_dequant) -> LayerResult:
    N, K = W.shape
    gs = group_size if 0 < group_size < K else (K if group_size > 0 else -1)
    scale = zero = None
    if gs <= 0:
        scale, zero = _ops.minmax_params(W.float(), bits, -1, 0)
    Wp = _ops.prepare_weight(W, perm=perm, dead=dead)
    # per-row sums of squared errors instead of the per-weight loss matrix:
    # sum(losses) = sum((w - q)^2 / d^2) / 2 = sum(err_sq) / 2
    res = _ops.quantize_sweep(Wp, U, bits, gs, blocksize, L.SWEEP_TRAILING, out_cols=perm,
                              dequant_dtype=W.dtype if want_dequant else None, scale=scale, zero=zero,
                              want_losses=False, want_err=True)
    del Wp
    ar = torch.arange(K, device=W.device, dtype=torch.int32)
    gcol = ar // gs if gs > 0 else torch.zeros_like(ar)
    if perm is None:
        g_idx = gcol
    else:
        g_idx = torch.empty_like(ar)
        g_idx[perm.long()] = gcol
    return LayerResult(codes=res["codes"], qweight=_ops.pack(res["codes"], bits), scale=res["scale"],
                       zero=res["zero"], g_idx=g_idx, dequant=res["dequant"], losses_sum=0.5 * res["err_sq"].sum(),
                       perm=perm)


class PendingLayers:
    """Layers being quantized on side streams; ``wait()`` orders the caller's
    current stream after them, checks positive-definiteness (one host sync)
    and returns the results."""

    def __init__(self, out, infos, streams, order, check):
        self._out, self._infos, self._streams, self._order, self._check = out, infos, streams, order, check

    def wait(self) -> Dict[str, LayerResult]:
        main = torch.cuda.current_stream(self._streams[0].device)
        for st in self._streams:
            main.wait_stream(st)
        if self._check:
            bad = torch.stack([i.reshape(()) for i in self._infos]).cpu()
            if bool((bad != 0).any()):
                raise torch.linalg.LinAlgError("a damped Hessian is not positive-definite")
        return {name: self._out[name] for name in self._order}


def quantize_layers_async(weights: Dict[str, torch.Tensor], hkeys: Dict[str, str],
                          hessians: Dict[str, Tuple[torch.Tensor, int]], bits: int = 4, group_size: int = 128,
                          blocksize: int = 128, percdamp: float = 0.01, actorder: bool = False,
                          want_dequant: bool = True, check: bool = True,
                          streams: Union[int, Sequence[torch.cuda.Stream]] = 3) -> PendingLayers:
    """Starts GPTQ (canonical) on every layer in ``weights`` (name -> (N, K)
    weight) with Hessian ``hessians[hkeys[name]]`` = (sum x x^T, nsamples):
    each Hessian's chain on one of ``streams`` (a count taken from a reusable
    pool, or explicit streams), after the work already enqueued on the
    caller's current stream.  Returns without waiting."""
    keys = list(dict.fromkeys(hkeys[n] for n in weights))
    dev = next(iter(weights.values())).device
    main = torch.cuda.current_stream(dev)
    # longest chains (largest K, then most rows) first, so they start first
    cost = {k: (hessians[k][0].shape[0], sum(weights[n].shape[0] for n in weights if hkeys[n] == k)) for k in keys}
    keys.sort(key=lambda k: cost[k], reverse=True)
    if isinstance(streams, int):
        pool = side_streams(dev, max(1, min(streams, len(keys))))
    else:
        pool = list(streams)
    for st in pool:
        st.wait_stream(main)
    infos = []
    out = {}
    for i, key in enumerate(keys):
        st = pool[i % len(pool)]
        with torch.cuda.stream(st):
            H, ns = hessians[key]
            U, perm, dead, info = factorize(H, ns, percdamp, actorder)
            infos.append(info)
            for name, W in weights.items():
                if hkeys[name] == key:
                    out[name] = _quantize_one(W, U, perm, dead, bits, group_size, blocksize, want_dequant)
    return PendingLayers(out, infos, pool, list(weights), check)


def quantize_layers(weights: Dict[str, torch.Tensor], hkeys: Dict[str, str],
                    hessians: Dict[str, Tuple[torch.Tensor, int]], bits: int = 4, group_size: int = 128,
                    blocksize: int = 128, percdamp: float = 0.01, actorder: bool = False,
                    want_dequant: bool = True, check: bool = True,
                    streams: Union[int, Sequence[torch.cuda.Stream]] = 3) -> Dict[str, LayerResult]:
    """GPTQ (canonical) on every layer in ``weights`` (name -> (N, K) weight),
    with Hessian ``hessians[hkeys[name]]`` = (sum x x^T, nsamples).  Results
    are ordered after the caller's current stream on return."""
    return quantize_layers_async(weights, hkeys, hessians, bits, group_size, blocksize, percdamp, actorder,
                                 want_dequant, check, streams).wait()
