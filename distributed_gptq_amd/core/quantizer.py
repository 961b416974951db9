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

import logging
import time
from dataclasses import asdict, dataclass
from enum import Enum
from typing import Any, Callable, Dict, List, Optional, Tuple, Union

import torch
import torch.nn as nn

from .. import _lib as L
from .. import _ops

logger = logging.getLogger(__name__)


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
    # quantize block by block, and the layer groups of a block one after
    # another, each calibrated on the quantized predecessors' outputs (the
    # reference CLI's --true-sequential, cli.py:207-211, which its config
    # lacks)
    true_sequential: bool = False

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


# ------------------------------------------------- process configuration --

class QuantizationMode(Enum):
    """Processing modes (distributed/coordinator.py:21-26).  This build runs
    one process on one GPU: only SINGLE_GPU is accepted by the driver."""
    SINGLE_GPU = "single_gpu"
    DATA_PARALLEL = "data_parallel"
    MODEL_PARALLEL = "model_parallel"
    PIPELINE_PARALLEL = "pipeline_parallel"


@dataclass
class DistributedConfig:
    """Process configuration (distributed/coordinator.py:29-47), accepted by
    DistributedGPTQuantizer; world_size must be 1 here."""
    mode: QuantizationMode = QuantizationMode.SINGLE_GPU
    world_size: int = 1
    rank: int = 0
    local_rank: int = 0
    master_addr: str = "localhost"
    master_port: str = "12355"
    backend: str = "nccl"
    init_timeout: int = 1800

    @property
    def is_distributed(self) -> bool:
        return self.world_size > 1

    @property
    def is_main_process(self) -> bool:
        return self.rank == 0


def create_distributed_config(mode: Union[str, QuantizationMode] = "auto") -> DistributedConfig:
    """From the launcher's environment (WORLD_SIZE, RANK, LOCAL_RANK,
    MASTER_ADDR, MASTER_PORT), as distributed/coordinator.py:264-301."""
    import os
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if mode == "auto":
        mode = QuantizationMode.SINGLE_GPU if world == 1 else QuantizationMode.DATA_PARALLEL
    elif isinstance(mode, str):
        mode = QuantizationMode(mode)
    return DistributedConfig(mode=mode, world_size=world, rank=int(os.environ.get("RANK", "0")),
                             local_rank=int(os.environ.get("LOCAL_RANK", "0")),
                             master_addr=os.environ.get("MASTER_ADDR", "localhost"),
                             master_port=os.environ.get("MASTER_PORT", "12355"))


# ------------------------------------------------------------- driver --

class _HookError(RuntimeError):
    """A failure inside the Hessian hooks (never skipped like a failing
    calibration batch)."""


class _StopForward(Exception):
    """Ends a calibration forward early: once the first block's inputs are
    taken, or once the last layer a pass calibrates has run."""


def _find_blocks(model: nn.Module, layers: Dict[str, nn.Linear]):
    """(name, ModuleList) of the module list whose entries hold the most of
    ``layers`` (a transformer's decoder blocks), or None."""
    best, best_n = None, 0
    for name, mod in model.named_modules():
        if isinstance(mod, nn.ModuleList) and len(mod) > 0 and name:
            n = sum(1 for k in layers if k.startswith(name + "."))
            if n > best_n:
                best, best_n = (name, mod), n
    return best


class _SharedHessians:
    """Hessians of a calibration pass, one per group of layers that received
    the same input tensor in every batch so far (q/k/v, gate/up).

    Every layer starts alone.  A layer with no samples yet joins a group
    that also had none before this batch and has been given the same tensor,
    and nothing else, in it (both Hessians are then that tensor's X^T X).
    A group of several layers
    adds its input once every member has seen the batch: members whose input
    differs from the first member's leave the group with a copy of the
    group's Hessian as it was before this batch (exact: nothing of this batch
    has been added yet), and each distinct input is added once.  Inputs are
    compared by storage, offset, shape, stride, dtype and version counter
    (inference tensors, which have none: and by value against a clone);
    a group's pending inputs are kept referenced (so a reused allocation
    cannot pass for the same input) and cloned (so an in-place change after
    the first member's call is seen as a different input, not lost).  With
    ``share=False`` every layer keeps its own Hessian."""

    def __init__(self, layers: Dict[str, nn.Linear], device: torch.device, share: bool, make_acc=None):
        if make_acc is None:
            from .gptq import GPTQ

            def make_acc(layer):
                return GPTQ(layer, device=device, token_buffer=0)
        # make_acc(layer) -> an object with add_batch(x), the H property,
        # nsamples and free(): the GPTQ class, or a stand-in in tests
        self._make_acc = make_acc
        self.layers, self.device, self.share = layers, device, share
        self.group_of: Dict[str, int] = {}
        self.members: Dict[int, List[str]] = {}
        self.acc: Dict[int, Any] = {}
        for name in layers:
            self._new_group([name], None)
        # this batch: group -> {key: (input, clone, members)} still to settle,
        # and key -> (group, input) for groups that had no samples before it
        self.pending: Dict[int, Dict[tuple, Tuple[torch.Tensor, torch.Tensor, List[str]]]] = {}
        self.fresh: Dict[tuple, Tuple[int, torch.Tensor]] = {}
        self.fresh_key: Dict[int, tuple] = {}

    def _new_group(self, names: List[str], copy_from) -> int:
        gid = len(self.acc)
        q = self._make_acc(self.layers[names[0]])
        if copy_from is not None and copy_from.nsamples:
            q.H = copy_from.H.clone()
            q.nsamples = copy_from.nsamples
        self.acc[gid], self.members[gid] = q, list(names)
        for n in names:
            self.group_of[n] = gid
        return gid

    @staticmethod
    def _key(x: torch.Tensor) -> tuple:
        # inference tensors (torch.inference_mode) have no version counter:
        # an in-place change between two layers is then found by comparing
        # values with a clone (_same)
        return (x.untyped_storage().data_ptr(), x.storage_offset(), tuple(x.shape), tuple(x.stride()), x.dtype,
                None if x.is_inference() else x._version)

    @staticmethod
    def _same(x: torch.Tensor, seen: torch.Tensor) -> bool:
        """x has the key of ``seen`` (a clone taken at the earlier call):
        the same tensor, unchanged, unless an inference tensor changed in
        place (one comparison on the device)."""
        return not x.is_inference() or bool(torch.equal(x, seen))

    def add(self, name: str, x: torch.Tensor) -> None:
        gid = self.group_of[name]
        if not self.share:
            self.acc[gid].add_batch(x)
            return
        key = self._key(x)
        if len(self.members[gid]) == 1:
            acc = self.acc[gid]
            if acc.nsamples == 0:
                hit = self.fresh.get(key)
                if hit is not None and hit[0] != gid and self._same(x, hit[1]):
                    g = hit[0]
                    self.members[g].append(name)
                    self.group_of[name] = g
                    self.members[gid] = []
                    return
                self.fresh[key] = (gid, x.clone() if x.is_inference() else x)
                self.fresh_key[gid] = key
            else:
                # a second tensor for this group in this batch: its Hessian is
                # no longer that of the tensor it was registered under, so no
                # later layer may join it
                k0 = self.fresh_key.pop(gid, None)
                if k0 is not None:
                    self.fresh.pop(k0, None)
            acc.add_batch(x)
            return
        if any(name in names for _, _, names in self.pending.get(gid, {}).values()):
            # a layer called twice in one forward: settle what the group has
            # seen so far (members not yet called split off), then go on
            self._settle(gid)
            self.add(name, x)
            return
        part = self.pending.setdefault(gid, {})
        while key in part and not self._same(x, part[key][1]):
            key = key + ("changed",)  # an inference tensor changed in place since
        if key not in part:
            part[key] = (x, x.clone(), [])
        part[key][2].append(name)
        if sum(len(v[2]) for v in part.values()) == len(self.members[gid]):
            self._settle(gid)

    def _settle(self, gid: int) -> None:
        part = list(self.pending.pop(gid).values())
        fired = {n for _, _, names in part for n in names}
        idle = [n for n in self.members[gid] if n not in fired]
        acc = self.acc[gid]
        # split before adding anything of this batch, so the copies are exact
        moved = [(self._new_group(names, acc), xc) for _, xc, names in part[1:]]
        if idle:
            self._new_group(idle, acc)
        self.members[gid] = list(part[0][2])
        for g, xc in [(gid, part[0][1])] + moved:
            self.acc[g].add_batch(xc)

    def end_batch(self) -> None:
        for gid in list(self.pending):
            self._settle(gid)
        self.fresh.clear()
        self.fresh_key.clear()

    def groups(self) -> Dict[int, List[str]]:
        return {g: list(m) for g, m in self.members.items() if m}


class DistributedGPTQuantizer:
    """Model-level GPTQ driver (core/quantizer.py:52-356) on one GPU.

    ``quantize_model`` finds the nn.Linear layers (:167-179), runs the
    calibration forward with hooks (:194-246) and quantizes every layer with
    canonical GPTQ (:129-151).  The reference stores every layer input on the
    host (``.cpu()``, :210) and later runs each layer again per batch to feed
    ``add_batch`` (distributed/coordinator.py:213-218); here the hooks feed
    each input straight into the Hessian kernel, and layers fed the same
    tensor share one Hessian and one factorisation (bit-identical results,
    less work).  Layers are quantized a few Hessian groups at a time on side
    streams (``pipeline.quantize_layers``).

    With ``quantization_config.save_packed`` (the default) each quantized
    layer is replaced by a QuantizedLinear holding its packed codes, the form
    the W4A16/W3A16 kernels serve; otherwise the nn.Linear keeps the
    dequantized weights.  Divergences: nn.Conv2d layers are not quantized;
    a list of calibration tensors is iterated one tensor per batch (the
    reference wraps it in ``TensorDataset(*data)``, :185-192, which yields
    only the first tensor's rows); ``distributed_config`` with more than one
    process is refused.
    """

    def __init__(self, quantization_config: Optional[QuantizationConfig] = None, distributed_config=None,
                 device: Optional[Union[str, torch.device]] = None, share_hessians: bool = True,
                 groups_per_step: int = 4):
        self.quant_config = quantization_config or QuantizationConfig()
        self.quant_config.validate()
        world = getattr(distributed_config, "world_size", 1) if distributed_config is not None else 1
        if world > 1:
            raise NotImplementedError("this build quantizes on one GPU per process (world_size must be 1)")
        self.dist_config = distributed_config
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device()
                                                                                  if torch.cuda.is_available() else 0)
        self.share_hessians = share_hessians
        self.groups_per_step = max(1, int(groups_per_step))
        self.quantized_layers: Dict[str, Dict[str, Any]] = {}
        self.quantization_errors: Dict[str, float] = {}

    @property
    def config(self) -> QuantizationConfig:
        return self.quant_config

    # ------------------------------------------------------------ layers --
    def _find_layers_to_quantize(self, model: nn.Module) -> Dict[str, nn.Linear]:
        """nn.Linear layers with more than 1000 weights (:167-179)."""
        return {n: m for n, m in model.named_modules() if isinstance(m, nn.Linear) and m.weight.numel() > 1000}

    def _get_quantizable_layers(self, model: nn.Module) -> List[Tuple[str, nn.Linear]]:
        return list(self._find_layers_to_quantize(model).items())

    def _resolve_layers(self, model, layers_to_quantize) -> Dict[str, nn.Linear]:
        if layers_to_quantize is None:
            return self._find_layers_to_quantize(model)
        mods = dict(model.named_modules())
        if isinstance(layers_to_quantize, dict):
            layers = dict(layers_to_quantize)
        else:
            missing = [n for n in layers_to_quantize if n not in mods]
            if missing:
                raise ValueError(f"no such modules in the model: {missing}")
            layers = {n: mods[n] for n in layers_to_quantize}
        bad = [n for n, m in layers.items() if not isinstance(m, nn.Linear)]
        if bad:
            raise NotImplementedError(f"only nn.Linear layers are quantized here, not {bad}")
        return layers

    # ------------------------------------------------------- calibration --
    @staticmethod
    def _inputs(batch):
        if isinstance(batch, (list, tuple)):
            batch = batch[0]
        return batch

    def _model_batches(self, model: nn.Module, calibration_data):
        """Runs the calibration forwards of the whole model, at most
        ``calibration_samples`` rows; yields once per batch (True if it ran,
        False if it failed and was skipped, as the reference does, :232-236)."""
        seen = 0
        for batch in calibration_data:
            if seen >= self.quant_config.calibration_samples:
                break
            b = self._inputs(batch)
            try:
                if isinstance(b, dict):
                    b = {k: v.to(self.device) if torch.is_tensor(v) else v for k, v in b.items()}
                    rows = next(v for v in b.values() if torch.is_tensor(v)).shape[0]
                    model(**b)
                else:
                    b = b.to(self.device)
                    rows = b.shape[0]
                    model(b)
                ok = True
            except _HookError:
                raise
            except _StopForward:  # the first block's inputs are taken
                rows = (b if torch.is_tensor(b) else next(v for v in b.values() if torch.is_tensor(v))).shape[0]
                ok = True
            except Exception as e:  # noqa: BLE001
                logger.warning("error during calibration forward, batch skipped: %s", e)
                rows, ok = 0, False
            seen += rows
            yield ok

    @torch.no_grad()
    def _collect_hessians(self, model: nn.Module, calibration_data, layers: Dict[str, nn.Linear],
                          batches=None, stop_after: bool = False) -> _SharedHessians:
        """Calibration forward (:194-246) with the Hessians accumulated in the
        hooks.  ``batches`` (an iterator that runs one forward per step and
        yields whether it ran) defaults to the whole model over
        ``calibration_data``; with ``stop_after`` each forward ends (by
        _StopForward, which ``batches`` catches) once every layer has run."""
        hs = _SharedHessians(layers, self.device, self.share_hessians)
        self._call_order: List[str] = []

        def hook_for(name):
            def hook(module, inp, out):
                x = inp[0] if isinstance(inp, tuple) else inp
                if name not in self._call_order:
                    self._call_order.append(name)
                try:
                    hs.add(name, x.detach())
                except Exception as e:
                    raise _HookError(f"Hessian accumulation for {name}: {e}") from e
            return hook

        handles = [m.register_forward_hook(hook_for(n)) for n, m in layers.items()]
        if stop_after:
            handles += self._stop_hooks(layers)
        it = batches if batches is not None else self._model_batches(model, calibration_data)
        ok = 0
        try:
            while True:
                try:
                    ran = next(it)
                except StopIteration:
                    break
                finally:
                    hs.end_batch()
                ok += int(ran)
        finally:
            for h in handles:
                h.remove()
        if ok == 0:
            raise ValueError("no calibration batch ran through the model")
        return hs

    # ---------------------------------------------------------- quantize --
    def _quantize_groups(self, model, hs: _SharedHessians, gids: List[int], layers: Dict[str, nn.Linear],
                         progress: Optional[Callable], counter: List[int]) -> None:
        """GPTQ on the layers of Hessian groups ``gids`` (largest Hessians
        first, a few groups per step), each replaced by a QuantizedLinear
        (``save_packed``) or given its dequantized weights."""
        from .. import pipeline
        from ..models.layers import QuantizedLinear
        cfg = self.quant_config
        groups = hs.groups()
        for g in gids:
            if hs.acc[g].nsamples == 0:
                raise ValueError(f"layers {groups[g]} received no calibration input")
        order = sorted(gids, key=lambda g: -layers[groups[g][0]].in_features)
        parents = dict(model.named_modules())
        for i in range(0, len(order), self.groups_per_step):
            step = order[i:i + self.groups_per_step]
            weights = {n: layers[n].weight.data for g in step for n in groups[g]}
            hkeys = {n: str(g) for g in step for n in groups[g]}
            hess = {str(g): (hs.acc[g].H, hs.acc[g].nsamples) for g in step}
            res = pipeline.quantize_layers(weights, hkeys, hess, bits=cfg.bits, group_size=cfg.group_size,
                                           blocksize=cfg.blocksize, percdamp=cfg.percdamp, actorder=cfg.actorder,
                                           want_dequant=not cfg.save_packed)
            for g in step:
                hs.acc[g].free()
            for g in step:
                for n in groups[g]:
                    r, lin = res[n], layers[n]
                    if cfg.save_packed:
                        K = lin.in_features
                        gs = K if cfg.group_size <= 0 or cfg.group_size > K else cfg.group_size
                        q = QuantizedLinear(cfg.bits, gs, K, lin.out_features, bias=lin.bias is not None,
                                            packed=True).to(lin.weight.device)
                        q.pack_weights(r.codes, r.scale, r.zero, r.g_idx, perm=r.perm)
                        if lin.bias is not None:
                            q.bias.data = lin.bias.data.clone()
                        parent_name, _, attr = n.rpartition(".")
                        setattr(parents[parent_name] if parent_name else model, attr, q)
                    else:
                        lin.weight.data.copy_(r.dequant)
                    err = float(r.losses_sum)
                    stats = {"total_error": err, "bits": cfg.bits, "group_size": cfg.group_size,
                             "nsamples": hs.acc[g].nsamples, "hessian_shared_with": [m for m in groups[g] if m != n]}
                    self.quantized_layers[n] = stats
                    self.quantization_errors[n] = err
                    counter[0] += 1
                    if progress is not None:
                        progress(counter[0], counter[1], n, stats)
            del res

    def quantize_model(self, model: nn.Module, calibration_data, layers_to_quantize=None,
                       save_path: Optional[str] = None, progress_callback: Optional[Callable] = None,
                       blockwise: Optional[bool] = None) -> nn.Module:
        """core/quantizer.py:79-165: calibrate, quantize every layer, optionally
        save.  ``progress_callback(done, total, name, stats)`` after each
        layer.

        By default, as the reference: one calibration pass over the
        unquantized model gives every layer's Hessian.  With ``blockwise``
        (or ``quantization_config.true_sequential``, the reference CLI's
        --true-sequential, cli.py:207-211) the decoder blocks (the model's
        largest nn.ModuleList holding the layers) are quantized one at a
        time, each calibrated on the previous quantized blocks' outputs, and
        only one block's Hessians are held; with ``true_sequential`` the
        layer groups inside a block (those fed the same input: q/k/v, then
        o, gate/up, down) are also calibrated one after another on the
        outputs of the groups already quantized."""
        L.require_gpu()
        t0 = time.time()
        model.eval()
        layers = self._resolve_layers(model, layers_to_quantize)
        if not layers:
            return model
        for n, m in layers.items():
            if m.weight.device.type != "cuda":
                raise ValueError(f"layer {n} is on {m.weight.device}; move the model to the GPU first")
        logger.info("found %d layers to quantize", len(layers))
        counter = [0, len(layers)]
        seq = self.quant_config.true_sequential
        blocks = _find_blocks(model, layers) if (blockwise or seq) else None
        if (blockwise or seq) and blocks is None:
            logger.warning("no block list holding the layers was found: one calibration pass for all layers")
        if blocks is None:
            hs = self._collect_hessians(model, calibration_data, layers)
            self._quantize_groups(model, hs, list(hs.groups()), layers, progress_callback, counter)
        else:
            self._quantize_blockwise(model, calibration_data, layers, blocks, seq, progress_callback, counter)
        self._log_quantization_summary(time.time() - t0)
        if save_path:
            self.save_quantized_model(model, save_path)
        return model

    @torch.no_grad()
    def _quantize_blockwise(self, model, calibration_data, layers, blocks, true_sequential, progress, counter):
        prefix, mods = blocks
        inputs = self._capture_block_inputs(model, calibration_data, mods[0])
        if not inputs:
            raise ValueError("no calibration batch reached the first block")
        cfg_model = getattr(model, "config", None)
        # true sequential: the layer groups of a block in forward order, as
        # name suffixes, learnt from the first full pass over a block
        plan: Optional[List[List[str]]] = None
        for i, block in enumerate(mods):
            pre = f"{prefix}.{i}."
            mine = {n: m for n, m in layers.items() if n.startswith(pre)}
            step = 0
            while mine:
                # a planned group is calibrated alone: hooks on its layers only,
                # and the block's forward stops after the last of them has run
                want = None
                if true_sequential and plan is not None and step < len(plan):
                    names = [pre + sfx for sfx in plan[step]]
                    if all(n in mine for n in names):
                        want = {n: mine[n] for n in names}

                def batches(block=block):
                    for args, kwargs in inputs:
                        try:
                            block(*args, **kwargs)
                        except _StopForward:
                            pass
                        yield True
                hs = self._collect_hessians(model, None, want if want is not None else mine, batches=batches(),
                                            stop_after=want is not None)
                groups = hs.groups()
                if true_sequential:
                    # the group of the first layer the forward reached; the
                    # other Hessians saw unquantized predecessors: dropped
                    first = next(n for n in self._call_order if n in mine)
                    gids = [next(g for g, m in groups.items() if first in m)]
                    if want is None and step == 0 and plan is None:
                        plan = self._group_plan(groups, pre)
                else:
                    gids = list(groups)
                self._quantize_groups(model, hs, gids, mine, progress, counter)
                done = {n for g in gids for n in groups[g]}
                for g in groups:
                    hs.acc[g].free()
                mine = {n: m for n, m in mine.items() if n not in done}
                step += 1
            # this block's outputs (its layers now quantized) feed the next
            for j, (args, kwargs) in enumerate(inputs):
                out = block(*args, **kwargs)
                h = out[0] if isinstance(out, (tuple, list)) else out
                inputs[j] = ((h,) + tuple(args[1:]), kwargs)
        rest = {n: m for n, m in layers.items() if not n.startswith(prefix + ".")}
        if rest:
            # layers outside the blocks (e.g. a head): one pass over the model,
            # whose blocks are quantized now
            hs = self._collect_hessians(model, calibration_data, rest)
            self._quantize_groups(model, hs, list(hs.groups()), rest, progress, counter)
        del cfg_model

    def _group_plan(self, groups, pre: str) -> Optional[List[List[str]]]:
        """The Hessian groups of a block's first pass in the order the forward
        reached them, as name suffixes (None if a layer ran twice or a group
        was never reached)."""
        order = {n: k for k, n in enumerate(self._call_order)}
        if any(n not in order for m in groups.values() for n in m):
            return None
        ranked = sorted(groups.values(), key=lambda m: min(order[n] for n in m))
        return [[n[len(pre):] for n in sorted(m, key=lambda n: order[n])] for m in ranked]

    @staticmethod
    def _stop_hooks(layers: Dict[str, nn.Linear]) -> list:
        """Forward hooks that end a forward once every layer of ``layers`` has
        run in it (registered after the Hessian hooks, so they run after the
        last of them)."""
        left, seen = set(layers), set()

        def make(name):
            def hook(module, inp, out):
                seen.add(name)
                if seen >= left:
                    seen.clear()
                    raise _StopForward
            return hook
        return [m.register_forward_hook(make(n)) for n, m in layers.items()]

    def _capture_block_inputs(self, model, calibration_data, first_block) -> List[Tuple[tuple, dict]]:
        """(args, kwargs) of the first block's call in each calibration
        forward; the forward stops there.  The model's KV cache is turned off
        meanwhile (a block is run several times on the same inputs)."""
        inputs: List[Tuple[tuple, dict]] = []

        def grab(module, args, kwargs):
            kw = {k: v for k, v in kwargs.items() if k not in ("past_key_value", "past_key_values")}
            if "use_cache" in kw:
                kw["use_cache"] = False
            inputs.append((tuple(args), kw))
            raise _StopForward

        cfg = getattr(model, "config", None)
        saved = getattr(cfg, "use_cache", None)
        if saved is not None:
            cfg.use_cache = False
        h = first_block.register_forward_pre_hook(grab, with_kwargs=True)
        try:
            for _ in self._model_batches(model, calibration_data):
                pass
        finally:
            h.remove()
            if saved is not None:
                cfg.use_cache = saved
        if inputs and not torch.is_tensor(inputs[0][0][0] if inputs[0][0] else None):
            # hidden states passed by keyword
            fixed = []
            for args, kw in inputs:
                hs = kw.pop("hidden_states")
                fixed.append(((hs,) + tuple(args), kw))
            inputs = fixed
        return inputs

    def _log_quantization_summary(self, elapsed_time: float) -> None:
        total = sum(self.quantization_errors.values())
        n = len(self.quantization_errors)
        logger.info("quantized %d layers in %.2f s, total error %.6g, average %.6g", n, elapsed_time, total,
                    total / n if n else 0.0)

    # ------------------------------------------------------- save / load --
    def save_quantized_model(self, model: nn.Module, save_path: str, save_format: str = "safetensors") -> None:
        """core/quantizer.py:248-291."""
        from .checkpoint import save_quantized_model
        save_quantized_model(model, save_path, save_format, quant_config=self.quant_config,
                             quantization_errors=self.quantization_errors,
                             quantized_layers=list(self.quantized_layers))

    def load_quantized_model(self, model: nn.Module, load_path: str, load_format: str = "safetensors") -> nn.Module:
        """core/quantizer.py:293-335: restores the config, layer list and
        errors along with the weights."""
        from .checkpoint import load_quantized_model
        model, meta = load_quantized_model(model, load_path, load_format, return_metadata=True)
        self.quant_config = meta["quant_config"]
        self.quantized_layers = {n: {} for n in meta["quantized_layers"]}
        self.quantization_errors = meta["quantization_errors"]
        return model


def quantize_model_simple(model: nn.Module, calibration_data, bits: int = 4,
                          save_path: Optional[str] = None) -> nn.Module:
    """core/quantizer.py:358-383."""
    return DistributedGPTQuantizer(QuantizationConfig(bits=bits)).quantize_model(model, calibration_data,
                                                                               save_path=save_path)
