"""Quantized-model checkpoints: a safetensors state dict plus a JSON sidecar.

Format (src/distributed_gptq/core/quantizer.py:248-291):

* ``save_format="safetensors"``: the model's ``state_dict()`` written with
  safetensors at ``save_path``; beside it ``save_path.with_suffix('.json')``
  holds ``quantization_config`` (the config's fields), ``quantized_layers``
  (module names) and ``quantization_errors`` (name -> loss) (:265-280).
* ``save_format="pytorch"``: one ``torch.save`` dict with the same three keys
  and ``model_state_dict`` (:284-291).

This module adds one key, ``layers`` (name -> bits, group_size, packed,
in/out features, bias), so that loading does not depend on the model already
holding QuantizedLinear modules.  The reference loads with a strict
``load_state_dict`` (:319-320), which needs every quantized layer of ``model``
to be a QuantizedLinear of the right shape already; here each name in
``quantized_layers`` that is still an ``nn.Linear`` is first replaced by a
QuantizedLinear whose buffers take the saved shapes and dtypes. Quantized
layers saved as ``nn.Linear`` (dequantized weights, the reference's in-place
result) have no ``layers`` entry and load as they are. A file without
``layers`` (the reference's own) is read by inferring the layout from the
buffer shapes and ``quantization_config.bits``.

Tensors are stored as they are: packed uint8 codes, fp16 scales and zeros,
int32 g_idx and the bias all round-trip bit-exactly.  Act-order layers are
written in the reference's column order (QuantizedLinear's state dict holds
the codes in input-column order and no ``perm``); loading re-derives the
serving order from g_idx.  Files from the earlier format with a ``perm`` key
(codes in that stored order) still load. Loading uses only
loaders that execute nothing from the file: safetensors, and ``torch.load``
with ``weights_only=True`` for the pytorch format. The reference writes only
on rank 0 (:281-283, :288-290); this module runs in one process and always
writes.
"""
from __future__ import annotations

import json
import math
from dataclasses import asdict
from pathlib import Path
from typing import Dict, Iterable, Optional, Union

import torch
import torch.nn as nn

from ..models.layers import QuantizedLinear
from .quantizer import QuantizationConfig

_FORMATS = ("safetensors", "pytorch")
_BUFFERS = ("qweight", "scales", "zeros", "g_idx")


def _quantized_modules(model: nn.Module) -> Dict[str, QuantizedLinear]:
    return {n: m for n, m in model.named_modules() if isinstance(m, QuantizedLinear)}


def _layer_info(m: QuantizedLinear) -> dict:
    return {"bits": int(m.bits), "group_size": int(m.group_size), "packed": bool(m.packed),
            "in_features": int(m.in_features), "out_features": int(m.out_features), "bias": m.bias is not None}


# the reference's QuantizationConfig fields (core/quantizer.py:27-34): the
# sidecar holds exactly these, so the reference's loader can read it
_REF_CONFIG_KEYS = ("bits", "group_size", "actorder", "percdamp", "blocksize", "calibration_samples", "use_triton",
                    "save_packed")


def _config_dict(config: Union[QuantizationConfig, dict, None], qmods: Dict[str, QuantizedLinear]) -> dict:
    if isinstance(config, QuantizationConfig):
        d = asdict(config)
    elif isinstance(config, dict):
        d = asdict(QuantizationConfig(**config))
    else:
        first = next(iter(qmods.values()), None)
        d = asdict(QuantizationConfig() if first is None else
                   QuantizationConfig(bits=first.bits, group_size=first.group_size))
    return {k: d[k] for k in _REF_CONFIG_KEYS}


def _cpu_state(model: nn.Module) -> Dict[str, torch.Tensor]:
    # one contiguous CPU copy per key: safetensors refuses strided views and
    # tensors that share storage (tied weights)
    return {k: v.detach().to("cpu", copy=True).contiguous() for k, v in model.state_dict().items()}


def save_quantized_model(model: nn.Module, save_path: Union[str, Path], save_format: str = "safetensors",
                         quant_config: Union[QuantizationConfig, dict, None] = None,
                         quantization_errors: Optional[Dict[str, float]] = None,
                         quantized_layers: Optional[Iterable[str]] = None) -> None:
    """Write ``model`` (core/quantizer.py:248-291).

    ``quantized_layers`` defaults to every QuantizedLinear in ``model``;
    ``quant_config`` to the bits and group size of the first of them.
    """
    if save_format not in _FORMATS:
        raise ValueError(f"save_format must be one of {_FORMATS}, got {save_format!r}")
    save_path = Path(save_path)
    save_path.parent.mkdir(parents=True, exist_ok=True)
    qmods = _quantized_modules(model)
    names = list(quantized_layers) if quantized_layers is not None else list(qmods)
    mods = dict(model.named_modules())
    bad = [n for n in names if not isinstance(mods.get(n), (QuantizedLinear, nn.Linear))]
    if bad:
        raise ValueError(f"neither QuantizedLinear nor nn.Linear modules of the model: {bad}")
    meta = {
        "quantization_config": _config_dict(quant_config, qmods),
        "quantized_layers": names,
        "quantization_errors": {k: float(v) for k, v in (quantization_errors or {}).items()},
        # layers kept as nn.Linear (holding dequantized weights) need no layout
        "layers": {n: _layer_info(qmods[n]) for n in names if n in qmods},
    }
    state = _cpu_state(model)
    if save_format == "safetensors":
        from safetensors.torch import save_file
        with open(save_path.with_suffix(".json"), "w") as f:
            json.dump(meta, f, indent=2)
        save_file(state, str(save_path))
    else:
        torch.save({**meta, "model_state_dict": state}, save_path)


def _infer_info(name: str, state: Dict[str, torch.Tensor], config: QuantizationConfig) -> dict:
    """Layout of a layer from its buffers, for sidecars without ``layers``."""
    try:
        qw, sc, gi = state[f"{name}.qweight"], state[f"{name}.scales"], state[f"{name}.g_idx"]
    except KeyError as e:
        raise ValueError(f"checkpoint has no buffers for quantized layer {name!r}: {e}") from None
    N, K, bits = qw.shape[0], gi.shape[0], config.bits
    # 4-bit rows are always packed (two codes a byte); other widths are packed
    # exactly when a row is narrower than K bytes (8-bit rows are K either way)
    packed = bits == 4 or qw.shape[1] != K
    gs = config.group_size if config.group_size > 0 else K
    if sc.shape[1] != math.ceil(K / gs):
        raise ValueError(f"{name}: {sc.shape[1]} scale groups do not match K={K}, group_size={gs}")
    return {"bits": bits, "group_size": gs, "packed": packed, "in_features": K, "out_features": N,
            "bias": f"{name}.bias" in state}


def _row_bytes(info: dict) -> int:
    K, bits = info["in_features"], info["bits"]
    return (K * bits + 7) // 8 if (info["packed"] or bits == 4) else K


def _layout(info: dict) -> tuple:
    return (info["bits"], info["group_size"], info["in_features"], info["out_features"], bool(info["bias"]),
            _row_bytes(info))


def _check_buffers(name: str, info: dict, state: Dict[str, torch.Tensor]) -> None:
    N, K, gs = info["out_features"], info["in_features"], info["group_size"]
    want = {"qweight": (N, _row_bytes(info)), "scales": (N, math.ceil(K / gs)),
            "zeros": (N, math.ceil(K / gs)), "g_idx": (K,)}
    for key, shape in want.items():
        t = state.get(f"{name}.{key}")
        if t is None:
            raise ValueError(f"checkpoint has no {name}.{key}")
        if tuple(t.shape) != shape:
            raise ValueError(f"{name}.{key}: saved shape {tuple(t.shape)}, layout wants {shape}")
    if info["bias"] != (f"{name}.bias" in state):
        raise ValueError(f"{name}: bias presence differs between the sidecar and the state dict")
    perm = state.get(f"{name}.perm")
    if perm is not None and tuple(perm.shape) not in ((0,), (K,)):
        raise ValueError(f"{name}.perm: saved shape {tuple(perm.shape)}, expected (0,) or ({K},)")


def _install(model: nn.Module, name: str, info: dict, state: Dict[str, torch.Tensor]) -> None:
    """Put a QuantizedLinear of the saved layout at ``name``, its buffers
    shaped and typed like the saved tensors (load_state_dict then copies the
    values without conversion)."""
    parts = name.split(".")
    parent = model
    for p in parts[:-1]:
        parent = getattr(parent, p)
    old = getattr(parent, parts[-1])
    K, N = info["in_features"], info["out_features"]
    if isinstance(old, QuantizedLinear):
        if _layout(_layer_info(old)) != _layout(info):
            raise ValueError(f"{name}: model layer {_layer_info(old)} differs from the saved layout {info}")
        q, device = old, old.qweight.device
    elif isinstance(old, nn.Linear):
        if (old.in_features, old.out_features) != (K, N) or (old.bias is not None) != info["bias"]:
            raise ValueError(f"{name}: nn.Linear({old.in_features}, {old.out_features}, bias="
                             f"{old.bias is not None}) does not match the saved layer ({K}, {N}, bias={info['bias']})")
        device = old.weight.device
        q = QuantizedLinear(info["bits"], info["group_size"], K, N, bias=info["bias"], packed=info["packed"]).to(device)
        setattr(parent, parts[-1], q)
    else:
        raise TypeError(f"{name}: expected nn.Linear or QuantizedLinear, found {type(old).__name__}")
    extra = ("bias",) if info["bias"] else ()
    for key in _BUFFERS + extra:
        t = state[f"{name}.{key}"]
        getattr(q, key).data = torch.empty(t.shape, dtype=t.dtype, device=device)


def load_quantized_model(model: nn.Module, load_path: Union[str, Path], load_format: str = "safetensors",
                         return_metadata: bool = False):
    """Load a checkpoint written by :func:`save_quantized_model` or by the
    reference (core/quantizer.py:293-335) into ``model``, quantized or not.

    Returns ``model`` (with ``return_metadata``: ``(model, metadata)``, where
    metadata holds ``quant_config`` (a QuantizationConfig),
    ``quantized_layers`` and ``quantization_errors``, the reference's
    attributes after loading, :322-324).
    """
    if load_format not in _FORMATS:
        raise ValueError(f"load_format must be one of {_FORMATS}, got {load_format!r}")
    load_path = Path(load_path)
    if load_format == "safetensors":
        from safetensors.torch import load_file
        with open(load_path.with_suffix(".json")) as f:
            meta = json.load(f)
        state = load_file(str(load_path))
    else:
        ckpt = torch.load(load_path, map_location="cpu", weights_only=True)
        state = ckpt["model_state_dict"]
        meta = {k: v for k, v in ckpt.items() if k != "model_state_dict"}
    config = QuantizationConfig(**meta["quantization_config"])
    layers = meta.get("layers") or {}
    for name in meta["quantized_layers"]:
        if name not in layers and f"{name}.qweight" not in state and f"{name}.weight" in state:
            continue  # an nn.Linear holding dequantized weights: loaded as it is
        info = layers.get(name) or _infer_info(name, state, config)
        _check_buffers(name, info, state)
        _install(model, name, info, state)
    model.load_state_dict(state)
    if not return_metadata:
        return model
    return model, {"quant_config": config, "quantized_layers": list(meta["quantized_layers"]),
                   "quantization_errors": dict(meta.get("quantization_errors") or {})}
