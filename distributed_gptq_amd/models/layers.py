"""QuantizedLinear and the ``gptq::linear`` operator (models/layers.py:15-188).

The reference's forward calls ``torch.ops.gptq.linear(x, qweight, scales,
zeros, g_idx, bias)`` whenever ``torch.ops.gptq`` exists (:150-153) and
otherwise ``F.linear(x, unpack_weights(), bias)`` (:155-157).  This module
registers that operator, implemented by the HIP dequant-GEMV/GEMM, with the
fallback's semantics (fp32 dequantized weights, fp32 accumulation, output in
x's dtype).

Buffers keep the reference layout: qweight uint8 (N, ceil(K/2)) for 4-bit
(byte = w[2i] | w[2i+1] << 4) and (N, K) one code per byte otherwise
(:49-55); fp16 scales/zeros (N, ceil(K/g)) (:56-57).  ``packed=True`` stores
2/3-bit codes as LSB-first bit streams too (ceil(K*bits/8) bytes per row),
the layout of the W3A16 GEMV.  ``g_idx[k]`` holds the group of input column
k (k // group_size unless act-order reordered the groups); the reference's
placeholder arange(K) (:60, unused by its own unpack) is read as contiguous
groups of ``group_size`` (rewritten to arange(K) // group_size when loaded).

One buffer is added: ``perm`` (int32).  Empty, the weight columns are in
input order.  With act-order it holds K entries and weight column j holds
input column perm[j], stored so that groups are contiguous (g_idx[perm[j]]
= j // group_size; perm is the stable sort of g_idx, i.e. within a group the
input columns ascend): the layer is then served by
the same fast kernels, x gathered through perm, instead of a per-weight
group lookup.  The operator takes it as an optional last argument, so the
reference's six-argument call is unchanged.  ``perm`` is not part of the
state dict: ``state_dict()`` writes qweight in input-column order (the
reference's layout, so its strict ``load_state_dict`` takes the file), and
loading re-derives perm as the stable sort of g_idx, as ``pack_weights``
does, and reorders the codes again.
"""
from __future__ import annotations

import math
import weakref
from typing import Optional

import torch
import torch.nn as nn

from .. import _ops

# ------------------------------------------------------------- operator --

_OP_LIB = None
# (id(g_idx), id(perm)) -> (weakrefs, stamps, result); tensors cannot be dict
# keys by value (their == is elementwise)
_layout_cache: dict = {}


def _infer_bits(qweight: torch.Tensor, K: int) -> int:
    """Code width from the row length: K -> one code per byte (0), else the
    packed width whose pitch ceil(K*b/8) matches (4 preferred)."""
    pitch = qweight.shape[1]
    if pitch == K:
        return 0
    for b in (4, 3, 2):
        if pitch == (K * b + 7) // 8:
            return b
    raise ValueError(f"qweight rows of {pitch} bytes match no code width for in_features={K}")


def _stamp(t):
    if t is None:
        return None
    # inference tensors have no version counter
    return (id(t), None if t.is_inference() else t._version, t.data_ptr())


def _group_layout(g_idx: torch.Tensor, K: int, ngroups: int, perm: Optional[torch.Tensor] = None):
    """(group_size, g_idx or None) of the stored weight columns: contiguous
    groups are passed as a group size (fast kernels), anything else as the
    per-column group gather (in stored order: g_idx[perm[j]] with perm).
    The answer is cached per g_idx/perm tensor and version (a few device
    syncs the first time)."""
    key = (id(g_idx), id(perm) if perm is not None else 0)
    stamp = (_stamp(g_idx), _stamp(perm))
    hit = _layout_cache.get(key)
    if hit is not None and hit[0]() is g_idx and hit[1] == stamp:
        return hit[2]
    ar = torch.arange(K, device=g_idx.device, dtype=torch.int32)
    gi = g_idx.to(torch.int32)
    if perm is not None:
        gi = gi[perm.to(device=g_idx.device).long()]
    if perm is None and ngroups != K and bool(torch.equal(gi, ar)):
        # the reference's placeholder arange(K): contiguous groups, whose size
        # only ngroups tells; it is unambiguous when K is a whole number of them
        gs = math.ceil(K / ngroups)
        if K % gs:
            raise ValueError(f"g_idx is the placeholder arange({K}) and {ngroups} groups do not divide K evenly; "
                             "the group size is ambiguous: pass g_idx = arange(K) // group_size")
        res = (gs, None)
    else:
        gs = int((gi == 0).sum().item())
        if gs > 0 and math.ceil(K / gs) <= ngroups and bool(torch.equal(gi, ar // gs)):
            res = (gs, None)
        else:
            res = (math.ceil(K / ngroups), gi.contiguous())
    _layout_cache[key] = (weakref.ref(g_idx, lambda _r, k=key: _layout_cache.pop(k, None)), stamp, res)
    return res


# Rows of x from which the weights are dequantised once (to x's dtype) and
# multiplied by the library GEMM instead of the fused kernels, which decode
# every weight once per 128 rows.  Measured on MI355X (4-bit, fp16/bf16, the
# Llama-3-8B and 13B layer shapes): at 384 rows the two are even or the GEMM
# wins, at 512 it wins everywhere, at 16384 rows by 3.4-3.7x.
DEQUANT_GEMM_ROWS = 384


def _unpack_rows(qweight: torch.Tensor, bits: int, K: int) -> torch.Tensor:
    """(N, K) uint8 codes of LSB-first b-bit rows (any device; byte ops
    only -- a checkpoint's storage order, not the compute path)."""
    N = qweight.shape[0]
    if bits in (2, 4, 8):
        per = 8 // bits
        sh = torch.arange(0, 8, bits, device=qweight.device, dtype=torch.uint8)
        c = (qweight.unsqueeze(-1) >> sh) & ((1 << bits) - 1)
        return c.reshape(N, -1)[:, :K].contiguous() if per > 1 else qweight[:, :K].contiguous()
    sh = torch.arange(8, device=qweight.device, dtype=torch.uint8)
    b = ((qweight.unsqueeze(-1) >> sh) & 1).reshape(N, -1)[:, :K * bits].reshape(N, K, bits)
    out = b[..., 0].clone()
    for i in range(1, bits):
        out |= b[..., i] << i
    return out


def _pack_rows(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of ``_unpack_rows``: ceil(K * bits / 8) bytes per row."""
    N, K = codes.shape
    pitch = (K * bits + 7) // 8
    if bits in (2, 4, 8):
        per = 8 // bits
        c = torch.zeros(N, pitch * per, device=codes.device, dtype=torch.uint8)
        c[:, :K] = codes
        c = c.reshape(N, pitch, per)
        out = c[..., 0].clone()
        for i in range(1, per):
            out |= c[..., i] << (bits * i)
        return out
    sh = torch.arange(bits, device=codes.device, dtype=torch.uint8)
    b = torch.zeros(N, pitch * 8, device=codes.device, dtype=torch.uint8)
    b[:, :K * bits] = ((codes.unsqueeze(-1) >> sh) & 1).reshape(N, -1)
    b = b.reshape(N, pitch, 8)
    out = b[..., 0].clone()
    for i in range(1, 8):
        out |= b[..., i] << i
    return out


def _gather_code_columns(qweight: torch.Tensor, bits: int, packed: bool, K: int, idx: torch.Tensor) -> torch.Tensor:
    """Stored codes with column j of the result taken from column idx[j]."""
    idx = idx.to(device=qweight.device).long()
    if not packed or bits == 8:
        return qweight[:, idx].contiguous()
    return _pack_rows(_unpack_rows(qweight, bits, K)[:, idx], bits)


def _linear_impl(x, qweight, scales, zeros, g_idx, bias, perm=None):
    K = g_idx.numel()
    bits = _infer_bits(qweight, K)
    if perm is not None and perm.numel() == 0:
        perm = None
    gs, gi = _group_layout(g_idx, K, scales.shape[1], perm)
    rows = x.numel() // K if K else 0
    if rows >= DEQUANT_GEMM_ROWS and x.dtype in (torch.float16, torch.bfloat16):
        # the reference's fallback F.linear(x, unpack_weights(), bias)
        # (models/layers.py:155-157), with the weights rounded to x's dtype once
        W = _ops.dequant(qweight, bits, scales, zeros, K, g_idx=gi, group_size=gs, dtype=x.dtype)
        if perm is not None:
            if rows < W.shape[0]:
                x = x.index_select(-1, perm.long())
            else:
                Wi = torch.empty_like(W)
                Wi[:, perm.long()] = W
                W = Wi
        # fp32 accumulation and output, the bias added in fp32, one rounding to
        # x's dtype (a 16-bit product may otherwise reduce split-K partials in
        # 16 bits, torch's allow_*_reduced_precision_reduction default)
        x2 = x.reshape(-1, K)
        if bias is None:
            y = torch.mm(x2, W.t(), out_dtype=torch.float32)
        else:
            y = torch.addmm(bias.to(torch.float32), x2, W.t(), out_dtype=torch.float32)
        return y.to(x.dtype).reshape(*x.shape[:-1], W.shape[0])
    return _ops.linear(x, qweight, bits, scales, zeros, K, g_idx=gi, group_size=gs, bias=bias, perm=perm)


def _dequant_input_order(qweight, scales, zeros, g_idx, perm=None) -> torch.Tensor:
    """fp32 (N, K) dequantised weights in input-column order."""
    K = g_idx.numel()
    if perm is not None and perm.numel() == 0:
        perm = None
    gs, gi = _group_layout(g_idx, K, scales.shape[1], perm)
    W = _ops.dequant(qweight, _infer_bits(qweight, K), scales, zeros, K, g_idx=gi, group_size=gs)
    if perm is None:
        return W
    out = torch.empty_like(W)
    out[:, perm.long()] = W
    return out


def _linear_setup(ctx, inputs, output):
    x, qweight, scales, zeros, g_idx, bias, perm = inputs
    ctx.save_for_backward(qweight, scales, zeros, g_idx, perm)
    ctx.x_dtype = x.dtype
    ctx.has_bias = bias is not None


def _linear_backward(ctx, grad):
    """Gradients of the fallback F.linear(x, unpack_weights(), bias): the
    quantized weights are constants; x and bias get their usual gradients."""
    qweight, scales, zeros, g_idx, perm = ctx.saved_tensors
    gx = gb = None
    if ctx.needs_input_grad[0]:
        W = _dequant_input_order(qweight, scales, zeros, g_idx, perm)
        gx = (grad.float() @ W).to(ctx.x_dtype)
    if ctx.has_bias and ctx.needs_input_grad[5]:
        gb = grad.reshape(-1, grad.shape[-1]).float().sum(0)
    return gx, None, None, None, None, gb, None


def register_ops():
    """Define gptq::linear with its CUDA kernel and autograd (idempotent)."""
    global _OP_LIB
    if _OP_LIB is not None:
        return
    if hasattr(torch.ops, "gptq") and hasattr(torch.ops.gptq, "linear"):
        return
    lib = torch.library.Library("gptq", "DEF")
    lib.define("linear(Tensor x, Tensor qweight, Tensor scales, Tensor zeros, Tensor g_idx, Tensor? bias, "
               "Tensor? perm=None) -> Tensor")
    lib.impl("linear", _linear_impl, "CUDA")
    torch.library.register_autograd("gptq::linear", _linear_backward, setup_context=_linear_setup, lib=lib)
    _OP_LIB = lib


register_ops()


# -------------------------------------------------------- QuantizedLinear --

class QuantizedLinear(nn.Module):
    """Quantized Linear layer (models/layers.py:15-188)."""

    def __init__(self, bits: int, group_size: int, in_features: int, out_features: int, bias: bool = True,
                 packed: bool = False):
        super().__init__()
        self.bits = bits
        self.group_size = group_size if group_size > 0 else in_features
        self.in_features = in_features
        self.out_features = out_features
        self.packed = packed or bits == 4
        self.num_groups = math.ceil(in_features / self.group_size)
        if self.packed:
            weight_shape = (out_features, (in_features * bits + 7) // 8)
        else:
            weight_shape = (out_features, in_features)
        self.register_buffer("qweight", torch.zeros(weight_shape, dtype=torch.uint8))
        self.register_buffer("scales", torch.zeros((out_features, self.num_groups), dtype=torch.float16))
        self.register_buffer("zeros", torch.zeros((out_features, self.num_groups), dtype=torch.float16))
        self.register_buffer("g_idx", torch.arange(in_features, dtype=torch.int32) // self.group_size)
        self.register_buffer("perm", torch.zeros(0, dtype=torch.int32), persistent=False)
        if bias:
            self.register_parameter("bias", nn.Parameter(torch.zeros(out_features)))
        else:
            self.register_parameter("bias", None)

    def _contiguous_order(self, gi: torch.Tensor) -> Optional[torch.Tensor]:
        """The stored column order that makes an act-order g_idx's groups
        contiguous (the stable sort of g_idx), or None when g_idx already is
        k // group_size or no order makes it so."""
        ar = torch.arange(self.in_features, dtype=torch.int32, device=gi.device)
        contiguous = ar // self.group_size
        if bool(torch.equal(gi, contiguous)):
            return None
        cand = torch.argsort(gi, stable=True).to(torch.int32)
        if bool(torch.equal(gi[cand.long()], contiguous)):
            return cand
        return None

    def pack_weights(self, weight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                     g_idx: Optional[torch.Tensor] = None, perm: Optional[torch.Tensor] = None):
        """Store integer codes (N, K, input-column order) and fp16
        scales/zeros (:67-96).  With an act-order ``g_idx`` (groups out of
        input order) the columns are stored in the order that makes the
        groups contiguous: the stable sort of g_idx, the order a loaded
        checkpoint re-derives (a given ``perm``, e.g. GPTQ's sweep order,
        must make the groups contiguous too; it is replaced by that order,
        which holds the same groups).  ``g_idx`` itself keeps its meaning
        (group of input column k)."""
        codes = weight.to(torch.uint8)
        dev = codes.device
        self.scales.data = scales.to(torch.float16).reshape(self.out_features, -1).contiguous()
        self.zeros.data = zeros.to(torch.float16).reshape(self.out_features, -1).contiguous()
        if g_idx is not None:
            self.g_idx.data = g_idx.to(torch.int32).to(dev)
        gi = self.g_idx.to(dev)
        if perm is not None:
            perm = perm.to(device=dev, dtype=torch.long)
            contiguous = torch.arange(self.in_features, dtype=torch.int32, device=dev) // self.group_size
            if perm.numel() != self.in_features or not bool(torch.equal(gi[perm], contiguous)):
                raise ValueError("pack_weights: perm does not make the groups of g_idx contiguous")
        perm = self._contiguous_order(gi)
        if perm is not None:
            codes = codes[:, perm.long()]
            self.perm.data = perm.contiguous()
        else:
            self.perm.data = torch.zeros(0, dtype=torch.int32, device=dev)
        self.qweight.data = _ops.pack(codes, self.bits) if self.packed else codes.contiguous()

    def unpack_weights(self) -> torch.Tensor:
        """fp32 (N, K) = (q - zero) * scale per group (:98-138), bit-exact,
        in input-column order."""
        return _dequant_input_order(self.qweight, self.scales, self.zeros, self.g_idx, self.perm)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """:140-157 -- the gptq::linear operator, registered above."""
        if self.perm.numel():
            return torch.ops.gptq.linear(x, self.qweight, self.scales, self.zeros, self.g_idx, self.bias, self.perm)
        return torch.ops.gptq.linear(x, self.qweight, self.scales, self.zeros, self.g_idx, self.bias)

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        # the reference's layout: codes in input-column order, no perm
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self.perm.numel():
            inv = torch.argsort(self.perm.long())  # input column k sits at stored column inv[k]
            destination[prefix + "qweight"] = _gather_code_columns(self.qweight.detach(), self.bits, self.packed,
                                                                   self.in_features, inv)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        # Files hold qweight in input-column order (the reference's layout,
        # and what state_dict() writes); files written with a ``perm`` key
        # (K entries) hold it in that stored order instead.
        key = prefix + "perm"
        saved = state_dict.get(key)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)
        if key in unexpected_keys:
            unexpected_keys.remove(key)
        dev = self.qweight.device
        K = self.in_features
        if saved is not None and saved.numel():
            if saved.shape != (K,):
                error_msgs.append(f"{key}: saved shape {tuple(saved.shape)}, expected (0,) or ({K},)")
                return
            self.perm.data = saved.to(device=dev, dtype=torch.int32).contiguous()
            return
        self.perm.data = torch.zeros(0, dtype=torch.int32, device=dev)
        if self.g_idx.numel() != K:
            return
        gi = self.g_idx.to(torch.int32)
        ar = torch.arange(K, dtype=torch.int32, device=gi.device)
        if self.num_groups != K and bool(torch.equal(gi, ar)):
            # the reference's placeholder g_idx = arange(K) (models/layers.py:60)
            # means contiguous groups of group_size
            self.g_idx.data = ar // self.group_size
            return
        perm = self._contiguous_order(gi)
        if perm is not None:
            self.qweight.data = _gather_code_columns(self.qweight, self.bits, self.packed, K, perm)
            self.perm.data = perm.to(dev).contiguous()

    @classmethod
    def from_linear(cls, linear_layer: nn.Linear, bits: int = 4, group_size: int = 128,
                    packed: bool = False) -> "QuantizedLinear":
        """:159-188 (shape and bias only; codes come from pack_weights /
        from_gptq)."""
        q = cls(bits=bits, group_size=group_size, in_features=linear_layer.in_features,
                out_features=linear_layer.out_features, bias=linear_layer.bias is not None, packed=packed)
        q = q.to(linear_layer.weight.device)
        if linear_layer.bias is not None:
            q.bias.data = linear_layer.bias.data
        return q

    @classmethod
    def from_gptq(cls, gptq, linear_layer: Optional[nn.Linear] = None, packed: bool = True) -> "QuantizedLinear":
        """Build from a GPTQ object after ``fasterquant()``: codes, scales,
        zeros and act-order g_idx."""
        layer = linear_layer if linear_layer is not None else gptq.layer
        gs = getattr(gptq, "_gs_used", gptq.group_size)
        q = cls(bits=gptq.bits, group_size=gs if gs > 0 else layer.in_features, in_features=layer.in_features,
                out_features=layer.out_features, bias=layer.bias is not None, packed=packed)
        q = q.to(layer.weight.device)
        q.pack_weights(gptq.qcodes, gptq.scale, gptq.zero, gptq.g_idx, perm=gptq.perm)
        if layer.bias is not None:
            q.bias.data = layer.bias.data.clone()
        return q


class FusedQuantizedLinear(nn.Module):
    """Several QuantizedLinear layers that read the same input (q/k/v,
    gate/up) served by one gptq::linear call: their weights, scales, zeros
    and biases are concatenated along the output rows, so a decode step pays
    one launch, and its fixed start-up cost, for all of them.  forward
    returns one output per layer, in the order given.  The layers must agree
    on in_features, bits, group size, storage and column order (g_idx and
    perm): layers quantized against one shared Hessian do."""

    def __init__(self, layers):
        super().__init__()
        layers = list(layers)
        if not layers:
            raise ValueError("FusedQuantizedLinear: no layers")
        first = layers[0]
        for q in layers[1:]:
            same = (q.in_features == first.in_features and q.bits == first.bits
                    and q.group_size == first.group_size and q.packed == first.packed
                    and torch.equal(q.g_idx, first.g_idx) and torch.equal(q.perm, first.perm))
            if not same:
                raise ValueError("FusedQuantizedLinear: the layers differ in in_features, bits, group size, "
                                 "storage or column order (g_idx / perm)")
        self.bits, self.group_size, self.packed = first.bits, first.group_size, first.packed
        self.in_features = first.in_features
        self.splits = [q.out_features for q in layers]
        self.out_features = sum(self.splits)
        self.register_buffer("qweight", torch.cat([q.qweight for q in layers], 0))
        self.register_buffer("scales", torch.cat([q.scales for q in layers], 0))
        self.register_buffer("zeros", torch.cat([q.zeros for q in layers], 0))
        self.register_buffer("g_idx", first.g_idx.clone())
        self.register_buffer("perm", first.perm.clone())
        if any(q.bias is not None for q in layers):
            b = [q.bias.data if q.bias is not None else torch.zeros(q.out_features, device=q.qweight.device)
                 for q in layers]
            self.register_parameter("bias", nn.Parameter(torch.cat([t.float() for t in b], 0)))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor):
        if self.perm.numel():
            y = torch.ops.gptq.linear(x, self.qweight, self.scales, self.zeros, self.g_idx, self.bias, self.perm)
        else:
            y = torch.ops.gptq.linear(x, self.qweight, self.scales, self.zeros, self.g_idx, self.bias)
        return tuple(y.split(self.splits, dim=-1))


def replace_with_quantized_layers(model: nn.Module, quantizers: dict, packed: bool = True) -> nn.Module:
    """models/layers.py:285-315: swap each quantized nn.Linear (by name) for a
    QuantizedLinear built from its GPTQ result."""
    for name, gptq in quantizers.items():
        parent = model
        parts = name.split(".")
        for p in parts[:-1]:
            parent = getattr(parent, p)
        old = getattr(parent, parts[-1])
        setattr(parent, parts[-1], QuantizedLinear.from_gptq(gptq, old, packed=packed))
    return model
