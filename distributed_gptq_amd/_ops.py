"""Host wrappers: torch tensors in, C-ABI calls out (no compute in Python).

Every wrapper checks shapes/dtypes on the host before launching, allocates
outputs and workspaces with torch (the library never allocates), and
enqueues on torch's current stream of the tensor's device.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib as L

DTYPES = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _gpu(*ts):
    for t in ts:
        if t is not None:
            L.require_gpu(t)


_ws: dict = {}
_ws_in_graph: set = set()   # keys whose current buffer a graph capture has used
_ws_retired: list = []      # replaced buffers a captured graph may still write


def workspace(nbytes: int, device) -> torch.Tensor:
    """Scratch buffer per (device, stream), grown on demand.  Work on one
    stream is ordered, so reuse across calls is safe.  A graph captured on
    the stream bakes the buffer's address into its kernels, so a buffer
    handed out during a capture is never freed when a later, larger call
    replaces it: it is kept until ``release_workspaces()``."""
    dev = torch.device(device)
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None and key in _ws_in_graph:
            _ws_retired.append(buf)
            _ws_in_graph.discard(key)
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        _ws[key] = buf
    if torch.cuda.is_current_stream_capturing():
        _ws_in_graph.add(key)
    return buf


def release_workspaces():
    """Drop every cached workspace.  Graphs captured with them must be
    dropped first."""
    _ws.clear()
    _ws_in_graph.clear()
    _ws_retired.clear()


# ------------------------------------------------------------- Hessian --

# Bytes of Hessian workspace (partial tiles) a call may use; beyond it the
# tokens go through in runs (a little slower).  The full size for 262144
# tokens is 1.7 GB at K = 14336 (4 splits) and 0.9 GB at K = 4096 (26).
HESSIAN_WORKSPACE_CAP = 8 << 30


def hessian_accumulate(H: torch.Tensor, X: torch.Tensor, workspace_cap: int | None = None) -> None:
    """H += X^T X (H: K x K fp32 symmetric; X: (..., K) float rows).  The
    partial-tile workspace is at most ``workspace_cap`` bytes
    (HESSIAN_WORKSPACE_CAP by default), and at least one token split's."""
    _gpu(H, X)
    K = H.shape[0]
    if H.shape != (K, K) or H.dtype != torch.float32 or not H.is_contiguous():
        raise ValueError("H must be a contiguous (K, K) float32 tensor")
    if X.shape[-1] != K:
        raise ValueError(f"input has {X.shape[-1]} features, Hessian is {K} x {K}")
    X2 = X.reshape(-1, K)
    if X2.stride(-1) != 1:
        X2 = X2.contiguous()
    n = X2.shape[0]
    if n == 0:
        return
    ldx = X2.stride(0) if n > 1 else K
    lib = L.lib()
    cap = HESSIAN_WORKSPACE_CAP if workspace_cap is None else workspace_cap
    nb = min(lib.gptq_hessian_workspace_size(n, K), max(lib.gptq_hessian_workspace_min(K), cap))
    ws = workspace(nb, H.device)
    L.call("gptq_hessian_accumulate", _p(H), _p(X2), n, K, ldx, dtype_code(X2.dtype), _p(ws), nb,
           _stream(H.device))


# ------------------------------------------------------ damp + factor --

def damp_factor(H: torch.Tensor, scale: float, percdamp: float, perm: torch.Tensor | None = None,
                mode: int = L.FACTOR_UPPER_CHOL_INV, want_hd: bool = False, want_dead: bool = False):
    """Returns (out, Hd or None, dead or None, info) -- info is a 1-element
    int32 device tensor (0 = ok, >0 = not positive definite)."""
    _gpu(H)
    K = H.shape[0]
    if H.shape != (K, K) or H.dtype != torch.float32 or not H.is_contiguous():
        raise ValueError("H must be a contiguous (K, K) float32 tensor")
    dev = H.device
    out = torch.empty((K, K), dtype=torch.float32, device=dev)
    Hd = torch.empty((K, K), dtype=torch.float32, device=dev) if want_hd else None
    dead = torch.empty(K, dtype=torch.int32, device=dev) if want_dead else None
    info = torch.empty(1, dtype=torch.int32, device=dev)
    if perm is not None:
        perm = perm.to(device=dev, dtype=torch.int32).contiguous()
        if perm.numel() != K:
            raise ValueError("perm must have K entries")
    nb = L.lib().gptq_factor_workspace_size(K)
    ws = workspace(nb, dev)
    L.call("gptq_damp_factor", _p(H), K, ctypes.c_float(scale), ctypes.c_float(percdamp), _p(perm), mode,
           _p(Hd), _p(out), _p(dead), _p(info), _p(ws), ws.numel(), _stream(dev))
    return out, Hd, dead, info


# ---------------------------------------------------------- the sweep --

def prepare_weight(w: torch.Tensor, perm=None, dead=None, transpose: bool = False) -> torch.Tensor:
    """fp32 copy of a 2-D weight in sweep order (see gptq_prepare_weight)."""
    _gpu(w)
    if w.dim() != 2 or w.stride(-1) != 1:
        w = w.reshape(w.shape[0], -1).contiguous()
    R, C = w.shape
    rows, cols = (C, R) if transpose else (R, C)
    out = torch.empty((rows, cols), dtype=torch.float32, device=w.device)
    if perm is not None:
        perm = perm.to(device=w.device, dtype=torch.int32).contiguous()
    L.call("gptq_prepare_weight", _p(w), dtype_code(w.dtype), rows, cols, w.stride(0), _p(perm), _p(dead),
           1 if transpose else 0, _p(out), _stream(w.device))
    return out


def ngroups_of(cols: int, group_size: int) -> int:
    return math.ceil(cols / group_size) if group_size > 0 else 1


def quantize_sweep(W: torch.Tensor, T: torch.Tensor, bits: int, group_size: int, blocksize: int, flags: int,
                   W0=None, out_cols=None, dequant_dtype=None, scale=None, zero=None,
                   want_losses: bool = False, want_err: bool = True):
    """Runs gptq_quantize_sweep on W (rows x cols fp32, modified in place)
    with T (>= cols x cols, row stride T.stride(0)).  Returns a dict of
    codes, dequant, scale, zero, err_sq, losses (None where not asked)."""
    _gpu(W, T)
    rows, cols = W.shape
    if W.dtype != torch.float32 or not W.is_contiguous():
        raise ValueError("W must be contiguous float32")
    if T.dtype != torch.float32 or T.stride(1) != 1 or T.shape[0] < cols or T.shape[1] < cols:
        raise ValueError("T must be float32 with unit column stride and at least cols x cols")
    dev = W.device
    ng = ngroups_of(cols, group_size)
    if scale is None:
        if group_size <= 0:
            raise ValueError("per-row parameters must be given when group_size <= 0")
        scale = torch.empty((rows, ng), dtype=torch.float32, device=dev)
        zero = torch.empty((rows, ng), dtype=torch.float32, device=dev)
    codes = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
    dq = torch.empty((rows, cols), dtype=dequant_dtype, device=dev) if dequant_dtype is not None else None
    err = torch.empty(rows, dtype=torch.float32, device=dev) if want_err else None
    losses = torch.empty((rows, cols), dtype=torch.float32, device=dev) if want_losses else None
    if out_cols is not None:
        out_cols = out_cols.to(device=dev, dtype=torch.int32).contiguous()
    nb = L.lib().gptq_sweep_workspace_size(rows, cols, blocksize)
    ws = workspace(nb, dev)
    L.call("gptq_quantize_sweep", _p(W), _p(W0), _p(T), T.stride(0), rows, cols, bits, group_size, blocksize, flags,
           _p(out_cols), _p(codes), _p(dq), dtype_code(dq.dtype) if dq is not None else 0, _p(scale), _p(zero),
           _p(err), _p(losses), _p(ws), ws.numel(), _stream(dev))
    return dict(codes=codes, dequant=dq, scale=scale, zero=zero, err_sq=err, losses=losses)


def minmax_params(src: torch.Tensor, bits: int, group_size: int, flags: int):
    _gpu(src)
    if src.dtype != torch.float32 or src.stride(-1) != 1 or src.dim() != 2:
        src = src.reshape(src.shape[0], -1).float().contiguous()
    rows, cols = src.shape
    ng = ngroups_of(cols, group_size)
    scale = torch.empty((rows, ng), dtype=torch.float32, device=src.device)
    zero = torch.empty_like(scale)
    L.call("gptq_minmax_params", _p(src), rows, cols, src.stride(0), bits, group_size, flags, _p(scale), _p(zero),
           _stream(src.device))
    return scale, zero


def quantize_rows(x: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, bits: int, group_size: int, flags: int,
                  want_codes: bool = True, want_dequant: bool = True):
    _gpu(x)
    x = x.float().contiguous()
    rows, cols = x.shape
    ng = ngroups_of(cols, group_size)
    scale = scale.float().reshape(rows, ng).contiguous()
    zero = zero.float().reshape(rows, ng).contiguous()
    codes = torch.empty((rows, cols), dtype=torch.uint8, device=x.device) if want_codes else None
    dq = torch.empty((rows, cols), dtype=torch.float32, device=x.device) if want_dequant else None
    L.call("gptq_quantize_rows", _p(x), rows, cols, bits, group_size, flags, _p(scale), _p(zero), _p(codes), _p(dq),
           _stream(x.device))
    return codes, dq


# -------------------------------------------------------------- formats --

def packed_pitch(K: int, bits: int) -> int:
    return (K * bits + 7) // 8


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    _gpu(codes)
    codes = codes.to(torch.uint8).contiguous()
    N, K = codes.shape
    out = torch.empty((N, packed_pitch(K, bits)), dtype=torch.uint8, device=codes.device)
    L.call("gptq_pack", _p(codes), N, K, bits, _p(out), _stream(codes.device))
    return out


def unpack(packed: torch.Tensor, bits: int, K: int) -> torch.Tensor:
    _gpu(packed)
    packed = packed.contiguous()
    N = packed.shape[0]
    if packed.shape[1] != packed_pitch(K, bits):
        raise ValueError(f"packed rows have {packed.shape[1]} bytes, expected {packed_pitch(K, bits)}")
    out = torch.empty((N, K), dtype=torch.uint8, device=packed.device)
    L.call("gptq_unpack", _p(packed), N, K, bits, _p(out), _stream(packed.device))
    return out


def pack_reference_layout(codes: torch.Tensor, bits: int) -> torch.Tensor:
    _gpu(codes)
    codes = codes.to(torch.uint8).contiguous()
    N, K = codes.shape
    epb = {4: 2, 2: 4}.get(bits, 1)
    if N % epb:
        raise ValueError(f"{bits}-bit reference packing needs out_features % {epb} == 0")
    out = torch.empty((K, N // epb), dtype=torch.uint8, device=codes.device)
    L.call("gptq_pack_reference_layout", _p(codes), N, K, bits, _p(out), _stream(codes.device))
    return out.view(torch.int8) if bits == 8 else out


def dequant(packed: torch.Tensor, bits: int, scales: torch.Tensor, zeros: torch.Tensor, K: int,
            g_idx: torch.Tensor | None = None, group_size: int = 0,
            dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """(N x K) weights in ``dtype`` (fp32, or rounded once to fp16 / bf16).
    bits == 0: one code per byte (N x K)."""
    _gpu(packed, scales, zeros)
    packed = packed.contiguous()
    scales = scales.contiguous()
    zeros = zeros.to(scales.dtype).contiguous()
    N = packed.shape[0]
    ng = scales.shape[1]
    if g_idx is not None:
        g_idx = g_idx.to(device=packed.device, dtype=torch.int32).contiguous()
    out = torch.empty((N, K), dtype=dtype, device=packed.device)
    L.call("gptq_dequant_to", _p(packed), bits, _p(scales), _p(zeros), dtype_code(scales.dtype), _p(g_idx),
           group_size, ng, N, K, _p(out), dtype_code(dtype), _stream(packed.device))
    return out


def linear(x: torch.Tensor, packed: torch.Tensor, bits: int, scales: torch.Tensor, zeros: torch.Tensor, K: int,
           g_idx: torch.Tensor | None = None, group_size: int = 0, bias: torch.Tensor | None = None,
           out: torch.Tensor | None = None, perm: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ dequant(W)^T (+ bias), x (..., K) -> (..., N) in x.dtype.
    With ``perm`` (act-order storage: weight column j holds input column
    perm[j]) y = x[..., perm] @ dequant(W)^T (+ bias)."""
    _gpu(x, packed, scales, zeros)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    M = x2.shape[0]
    N = packed.shape[0]
    scales = scales.contiguous()
    zeros = zeros.to(scales.dtype).contiguous()
    if g_idx is not None:
        g_idx = g_idx.to(device=x.device, dtype=torch.int32).contiguous()
    if bias is not None:
        bias = bias.contiguous()
    y = out if out is not None else torch.empty((M, N), dtype=x.dtype, device=x.device)
    if perm is not None:
        perm = perm.to(device=x.device, dtype=torch.int32).contiguous()
        if perm.numel() != K:
            raise ValueError(f"perm has {perm.numel()} entries, in_features is {K}")
    # the gathered activations (act-order) and the split-K partial sums live
    # in one workspace; exactly the requested size is passed, so the kernel
    # choice depends on the shapes only
    nb = L.lib().gptq_linear_workspace_size(M, N, K, bits, group_size if g_idx is None else 0,
                                            dtype_code(x2.dtype), int(perm is not None))
    ws = workspace(nb, x.device) if nb else None
    L.call("gptq_linear_ws", _p(x2), dtype_code(x2.dtype), M, _p(perm), _p(packed), bits, _p(scales), _p(zeros),
           dtype_code(scales.dtype), _p(g_idx), group_size, scales.shape[1], _p(bias),
           dtype_code(bias.dtype) if bias is not None else 0, N, K, _p(y), _p(ws), nb, _stream(x.device))
    return y.reshape(*lead, N)


def quantize_tensor(x: torch.Tensor, bits: int, group_size: int, scales=None, zeros=None):
    """Flat-group min-max quantiser; with scales/zeros given only the
    elementwise pass runs."""
    _gpu(x)
    x = x.contiguous()
    n = x.numel()
    ng = math.ceil(n / group_size)
    q = torch.empty(n, dtype=torch.int8, device=x.device)
    flags = 0
    if scales is not None:
        scales = scales.float().reshape(-1).contiguous()
        zeros = zeros.float().reshape(-1).contiguous()
        if scales.numel() != ng or zeros.numel() != ng:
            raise ValueError(f"expected {ng} scales and zeros")
        flags = L.TENSOR_PARAMS_GIVEN
    else:
        scales = torch.empty(ng, dtype=torch.float32, device=x.device)
        zeros = torch.empty(ng, dtype=torch.float32, device=x.device)
    L.call("gptq_quantize_tensor", _p(x), dtype_code(x.dtype), n, bits, group_size, flags, _p(q), _p(scales),
           _p(zeros), _stream(x.device))
    return q.reshape(x.shape), scales, zeros


def dequantize_tensor(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group_size: int):
    _gpu(q)
    q = q.to(torch.int8).contiguous()
    n = q.numel()
    scales = scales.float().contiguous()
    zeros = zeros.float().contiguous()
    out = torch.empty(n, dtype=torch.float32, device=q.device)
    L.call("gptq_dequantize_tensor", _p(q), n, group_size, _p(scales), _p(zeros), _p(out), _stream(q.device))
    return out.reshape(q.shape)
