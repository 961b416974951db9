"""Per-element error bound for gptq::linear outputs against the fp64 oracle.

The reference's forward is ``F.linear(x, unpack_weights(), bias)``
(models/layers.py:155-157) with the weights dequantised in fp32 as
``(q - zero) * scale`` (models/layers.py:136).  For fp16 / bf16 activations the
HIP kernels compute one of two things, per call:

* exact weights: s * (sum x q - z sum x) per group, or products of x with the
  fp32 dequantised weight (the M = 1 GEMV, zero points folded per group);
* weights rounded once to x's dtype, then multiplied (the dequantise-then-
  MFMA kernels; what ``F.linear(x, unpack_weights().to(x.dtype))`` computes).

Both accumulate in fp32 and round the result once to x's dtype.  So each
output element must lie within

    1/2 ulp_out(|ref| + acc)  +  acc,    acc = d * 2^-24 * (sum_k |x_k| |w_k| + |bias|)

of the fp64 value ``ref`` of the same semantics.  acc is the worst-case bound
of an fp32 sum in which no term passes through more than d roundings
(Higham's gamma_d; a K-term sum in one sequential chain has d = K - 1).  These
kernels sum K products in chains of MFMA or dot steps: an MFMA adds k >= 8
products (k = 8-32) to its accumulator, so a product passes through at most
k - 1 roundings inside its step and one per later step, K / k + k in all,
then the cross-lane, cross-wave and split-K reductions (at most 6 + 4 + 8
levels), the per-group zero-point correction and the bias; the generic
kernel sums K / 64 terms per lane, then 6 levels.  d = K / 8 + 128 bounds
every one of these, and the library GEMM of the many-row route (fp32
accumulation through MFMAs of k >= 8, fp32 output).  A call passes when every
element is inside the bound of one of the two semantics.  The checker then plants one wrong code (the top bit of the
code flipped where |x| * scale is largest) into the oracle's input and
requires that the same output now fails the bound: that shows the bound is
tight enough to see a single wrong code.
"""
import numpy as np
import torch

U32 = 2.0 ** -24
_MANT = {torch.float16: (10, -14), torch.bfloat16: (7, -126), torch.float32: (23, -126)}


def _t64(a):
    if a is None:
        return None
    if isinstance(a, torch.Tensor):
        return a.detach().cpu().to(torch.float64)
    return torch.from_numpy(np.asarray(a)).to(torch.float64)


def ulp(v, dtype):
    """Spacing of ``dtype`` at magnitude |v| (subnormal spacing below the
    smallest normal)."""
    mant, emin = _MANT[dtype]
    a = torch.clamp(v.abs(), min=2.0 ** emin)
    e = torch.floor(torch.log2(a))
    return torch.pow(2.0, e - mant)


def _round_to(w32, dtype):
    """fp32 values rounded once to ``dtype`` (torch's round-to-nearest-even)."""
    return w32.to(torch.float32).to(dtype).to(torch.float64)


def dequant_weights(codes, scales, zeros, g_idx):
    """(q - z[g]) * s[g] in fp32, as the oracle's ``dequant`` computes it."""
    q = torch.from_numpy(np.asarray(codes)).to(torch.float32)
    gi = torch.from_numpy(np.asarray(g_idx)).long()
    s = _t64(scales).to(torch.float32)[:, gi]
    z = _t64(zeros).to(torch.float32)[:, gi]
    return (q - z) * s


class Violation(AssertionError):
    pass


def _margins(y, x, W, bias, K, odt):
    ref = x @ W.T
    mag = x.abs() @ W.abs().T
    if bias is not None:
        ref = ref + bias
        mag = mag + bias.abs()
    acc = (K / 8 + 128) * U32 * mag
    bound = 0.5 * ulp(ref.abs() + acc, odt) + acc
    return (y - ref).abs() / bound, ref, bound


def check_linear(y, x, codes, scales, zeros, g_idx, bias=None, *, bits=None, plant=True, label=""):
    """Assert ``y`` (M x N, x's dtype) is gptq::linear of ``x`` (M x K, in the
    input-column order of ``codes``) within the per-element bound of one of the
    two semantics above; with ``plant``, also assert that one planted wrong
    code is caught.  Returns the largest |y - ref| / bound of the passing
    semantics."""
    odt = y.dtype
    y64 = y.detach().cpu().to(torch.float64)
    x64 = _t64(x)
    b64 = _t64(bias)
    K = x64.shape[1]
    W32 = dequant_weights(codes, scales, zeros, g_idx)
    sems = {"exact": W32.to(torch.float64)}
    if odt != torch.float32:
        sems["rounded"] = _round_to(W32, odt)
    best = None
    for name, W in sems.items():
        r, ref, bound = _margins(y64, x64, W, b64, K, odt)
        worst = float(r.max()) if r.numel() else 0.0
        if best is None or worst < best[1]:
            best = (name, worst, W, ref, bound)
    name, worst, W, ref, bound = best
    print(f"{label} gptq::linear bound: {name} weights, max |y - ref| / bound = {worst:.3e}")
    if worst > 1.0:
        m, n = divmod(int(torch.argmax((y64 - ref).abs() / bound)), y64.shape[1])
        raise Violation(f"{label}: y[{m},{n}] = {float(y64[m, n])!r}, ref {float(ref[m, n])!r}, "
                        f"bound {float(bound[m, n]):.3e} ({name} weights; ratio {worst:.3e})")
    if plant and y64.numel():
        _check_plant(y64, x64, codes, scales, zeros, g_idx, b64, sems, odt, bits)
    return worst


def _check_plant(y64, x64, codes, scales, zeros, g_idx, b64, sems, odt, bits):
    """Flip the top bit of one code, at the (m, n, k) where |x| * scale is
    largest, in the oracle's input: the GPU output must now fail the bound
    under every semantics (only column n changes)."""
    codes = np.asarray(codes)
    if bits is None:
        bits = max(1, int(codes.max()).bit_length())
    gi = torch.from_numpy(np.asarray(g_idx)).long()
    s = _t64(scales)[:, gi].abs()                 # N x K
    xm = x64.abs().max(0)                         # best row of x per column
    score = s * xm.values[None, :]
    n, k = divmod(int(torch.argmax(score)), score.shape[1])
    m = int(xm.indices[k])
    bad = codes.copy()
    bad[n, k] ^= 1 << (bits - 1)
    Wn = dequant_weights(bad[n:n + 1], _t64(scales)[n:n + 1], _t64(zeros)[n:n + 1], g_idx)
    K = x64.shape[1]
    for name, W in sems.items():
        Wrow = Wn.to(torch.float64) if name == "exact" else _round_to(Wn, odt)
        bn = b64[n:n + 1] if b64 is not None else None
        r, _, _ = _margins(y64[:, n:n + 1], x64, Wrow, bn, K, odt)
        assert float(r.max()) > 1.0, (
            f"a wrong code at ({n}, {k}) (x row {m}) stays inside the bound under {name} weights: "
            f"ratio {float(r.max()):.3e}")
