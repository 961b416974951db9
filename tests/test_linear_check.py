"""The gptq::linear checker itself (tests/linear_check.py), on the CPU: outputs
computed the two ways the kernels do (weights rounded to x's dtype, and the
exact form with per-group zero folding and a magic-exponent offset) pass the
bound; a wrong code, a wrong group scale and a shifted code row fail it."""
import numpy as np
import pytest
import torch

from tests.linear_check import Violation, check_linear, dequant_weights


def _case(M, N, K, bits, gs, seed, xdt):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    ng = -(-K // gs)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, ng))).half()
    zeros = torch.from_numpy(rng.integers(0, 2 ** bits, (N, ng)).astype(np.float64)).half()
    x = torch.from_numpy(rng.standard_normal((M, K))).to(xdt)
    return codes, scales, zeros, x


def _rounded(x, codes, scales, zeros, gi, bias):
    """fp32 accumulation over 32-column steps of x times the weights rounded
    to x's dtype, rounded once to x's dtype."""
    W = dequant_weights(codes, scales, zeros, gi).to(x.dtype).float()
    xf = x.float()
    acc = torch.zeros(x.shape[0], codes.shape[0])
    for k0 in range(0, x.shape[1], 32):
        acc = acc + xf[:, k0:k0 + 32] @ W[:, k0:k0 + 32].T
    if bias is not None:
        acc = acc + bias.float()
    return acc.to(x.dtype)


def _folded(x, codes, scales, zeros, gi, bias, off=1264.0):
    """s (sum x (off + q) - (off + z) sum x) per 32-column chunk, in fp32 (the
    GEMV's magic-exponent decode with the zero point folded)."""
    q = torch.from_numpy(codes).float()
    g = torch.from_numpy(gi).long()
    s, z = scales.float()[:, g], zeros.float()[:, g]
    xf = x.float()
    acc = torch.zeros(x.shape[0], codes.shape[0])
    for k0 in range(0, x.shape[1], 32):
        sl = slice(k0, k0 + 32)
        t = xf[:, sl] @ (q[:, sl] + off).T - xf[:, sl].sum(1, keepdim=True) * (z[:, k0] + off)[None, :]
        acc = acc + t * s[:, k0][None, :]
    if bias is not None:
        acc = acc + bias.float()
    return acc.to(x.dtype)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("M,N,K,gs", [(1, 37, 4096, 128), (16, 64, 4096, 128), (3, 96, 1024, 32)])
@pytest.mark.parametrize("form", [_rounded, _folded])
def test_correct_outputs_pass_and_planted_code_is_caught(xdt, bits, M, N, K, gs, form):
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + bits, xdt)
    gi = np.arange(K) // gs
    bias = torch.randn(N, generator=torch.Generator().manual_seed(bits)).to(xdt)
    y = form(x, codes, scales, zeros, gi, bias)
    assert check_linear(y, x, codes, scales, zeros, gi, bias, bits=bits) <= 1.0


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_wrong_outputs_fail(xdt):
    M, N, K, gs, bits = 4, 64, 4096, 128, 4
    codes, scales, zeros, x = _case(M, N, K, bits, gs, 5, xdt)
    gi = np.arange(K) // gs
    # one code off by one step where |x| * s is largest
    xs = x.double().abs().max(0).values.numpy()
    n, k = divmod(int(np.argmax(scales.double().numpy()[:, gi] * xs[None, :])), K)
    bad = codes.copy()
    bad[n, k] = bad[n, k] + 1 if bad[n, k] < 15 else bad[n, k] - 1
    if xdt == torch.float16:  # a one-step error is below bf16's output rounding
        with pytest.raises(Violation):
            check_linear(_rounded(x, bad, scales, zeros, gi, None), x, codes, scales, zeros, gi, plant=False)
    # one row's codes shifted by one column (a dropped code)
    bad = codes.copy()
    bad[7] = np.roll(bad[7], 1)
    with pytest.raises(Violation):
        check_linear(_rounded(x, bad, scales, zeros, gi, None), x, codes, scales, zeros, gi, plant=False)
    # one group's scale taken from the next group
    s2 = scales.clone()
    s2[3, 5] = scales[3, 6]
    with pytest.raises(Violation):
        check_linear(_folded(x, codes, s2, zeros, gi, None), x, codes, scales, zeros, gi, plant=False)
