"""gptq_linear_perm_noalloc (no workspace, a static per-GPU scratch array)
against gptq_linear_perm (caller workspace), through the C ABI: identical
outputs on two calls in a row, the second smaller, and sizes beyond the
scratch refused before anything runs."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import gptq_oracle as O

pytestmark = pytest.mark.gpu


def _call_noalloc(lib, x, perm, packed, bits, scales, zeros, gs, bias, N, K, y):
    from distributed_gptq_amd import _ops
    P = ctypes.c_void_p
    return lib.gptq_linear_perm_noalloc(
        P(x.data_ptr()), _ops.dtype_code(x.dtype), x.shape[0], P(perm.data_ptr()), P(packed.data_ptr()), bits,
        P(scales.data_ptr()), P(zeros.data_ptr()), _ops.dtype_code(scales.dtype), None, gs, scales.shape[1],
        P(bias.data_ptr()) if bias is not None else None, _ops.dtype_code(bias.dtype) if bias is not None else 0,
        N, K, P(y.data_ptr()), P(torch.cuda.current_stream().cuda_stream))


def _case(M, N, K, bits, gs, seed, xdt):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, K // gs))).half().cuda()
    zeros = torch.from_numpy(rng.integers(0, 2 ** bits, (N, K // gs)).astype(np.float64)).half().cuda()
    perm = torch.from_numpy(rng.permutation(K).astype(np.int32)).cuda()
    x = torch.from_numpy(rng.standard_normal((M, K))).to(xdt).cuda()
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    bias = torch.from_numpy(rng.standard_normal(N)).to(xdt).cuda()
    return x, perm, packed, scales, zeros, bias


def _call_perm(lib, x, perm, packed, bits, scales, zeros, gs, bias, N, K, y):
    from distributed_gptq_amd import _ops
    P = ctypes.c_void_p
    nb = lib.gptq_linear_perm_workspace_size(x.shape[0], K, _ops.dtype_code(x.dtype))
    ws = torch.empty(nb, dtype=torch.uint8, device=x.device)
    return lib.gptq_linear_perm(
        P(x.data_ptr()), _ops.dtype_code(x.dtype), x.shape[0], P(perm.data_ptr()), P(packed.data_ptr()), bits,
        P(scales.data_ptr()), P(zeros.data_ptr()), _ops.dtype_code(scales.dtype), None, gs, scales.shape[1],
        P(bias.data_ptr()) if bias is not None else None, _ops.dtype_code(bias.dtype) if bias is not None else 0,
        N, K, P(y.data_ptr()), P(ws.data_ptr()), nb, P(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(hip, xdt):
    from distributed_gptq_amd import _lib
    lib = _lib.lib()
    assert lib.gptq_linear_perm_noalloc_max_bytes() == 4 << 20
    # two calls in a row, the second with a smaller input, then M = 1 (the
    # fused-gather GEMV, no scratch) and M = 16 again
    for M, N, K, bits in [(128, 4096, 4096, 4), (16, 1000, 1024, 3), (1, 2048, 4096, 4), (16, 4101, 4096, 4)]:
        x, perm, packed, scales, zeros, bias = _case(M, N, K, bits, 128, M + N, xdt)
        ref = torch.empty(M, N, dtype=xdt, device="cuda")
        assert _call_perm(lib, x, perm, packed, bits, scales, zeros, 128, bias, N, K, ref) == 0
        y = torch.empty(M, N, dtype=xdt, device="cuda")
        assert _call_noalloc(lib, x, perm, packed, bits, scales, zeros, 128, bias, N, K, y) == 0
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (M, N, K)


def test_noalloc_refuses_sizes_beyond_the_scratch(hip):
    from distributed_gptq_amd import _lib
    lib = _lib.lib()
    M, N, K = 1024, 256, 4096  # 8 MiB of fp16 activations > 4 MiB
    x, perm, packed, scales, zeros, bias = _case(M, N, K, 4, 128, 1, torch.float16)
    y = torch.zeros(M, N, dtype=torch.float16, device="cuda")
    rc = _call_noalloc(lib, x, perm, packed, 4, scales, zeros, 128, None, N, K, y)
    assert rc == _lib.ERR_WORKSPACE
    assert b"limit" in lib.gptq_last_error()
    torch.cuda.synchronize()
    assert not y.any()
