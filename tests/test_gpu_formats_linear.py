"""GPU parity of the packing formats (bit-exact), dequantisation (bit-exact
fp32) and the dequant GEMV/GEMM behind gptq::linear (fp32 accumulation;
every output element within half an output ulp plus the fp32 dot-product
bound of the fp64 oracle, and a planted wrong code caught: tests/linear_check.py)."""
import numpy as np
import pytest
import torch

from oracle import gptq_oracle as O
from tests.linear_check import check_linear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("N,K", [(5, 7), (16, 256), (33, 1000)])
def test_pack_unpack_bit_exact(hip, bits, N, K):
    from distributed_gptq_amd import _ops
    rng = np.random.default_rng(bits * K)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    p = _ops.pack(torch.from_numpy(codes).cuda(), bits)
    np.testing.assert_array_equal(p.cpu().numpy(), O.pack_bitstream(codes, bits))
    np.testing.assert_array_equal(_ops.unpack(p, bits, K).cpu().numpy(), codes)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_reference_layout_bit_exact(hip, bits):
    from distributed_gptq_amd import _ops
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 2 ** bits, (64, 40)).astype(np.uint8)
    out = _ops.pack_reference_layout(torch.from_numpy(codes).cuda(), bits).cpu().numpy()
    np.testing.assert_array_equal(out, O.ref_pack_weights(codes, bits))


@pytest.mark.parametrize("bits", [0, 2, 3, 4, 8])
@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_dequant_bit_exact(hip, bits, sdt):
    from distributed_gptq_amd import _ops
    rng = np.random.default_rng(bits + 10)
    N, K, gs = 24, 384, 128
    eb = 8 if bits == 0 else bits
    codes = rng.integers(0, 2 ** eb, (N, K)).astype(np.uint8)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, 3))).to(sdt)
    zeros = torch.from_numpy(rng.integers(0, 2 ** eb, (N, 3)).astype(np.float64) + 0.25).to(sdt)
    packed = codes if bits == 0 else O.pack_bitstream(codes, bits)
    out = _ops.dequant(torch.from_numpy(packed).cuda(), bits, scales.cuda(), zeros.cuda(), K, group_size=gs)
    ref = O.dequant(codes, scales.float().numpy(), zeros.float().numpy(), np.arange(K) // gs)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    # the reference's own formula in torch: (w - zeros) * scales on fp32
    w = torch.from_numpy(codes).float()
    tref = (w - zeros.repeat_interleave(gs, 1).float()) * scales.repeat_interleave(gs, 1).float()
    assert torch.equal(out.cpu(), tref)


@pytest.mark.parametrize("bits", [0, 2, 3, 4, 8])
@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K,gs,gidx", [(384, 128, False), (1024, 32, False), (200, 64, False), (256, 128, True)])
def test_dequant_typed_bit_exact(hip, bits, odt, K, gs, gidx):
    """Dequantised weights in fp16 / bf16 / fp32: the fp32 value rounded once
    (torch's own rounding), on the 32-code chunk kernel (K % 32 == 0, groups
    of a multiple of 32) and the per-element one (K = 200, g_idx)."""
    from distributed_gptq_amd import _ops
    rng = np.random.default_rng(bits + K)
    N = 40
    eb = 8 if bits == 0 else bits
    ng = -(-K // gs)
    codes = rng.integers(0, 2 ** eb, (N, K)).astype(np.uint8)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, ng))).half()
    zeros = torch.from_numpy(rng.integers(0, 2 ** eb, (N, ng)).astype(np.float64) + 0.5).half()
    g_idx = rng.permutation(np.arange(K) // gs) if gidx else np.arange(K) // gs
    packed = codes if bits == 0 else O.pack_bitstream(codes, bits)
    out = _ops.dequant(torch.from_numpy(packed).cuda(), bits, scales.cuda(), zeros.cuda(), K,
                       g_idx=torch.from_numpy(g_idx).cuda() if gidx else None, group_size=gs, dtype=odt)
    assert out.dtype == odt
    ref = torch.from_numpy(O.dequant(codes, scales.float().numpy(), zeros.float().numpy(), g_idx)).to(odt)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,actorder", [(384, 96, True), (400, 1024, True), (2048, 640, False),
                                          (3, 1024, True)])
def test_quantized_linear_many_rows(hip, xdt, M, N, actorder):
    """From DEQUANT_GEMM_ROWS rows of x the operator dequantises the weights
    to x's dtype once and runs the library GEMM (act-order: x's columns
    gathered when it has fewer rows than W, W's columns scattered otherwise);
    both agree with the oracle, and with the fused kernels below the
    threshold."""
    from distributed_gptq_amd.models import layers as Lm
    K, gs, bits = 512, 128, 4
    rng = np.random.default_rng(M + N)
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    perm = rng.permutation(K) if actorder else np.arange(K)
    g_idx = np.empty(K, np.int64)
    g_idx[perm] = np.arange(K) // gs  # column perm[j] sits at sweep position j
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, K // gs))).half()
    zeros = torch.from_numpy(rng.integers(0, 16, (N, K // gs)).astype(np.float64)).half()
    ql = Lm.QuantizedLinear(bits, gs, K, N, bias=True, packed=True).cuda()
    ql.pack_weights(torch.from_numpy(codes).cuda(), scales.cuda(), zeros.cuda(), torch.from_numpy(g_idx).int().cuda(),
                    perm=torch.from_numpy(perm).int().cuda() if actorder else None)
    assert ql.perm.numel() == (K if actorder else 0)
    with torch.no_grad():
        ql.bias.copy_(torch.randn(N))
    x = torch.randn(M, K, device="cuda").to(xdt)
    with torch.no_grad():
        y = ql(x)
    assert y.dtype == xdt and y.shape == (M, N)
    check_linear(y, x, codes, scales, zeros, g_idx, ql.bias, bits=bits)


def _case(M, N, K, bits, gs, seed, xdt):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    ng = -(-K // gs)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, ng))).half()
    zeros = torch.from_numpy(rng.integers(0, 2 ** bits, (N, ng)).astype(np.float64)).half()
    x = torch.from_numpy(rng.standard_normal((M, K))).to(xdt)
    return codes, scales, zeros, x


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("M", [1, 3, 16, 40, 128])
def test_linear_fast_paths(hip, xdt, bits, M):
    from distributed_gptq_amd import _ops
    N, K, gs = 96, 1024, 128
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M * 10 + bits, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda())
    assert y.dtype == xdt and y.shape == (M, N)
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("K,gs", [(1024, 128), (4096, 128), (6144, 64), (14336, 128), (20480, 32)])
def test_linear_m1_gemv(hip, xdt, bits, K, gs):
    """M = 1 kernel in each regime: one or two chunks per lane, and the
    four-wave split of long rows."""
    from distributed_gptq_amd import _ops
    N = 37
    codes, scales, zeros, x = _case(1, N, K, bits, gs, K + bits, xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs)
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("N,K", [(8192 + 37, 4096), (4096 + 5, 14336), (1024 + 3, 20480)])
def test_linear_m1_many_rows(hip, xdt, bits, N, K):
    """M = 1 with more rows than one pass of the grid covers, so every wave
    walks several double-buffered batches; a ragged last batch, a bias, and
    scales/zeros in the activation dtype."""
    from distributed_gptq_amd import _ops
    gs = 128
    codes, scales, zeros, x = _case(1, N, K, bits, gs, N + bits, xdt)
    scales, zeros = scales.to(xdt), zeros.to(xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda())
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_linear_generic_path_gidx_and_fp32(hip, xdt):
    """act-order g_idx gather and fp32 activations take the generic kernel."""
    from distributed_gptq_amd import _ops
    N, K, gs = 40, 200, 50
    codes, scales, zeros, x = _case(5, N, K, 4, gs, 3, xdt)
    g_idx = np.random.default_rng(0).permutation(np.arange(K) // gs).astype(np.int32)
    packed = torch.from_numpy(O.pack_bitstream(codes, 4)).cuda()
    y = _ops.linear(x.cuda(), packed, 4, scales.cuda(), zeros.cuda(), K, g_idx=torch.from_numpy(g_idx).cuda())
    check_linear(y, x, codes, scales, zeros, g_idx, bits=4)


def test_quantized_linear_op(hip):
    from distributed_gptq_amd.models.layers import QuantizedLinear
    N, K, gs = 64, 512, 128
    codes, scales, zeros, x = _case(2, N, K, 4, gs, 9, torch.float16)
    ql = QuantizedLinear(4, gs, K, N, bias=True).cuda()
    ql.pack_weights(torch.from_numpy(codes).cuda(), scales.cuda(), zeros.cuda())
    ql.bias.data = torch.randn(N, device="cuda")
    assert ql.qweight.shape == (N, K // 2)
    # packed buffer is the reference's byte layout (models/layers.py:85-89)
    np.testing.assert_array_equal(ql.qweight.cpu().numpy(), O.pack_bitstream(codes, 4))
    Wd = ql.unpack_weights()
    np.testing.assert_array_equal(Wd.cpu().numpy(), O.dequant(codes, scales.numpy(), zeros.numpy(),
                                                              np.arange(K) // gs))
    with torch.no_grad():
        y = ql(x.cuda())
        y2 = torch.ops.gptq.linear(x.cuda(), ql.qweight, ql.scales, ql.zeros, ql.g_idx, ql.bias)
    assert torch.equal(y, y2)
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, ql.bias, bits=4)
    # the reference's placeholder g_idx = arange(K) means contiguous groups
    ql.g_idx.data = torch.arange(K, dtype=torch.int32, device="cuda")
    with torch.no_grad():
        assert torch.equal(ql(x.cuda()), y)
    # gradients of F.linear(x, W, b) with the dequantized weight
    xg = x.cuda().float().requires_grad_(True)
    ql.g_idx.data = torch.arange(K, dtype=torch.int32, device="cuda") // gs
    out = ql(xg)
    out.backward(torch.ones_like(out))
    np.testing.assert_allclose(xg.grad.cpu().numpy(), np.tile(Wd.sum(0).cpu().numpy(), (2, 1)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ql.bias.grad.cpu().numpy(), np.full(N, 2.0))


def test_quantized_linear_from_gptq_actorder(hip):
    from distributed_gptq_amd import GPTQ
    from distributed_gptq_amd.models.layers import QuantizedLinear
    torch.manual_seed(2)
    lin = torch.nn.Linear(256, 64).cuda().half()
    X = torch.randn(2, 128, 256, device="cuda").half()
    q = GPTQ(lin, bits=3, group_size=64, actorder=True, device="cuda")
    q.add_batch(X)
    q.fasterquant()
    for packed in (True, False):
        ql = QuantizedLinear.from_gptq(q, packed=packed)
        Wd = ql.unpack_weights()
        # stored codes + fp16 scales/zeros (the reference's buffer dtype) and
        # the act-order g_idx reproduce the dequantized layer weight up to the
        # fp16 rounding of the scales
        np.testing.assert_array_equal(Wd.cpu().numpy(), O.dequant(
            q.qcodes.cpu().numpy(), ql.scales.cpu().numpy(), ql.zeros.cpu().numpy(), q.g_idx.cpu().numpy()))
        np.testing.assert_allclose(Wd.cpu().numpy(), lin.weight.data.float().cpu().numpy(), rtol=2e-3, atol=1e-4)
        with torch.no_grad():
            y = ql(X[0])
        check_linear(y, X[0], q.qcodes.cpu().numpy(), ql.scales, ql.zeros, q.g_idx.cpu().numpy(), ql.bias, bits=3)


def test_tensor_quantize_dequantize(hip):
    from distributed_gptq_amd import kernels
    assert kernels.check_triton_availability()
    x = torch.randn(10, 100)
    q, s, z = kernels.quantize_tensor(x, bits=4, group_size=128)
    xn = x.numpy().reshape(-1)
    for g in range(len(s)):
        seg = xn[g * 128:(g + 1) * 128]
        sg = np.float32((seg.max() - seg.min()) / np.float32(15))
        zg = np.float32(-seg.min() / sg)
        assert s[g].item() == pytest.approx(float(sg), rel=1e-6)
        assert z[g].item() == pytest.approx(float(zg), rel=1e-5, abs=1e-6)
        v = seg / sg + zg
        expect = np.clip(np.floor(np.abs(v) + 0.5) * np.sign(v), 0, 15)  # half away from zero
        np.testing.assert_array_equal(q.cpu().numpy().reshape(-1)[g * 128:(g + 1) * 128], expect)
    d = kernels.dequantize_tensor(q, s, z, 128).cpu()
    gi = np.arange(1000) // 128
    ref = (q.cpu().numpy().reshape(-1).astype(np.float32) - z.cpu().numpy()[gi]) * s.cpu().numpy()[gi]
    np.testing.assert_array_equal(d.numpy().reshape(-1), ref)


def test_triton_quantized_linear(hip):
    from distributed_gptq_amd import kernels
    tl = kernels.TritonQuantizedLinear(256, 32, bits=4, group_size=64)
    w = torch.randn(32, 256) * 0.02
    tl.quantize_weights(w)
    x = torch.randn(3, 256, device="cuda", dtype=torch.float16)
    y = tl.forward(x)
    s = tl.scales.float().cpu().numpy()
    z = tl.zeros.float().cpu().numpy()
    codes = tl.qweight.cpu().numpy().view(np.uint8)
    check_linear(y, x, codes, s, z, np.arange(256) // 64, bits=4)
    # dequantized weights are close to the originals
    Wd = O.dequant(codes, s, z, np.arange(256) // 64)
    assert np.abs(Wd - w.numpy()).max() < 0.02 * 8 / 15 + 1e-3


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("M,N,K,gs", [(16, 4101, 4096, 128), (9, 1000, 1024, 32), (64, 2050, 2048, 128),
                                      (100, 1027, 4096, 64), (128, 4096, 4096, 128),
                                      # tiled kernel: 64-row tiles with 128-column steps (odd step
                                      # count) and with 64-column steps, 128-row tiles
                                      (40, 8200, 512, 128), (128, 8256, 384, 128), (64, 16448, 384, 128),
                                      (100, 16448, 640, 128), (130, 16448, 256, 128), (64, 32832, 256, 128),
                                      # 64 < M <= 128 with 160-191 tiles (5120-row layers)
                                      (96, 5121, 384, 128), (128, 5120, 640, 64),
                                      # split-K with 32-row M tiles; 64 x 64 tiles and split-K for M > 128
                                      (24, 4100, 1024, 128), (32, 1000, 512, 64), (160, 4100, 512, 128),
                                      (200, 2000, 512, 128),
                                      # 112-row register workgroups (250 of them), ragged last one
                                      (5, 27900, 1024, 64), (16, 27904, 512, 128)])
def test_linear_dequant_gemm(hip, xdt, bits, M, N, K, gs):
    """M > 4: dequantise-then-MFMA kernels (split-K and tiled), ragged N and M,
    groups of 32-128 (one group per 32-code chunk), bias; through
    gptq_linear_ws (_ops.linear) and through gptq_linear, which has no
    workspace and so runs these kernels where the other takes the split
    register-decoded one."""
    from distributed_gptq_amd import _ops
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + bits, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    args = (x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K)
    for y in (_ops.linear(*args, group_size=gs, bias=bias.cuda()), _linear_plain(*args, gs, bias.cuda())):
        check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


def _linear_plain(x, packed, bits, scales, zeros, K, gs, bias):
    """gptq_linear through the C ABI (no workspace)."""
    from distributed_gptq_amd import _lib, _ops
    M, N = x.shape[0], scales.shape[0]
    y = torch.empty(M, N, dtype=x.dtype, device=x.device)
    _lib.call("gptq_linear", x.data_ptr(), _ops.dtype_code(x.dtype), M, packed.data_ptr(), bits, scales.data_ptr(),
              zeros.data_ptr(), _ops.dtype_code(scales.dtype), None, gs, scales.shape[1], bias.data_ptr(),
              _ops.dtype_code(bias.dtype), N, K, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return y


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("M,N,K,gs,zkind,sdt", [
    (128, 24576, 512, 128, "int", torch.float16),
    # ragged last workgroup (N % 128 = 4) and block count below the code slots
    (100, 24580, 384, 64, "int", torch.float16),
    # N % 4 != 0 (element stores), groups of 32 (a lane's chunk in its own group)
    (65, 24578, 256, 32, "int", torch.float16),
    # zeros that are not integers (the fp32 decode for fp16 activations) and fp32 scales
    (128, 24576, 640, 128, "frac", torch.float16),
    (128, 24576, 1152, 128, "int", torch.float32),
    # 64- and 32-row activation tiles
    (64, 24576, 512, 128, "frac", torch.float16),
    (33, 24580, 384, 64, "int", torch.float16),
    (32, 24576, 768, 128, "int", torch.float32),
    (20, 24578, 1024, 32, "int", torch.float16),
    # more than 256 workgroups of 112 rows: 8 compute waves of 16 rows
    (128, 28800, 256, 128, "int", torch.float16),
    (40, 32772, 384, 64, "frac", torch.float16),
    (17, 28804, 256, 32, "int", torch.float16),
    # two activation tiles: more than 256 workgroups, 7 waves
    (192, 24576, 256, 128, "int", torch.float16),
    (300, 16448, 384, 64, "frac", torch.float16),
    # 16385-24448 rows: unsplit on 7 waves (fewer than 192 workgroups of 128 rows)
    (128, 20480, 256, 128, "int", torch.float16),
    (40, 17410, 384, 64, "frac", torch.float16),
    (20, 22018, 1024, 32, "int", torch.float32)])
def test_linear_register_decoded_wide(hip, xdt, bits, M, N, K, gs, zkind, sdt):
    """16 < M <= 128 on layers of more than 16384 rows, unsplit (7 compute
    waves of 16 rows up to 256 x 112 rows, 8 beyond): the kernel that decodes
    the codes in registers (loader waves stage X), against the fp64 oracle."""
    from distributed_gptq_amd import _ops
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + bits + K, xdt)
    if zkind == "frac":
        rng = np.random.default_rng(N + K)
        zeros = torch.from_numpy(rng.uniform(0, 2 ** bits - 1, zeros.shape)).half()
    scales, zeros = scales.to(sdt), zeros.to(sdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda())
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("M,N,K,gs,zkind,sdt,act", [
    # 32 workgroups x 8 splits of 4 blocks
    (128, 4096, 4096, 128, "int", torch.float16, False),
    # ragged splits (11 blocks over 6 splits, the last one block), groups of 64
    (100, 5120, 1408, 64, "int", torch.float16, False),
    # one block per split, ragged last workgroup (N % 128 = 4), groups of 32
    (65, 1028, 640, 32, "int", torch.float16, False),
    # two splits; fractional zeros, fp32 scales; with act-order gather in front
    (128, 14336, 1024, 128, "frac", torch.float32, True),
    (96, 2048, 2048, 128, "int", torch.float16, True),
    # 64- and 32-row activation tiles (16 < M <= 64), ragged M
    (64, 4096, 1024, 128, "int", torch.float16, False),
    (50, 5120, 1408, 64, "frac", torch.float16, True),
    (32, 2048, 8320, 128, "int", torch.float32, False),
    (17, 1028, 17408, 32, "int", torch.float16, True),
    # M > 128: two or three 128-row activation tiles per workgroup column
    (256, 4096, 1024, 128, "int", torch.float16, False),
    (384, 4096, 512, 64, "frac", torch.float16, True),
    (150, 2052, 1024, 32, "int", torch.float32, False),
    # a few output rows: one workgroup column, most of its weight rows past N
    (100, 8, 1024, 128, "int", torch.float16, False),
    (65, 4, 2048, 64, "int", torch.float16, True)])
def test_linear_register_decoded_split_k(hip, xdt, bits, M, N, K, gs, zkind, sdt, act):
    """16 < M <= 384 on layers too narrow to fill the GPU unsplit: the register-decoded
    kernel with K split over workgroups (fp32 partials in the workspace,
    reduced in split order, bias added there), against the fp64 oracle;
    the same call twice gives identical bits."""
    from distributed_gptq_amd import _lib, _ops
    nb = _lib.lib().gptq_linear_workspace_size(M, N, K, bits, gs, _ops.dtype_code(xdt), int(act))
    assert nb >= 2 * M * N * 4  # the split path is the one under test
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + bits + K, xdt)
    if zkind == "frac":
        rng = np.random.default_rng(N + K)
        zeros = torch.from_numpy(rng.uniform(0, 2 ** bits - 1, zeros.shape)).half()
    scales, zeros = scales.to(sdt), zeros.to(sdt)
    bias = torch.randn(N).to(xdt)
    perm = torch.from_numpy(np.random.default_rng(K).permutation(K).astype(np.int32)) if act else None
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    args = (x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K)
    kw = dict(group_size=gs, bias=bias.cuda(), perm=perm.cuda() if act else None)
    y = _ops.linear(*args, **kw)
    assert torch.equal(y, _ops.linear(*args, **kw))
    xr = x[:, perm.long()] if act else x
    check_linear(y, xr, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("M,N,K,gs", [
    (16, 5120, 13824, 128),   # 32-row workgroups, K in 3 ranges
    (5, 5000, 8192, 64),      # ragged last workgroup, groups of 64 (per-weight dequantisation)
    (9, 6144, 4096, 128),     # unsplit (K < 8192)
    (12, 5122, 8320, 128),    # N % 4 != 0: unsplit
    (2, 5120, 8192, 128), (3, 6148, 4096, 64),
    # 8192 rows: 64-row workgroups, K in 2 ranges
    (16, 8192, 1024, 128), (4, 8192, 640, 64)])
def test_linear_register_mid_rows(hip, xdt, bits, M, N, K, gs):
    """1 < M <= 16 on layers of 4097-8191 rows: dq_reg4_k with 32-row
    workgroups, split over K (partials reduced in order, bias added there)
    when K >= 8192 and the workspace holds the partials; on 8192 rows
    64-row workgroups with K split in 2; through
    gptq_linear_ws and, unsplit, through gptq_linear; against the fp64
    oracle."""
    from distributed_gptq_amd import _lib, _ops
    nb = _lib.lib().gptq_linear_workspace_size(M, N, K, bits, gs, _ops.dtype_code(xdt), 0)
    assert nb == (2 * M * N * 4 if N == 8192 else 3 * M * N * 4 if K >= 8192 and N % 4 == 0 else 0)
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + K + bits, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    args = (x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K)
    y = _ops.linear(*args, group_size=gs, bias=bias.cuda())
    assert torch.equal(y, _ops.linear(*args, group_size=gs, bias=bias.cuda()))
    for out in (y, _linear_plain(*args, gs, bias.cuda())):
        check_linear(out, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("M,N,K,gs,split", [
    (16, 4096, 14336, 128, True),    # 128 workgroups of 32 rows x 2 K ranges
    (9, 4092, 10240, 128, True),     # M, K at their bounds; last workgroup of 28 rows
    (12, 3072, 11008, 128, True),    # 86 blocks in two ranges of 43
    (8, 4096, 14336, 128, False),    # M <= 8: 16-wave workgroups, unsplit
    (16, 4096, 8192, 128, False),    # K < 10240: 16 waves, unsplit
    (16, 2048, 14336, 128, False),   # < 3072 rows: 8 waves, unsplit
    (14, 4094, 14336, 128, False),   # N % 4 != 0: 8 waves, unsplit
    (6, 4000, 4096, 64, False)])     # groups of 64 (per-weight dequantisation), 16 waves
def test_linear_register_narrow_rows(hip, xdt, bits, M, N, K, gs, split):
    """1 < M <= 16 on layers of <= 4096 rows: 16-row workgroups of 16 waves
    over K, or of 8 waves for 8 < M <= 16 with K >= 10240; on 3072-4096 rows
    with 8 < M <= 16 and K >= 10240, 32-row workgroups of 16 waves with K in
    2 ranges (partials reduced in order, bias added there) when the workspace
    holds the partials, else the 8-wave workgroups.  Through gptq_linear_ws and
    gptq_linear (no workspace), against the fp64 oracle; repeated calls are
    bit-identical."""
    from distributed_gptq_amd import _lib, _ops
    nb = _lib.lib().gptq_linear_workspace_size(M, N, K, bits, gs, _ops.dtype_code(xdt), 0)
    assert nb == (2 * M * N * 4 if split else 0)
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + K + bits + 7, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    args = (x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K)
    y = _ops.linear(*args, group_size=gs, bias=bias.cuda())
    assert torch.equal(y, _ops.linear(*args, group_size=gs, bias=bias.cuda()))
    for out in (y, _linear_plain(*args, gs, bias.cuda())):
        check_linear(out, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


def test_linear_ws_workspace_alignment_and_size(hip):
    """gptq_linear_ws with a workspace that starts 4 bytes past a 256-byte
    boundary: the partial sums start at the next boundary, so the exact size
    no longer fits and the layer runs unsplit (still correct); 256 bytes more
    give the split result bit for bit.  No workspace at all runs unsplit."""
    from distributed_gptq_amd import _lib, _ops
    M, N, K, gs, bits, xdt = 128, 4096, 1024, 128, 4, torch.float16
    codes, scales, zeros, x = _case(M, N, K, bits, gs, 11, xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    xc, sc, zc = x.cuda(), scales.cuda(), zeros.cuda()
    nb = _lib.lib().gptq_linear_workspace_size(M, N, K, bits, gs, _ops.dtype_code(xdt), 0)
    assert nb == 8 * M * N * 4
    buf = torch.empty(nb + 1024, dtype=torch.uint8, device="cuda")
    assert buf.data_ptr() % 256 == 0

    def run(ws_ptr, ws_bytes):
        y = torch.empty(M, N, dtype=xdt, device="cuda")
        _lib.call("gptq_linear_ws", xc.data_ptr(), _ops.dtype_code(xdt), M, None, packed.data_ptr(), bits,
                  sc.data_ptr(), zc.data_ptr(), _ops.dtype_code(sc.dtype), None, gs, sc.shape[1], None, 0, N, K,
                  y.data_ptr(), ws_ptr, ws_bytes, torch.cuda.current_stream().cuda_stream)
        return y

    split = run(buf.data_ptr(), nb)
    assert torch.equal(split, _ops.linear(xc, packed, bits, sc, zc, K, group_size=gs))
    assert torch.equal(run(buf.data_ptr() + 4, nb + 256), split)
    for y in (run(buf.data_ptr() + 4, nb), run(None, 0)):
        check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N", [(1, 1030), (3, 1030), (16, 4101), (128, 8256)])
def test_linear_scales_at_odd_offset(hip, xdt, M, N):
    """Scales and zeros whose base is 2 but not 4-byte aligned (a contiguous
    view one element into its storage): the kernels read the aligned word
    holding each 16-bit element and must give exactly the aligned result."""
    from distributed_gptq_amd import _ops
    K, gs, bits = 1024, 128, 4
    codes, scales, zeros, x = _case(M, N, K, bits, gs, 7 + M, xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    s_al, z_al = scales.cuda(), zeros.cuda()
    s_buf = torch.zeros(scales.numel() + 1, dtype=scales.dtype, device="cuda")
    z_buf = torch.zeros(zeros.numel() + 1, dtype=zeros.dtype, device="cuda")
    s_odd, z_odd = s_buf[1:].view(scales.shape), z_buf[1:].view(zeros.shape)
    s_odd.copy_(s_al)
    z_odd.copy_(z_al)
    assert s_odd.data_ptr() % 4 == 2 and z_odd.data_ptr() % 4 == 2
    xc = x.cuda()
    y_al = _ops.linear(xc, packed, bits, s_al, z_al, K, group_size=gs)
    y_odd = _ops.linear(xc, packed, bits, s_odd, z_odd, K, group_size=gs)
    assert torch.equal(y_al, y_odd)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("gs", [128, 32])
@pytest.mark.parametrize("M,N", [(2, 8192 + 37), (4, 8192 + 37), (16, 8192 + 37), (3, 14336 - 20),
                                 (2, 16384 + 5), (4, 16384 + 5), (16, 16384 + 5)])
def test_linear_small_m_wide_n(hip, xdt, bits, gs, M, N):
    """M <= 16 with N >= 8192 and >= 16384: the register kernels (3/4-bit:
    dq_reg4_k with 64-row workgroups of 8 and 4 waves, and 32-row ones for
    M <= 4 below 16384 rows) and the wide split-K kernels (2/8-bit), ragged
    N (the last tile's clamp), with groups of 128 (zero points folded per
    block) and 32 (dequantised per weight)."""
    from distributed_gptq_amd import _ops
    K = 1024
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + bits + gs, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda())
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


@pytest.mark.parametrize("M,N,K,gs,bits,xdt", [
    (16, 28672 - 37, 4096, 128, 4, torch.float16),
    (5, 28672 - 37, 4096, 256, 3, torch.bfloat16),
    (2, 26881, 1024, 128, 4, torch.bfloat16),
    (16, 26881, 2048, 128, 3, torch.float16),
    (11, 28672, 1024, 256, 4, torch.float16),
    (16, 28672, 4096, 128, 3, torch.bfloat16),
    (1, 28672 - 37, 4096, 128, 4, torch.bfloat16),
])
def test_linear_row16(hip, M, N, K, gs, bits, xdt):
    """The 241-256-workgroup class of M <= 16 (dq_row16_k: 7 waves of 16 rows
    over all of K, X staged once per workgroup): ragged N (a last workgroup
    of 75 rows, and of 1 row at N = 26881), K of 1024-4096 (8-32 blocks
    through a ring of 4 slots), groups of 128 and 256 columns, M below 16
    (rows of X past M zero in LDS), bias, 3/4-bit, fp16/bf16.  The M = 1
    case takes the M = 1 GEMV at the same shape, the others dq_row16_k."""
    from distributed_gptq_amd import _ops
    codes, scales, zeros, x = _case(M, N, K, bits, gs, M + N + K + bits, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda())
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bias, bits=bits)


_C4 = {}


def _c4_weights(N, K, bits):
    """Config 4's weights (codes uniform, scales U(1e-3, 1e-2), zeros
    2^(bits-1), fp16), one shape cached."""
    key = (N, K, bits)
    if key not in _C4:
        _C4.clear()
        rng = np.random.default_rng(3)
        codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
        ng = K // 128
        scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, ng))).half()
        zeros = torch.full((N, ng), float(2 ** (bits - 1))).half()
        packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
        _C4[key] = (packed, scales, zeros, codes)
    return _C4[key]


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 3, 16, 64, 128])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("N,K", [(4096, 4096), (14336, 4096), (4096, 14336), (28672, 4096)])
def test_linear_config4_shapes(hip, xdt, M, bits, N, K):
    """Every kernel the bench's W4A16 / W3A16 rows run, at their shapes."""
    from distributed_gptq_amd import _ops
    packed, scales, zeros, codes = _c4_weights(N, K, bits)
    g = torch.Generator().manual_seed(M + bits)
    x = torch.randn(M, K, generator=g).to(xdt)
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=128)
    check_linear(y, x, codes, scales, zeros, np.arange(K) // 128, bits=bits)


def test_release_config4_cache(hip):
    _C4.clear()


# ------------------------------------------------ act-order serving layout --

def _actorder_case(M, N, K, bits, gs, seed, xdt):
    """Codes in input-column order with an act-order g_idx (groups of gs in a
    random column order), and the storage the serving layout uses: columns
    in perm order, perm = the stable sort of g_idx."""
    codes, scales, zeros, x = _case(M, N, K, bits, gs, seed, xdt)
    rng = np.random.default_rng(seed + 1)
    perm = rng.permutation(K).astype(np.int32)          # sweep order
    g_idx = np.empty(K, np.int32)
    g_idx[perm] = np.arange(K) // gs                    # group of input column k
    stored = codes[:, perm]
    return codes, stored, scales, zeros, x, g_idx, perm


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [3, 4, 8])
@pytest.mark.parametrize("M,N,K", [(1, 1000, 4096), (1, 37, 14336), (2, 8229, 1024), (16, 4101, 4096),
                                   (16, 16389, 1024), (128, 4096, 4096), (40, 1000, 1024)])
def test_linear_perm_matches_oracle(hip, xdt, bits, M, N, K):
    """gptq_linear_perm: the M = 1 GEMV with x gathered in the kernel, other
    M on the fast kernels after the gather; against the oracle on the
    input-order codes and act-order g_idx, at the fast path's tolerance."""
    from distributed_gptq_amd import _ops
    gs = 128
    codes, stored, scales, zeros, x, g_idx, perm = _actorder_case(M, N, K, bits, gs, M + N + bits, xdt)
    bias = torch.randn(N).to(xdt)
    packed = torch.from_numpy(O.pack_bitstream(stored, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs, bias=bias.cuda(),
                    perm=torch.from_numpy(perm).cuda())
    check_linear(y, x, codes, scales, zeros, g_idx, bias, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits,gs", [(4, 128), (3, 128), (8, 64), (2, 32)])
@pytest.mark.parametrize("N,K", [(1000, 4096), (300, 14336), (4100, 1024), (64, 32768)])
def test_linear_perm_m1_equals_pregathered_x(hip, xdt, bits, gs, N, K):
    """M = 1 with perm (x gathered through perm, then the GEMV): the result
    equals, bit for bit, the GEMV on x gathered beforehand, and the oracle
    within the fast path's tolerance."""
    from distributed_gptq_amd import _ops
    codes, scales, zeros, x = _case(1, N, K, bits, gs, N + K + bits, xdt)
    perm = np.random.default_rng(K + bits).permutation(K).astype(np.int32)
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    xc, sc, zc, pc = x.cuda(), scales.cuda(), zeros.cuda(), torch.from_numpy(perm).cuda()
    y = _ops.linear(xc, packed, bits, sc, zc, K, group_size=gs, perm=pc)
    y_pre = _ops.linear(xc[:, pc.long()].contiguous(), packed, bits, sc, zc, K, group_size=gs)
    assert torch.equal(y, y_pre)
    check_linear(y, x[:, torch.from_numpy(perm).long()], codes, scales, zeros, np.arange(K) // gs, bits=bits)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K,gs", [(200, 50), (204, 51), (1003, 59)])
def test_linear_perm_generic_and_fp32(hip, xdt, K, gs):
    """perm with layouts the fast kernels do not take (fp32 x; a g_idx that
    stays out of order in the stored order; K not a multiple of 8, where the
    gather writes element by element): gather, then the generic kernel."""
    from distributed_gptq_amd import _ops
    N = 40
    codes, scales, zeros, x = _case(5, N, K, 4, gs, 3, xdt)
    rng = np.random.default_rng(1)
    perm = rng.permutation(K).astype(np.int32)
    g_idx = rng.permutation(np.arange(K) // gs).astype(np.int32)   # group of input column k
    stored = codes[:, perm]
    packed = torch.from_numpy(O.pack_bitstream(stored, 4)).cuda()
    y = _ops.linear(x.cuda(), packed, 4, scales.cuda(), zeros.cuda(), K,
                    g_idx=torch.from_numpy(g_idx[perm]).cuda(), perm=torch.from_numpy(perm).cuda())
    check_linear(y, x, codes, scales, zeros, g_idx, bits=4)


@pytest.mark.parametrize("bits,gs,M", [(4, 128, 1), (4, 128, 7), (3, 64, 1), (8, 128, 16), (2, 32, 1)])
def test_quantized_linear_actorder_is_served_fast(hip, bits, gs, M):
    """GPTQ act-order output in a QuantizedLinear: stored in sweep order with
    perm, the operator takes the contiguous-group kernels (no per-weight
    group gather), outputs match the oracle on the input-order codes, the
    dequantised weight equals the layer's, gradients flow, and the state
    dict round-trips (a model without perm loads too)."""
    from distributed_gptq_amd import GPTQ
    from distributed_gptq_amd.models import layers as Lm
    torch.manual_seed(bits + gs)
    K, N = 512, 96
    lin = torch.nn.Linear(K, N).cuda().half()
    X = torch.randn(2, 128, K, device="cuda").half()
    X[..., :5] *= 10
    q = GPTQ(lin, bits=bits, group_size=gs, actorder=True, device="cuda")
    q.add_batch(X)
    q.fasterquant()
    ql = Lm.QuantizedLinear.from_gptq(q)
    # stored in the canonical act-order layout: the stable sort of g_idx, which
    # holds GPTQ's groups (the sweep order's) with input columns ascending in each
    assert ql.perm.numel() == K and torch.equal(ql.perm, torch.argsort(q.g_idx, stable=True).to(torch.int32))
    assert torch.equal(q.g_idx[ql.perm.long()], torch.arange(K, device="cuda", dtype=torch.int32) // gs)
    assert Lm._group_layout(ql.g_idx, K, ql.num_groups, ql.perm) == (gs, None)
    Wd = ql.unpack_weights()
    np.testing.assert_array_equal(Wd.cpu().numpy(), O.dequant(
        q.qcodes.cpu().numpy(), ql.scales.cpu().numpy(), ql.zeros.cpu().numpy(), q.g_idx.cpu().numpy()))
    x = torch.randn(M, K, device="cuda").half()
    with torch.no_grad():
        y = ql(x)
    check_linear(y, x, q.qcodes.cpu().numpy(), ql.scales, ql.zeros, q.g_idx.cpu().numpy(), ql.bias, bits=bits)
    # gradients of F.linear(x, unpack_weights(), bias)
    xg = x.float().requires_grad_(True)
    out = ql(xg)
    out.backward(torch.ones_like(out))
    np.testing.assert_allclose(xg.grad.cpu().numpy(), np.tile(Wd.sum(0).cpu().numpy(), (M, 1)), rtol=1e-4,
                               atol=1e-5)
    # state dict round trip into a fresh layer, and a perm-less (reference) one
    fresh = Lm.QuantizedLinear(bits, gs, K, N, bias=True, packed=True).cuda()
    fresh.load_state_dict(ql.state_dict())
    with torch.no_grad():
        assert torch.equal(fresh(x), y)
    plain = Lm.QuantizedLinear.from_gptq(q)
    plain.pack_weights(q.qcodes, q.scale, q.zero, torch.arange(K, device="cuda") // gs)
    assert plain.perm.numel() == 0
    sd = {k: v for k, v in plain.state_dict().items() if k != "perm"}
    fresh.load_state_dict(sd)
    assert fresh.perm.numel() == 0 and torch.equal(fresh.qweight, plain.qweight)


@pytest.mark.parametrize("M", [1, 16, 128, 512])
@pytest.mark.parametrize("actorder", [False, True])
def test_fused_quantized_linear(hip, M, actorder):
    """Layers sharing an input in one call: each output equals its own
    layer's (same oracle tolerance), for every kernel regime of M."""
    from distributed_gptq_amd.models import layers as Lm
    K, gs, bits = 512, 128, 4
    rows = [256, 64, 64]
    rng = np.random.default_rng(M + actorder)
    perm = rng.permutation(K) if actorder else np.arange(K)
    g_idx = np.empty(K, np.int64)
    g_idx[perm] = np.arange(K) // gs
    layers, refs = [], []
    x = torch.randn(M, K, device="cuda").half()
    for i, N in enumerate(rows):
        codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
        scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, K // gs))).half()
        zeros = torch.from_numpy(rng.integers(0, 16, (N, K // gs)).astype(np.float64)).half()
        ql = Lm.QuantizedLinear(bits, gs, K, N, bias=i != 1, packed=True).cuda()
        ql.pack_weights(torch.from_numpy(codes).cuda(), scales.cuda(), zeros.cuda(),
                        torch.from_numpy(g_idx).int().cuda(),
                        perm=torch.from_numpy(perm).int().cuda() if actorder else None)
        if ql.bias is not None:
            with torch.no_grad():
                ql.bias.copy_(torch.randn(N))
        layers.append(ql)
        refs.append((codes, scales, zeros, ql.bias))
    fused = Lm.FusedQuantizedLinear(layers)
    assert fused.out_features == sum(rows) and fused.qweight.shape[0] == sum(rows)
    with torch.no_grad():
        ys = fused(x)
        sep = [ql(x) for ql in layers]
    assert len(ys) == 3
    for y, y1, (codes, scales, zeros, bias) in zip(ys, sep, refs):
        assert y.shape == y1.shape
        check_linear(y, x, codes, scales, zeros, g_idx, bias, bits=bits)


@pytest.mark.parametrize("M,gs", [(64, 128), (128, 128), (16, 64), (128, 64)])
def test_linear_small_bf16_scales_with_fp16_x(hip, M, gs):
    """bf16 scales near 1e-5 (below fp16's smallest normal) with fp16
    activations and integer zero points: the packed fp16 decode, which casts
    the scale to fp16, must not be taken; every weight is (q - z) * s rounded
    once to fp16, so the output meets the half-ulp bound (the register-decoded
    kernels at M = 64 / 128, split over K; M = 16 with groups of 64 decodes
    per weight)."""
    from distributed_gptq_amd import _ops
    N, K, bits = 4096, 4096, 4
    rng = np.random.default_rng(M + gs)
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    scales = torch.from_numpy(rng.uniform(0.5e-5, 2e-5, (N, K // gs))).to(torch.bfloat16)
    zeros = torch.from_numpy(rng.integers(0, 16, (N, K // gs)).astype(np.float64)).to(torch.bfloat16)
    x = torch.from_numpy(rng.standard_normal((M, K))).half()
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    y = _ops.linear(x.cuda(), packed, bits, scales.cuda(), zeros.cuda(), K, group_size=gs)
    check_linear(y, x, codes, scales, zeros, np.arange(K) // gs, bits=bits)
