"""gptq::linear captured in a HIP graph: every route (the M = 1 GEMV, the act-order
gather, the register kernels with and without split-K partial sums in the
workspace, several activation tiles) replays to the eager result bit for bit,
replay after replay, with eager work and synchronisations in between, and reads
x at replay time."""
import numpy as np
import pytest
import torch

from oracle import gptq_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(M, N, K, bits, gs, act, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N, K // gs))).half().cuda()
    zeros = torch.from_numpy(rng.integers(0, 2 ** bits, (N, K // gs)).astype(np.float64)).half().cuda()
    packed = torch.from_numpy(O.pack_bitstream(codes, bits)).cuda()
    perm = torch.from_numpy(rng.permutation(K).astype(np.int32)).cuda() if act else None
    bias = torch.from_numpy(rng.standard_normal(N)).half().cuda()
    xs = [torch.from_numpy(rng.standard_normal((M, K))).half().cuda() for _ in range(3)]
    return packed, scales, zeros, perm, bias, xs


@pytest.mark.parametrize("M,N,K,bits,gs,act", [
    (1, 4096, 4096, 4, 128, False),      # GEMV
    (1, 4096, 4096, 4, 128, True),       # gather into the workspace, then the GEMV
    (16, 5120, 8192, 4, 128, False),     # 32-row register workgroups, K in 3 ranges, reduce
    (128, 4096, 4096, 3, 128, False),    # register-decoded, 8 K ranges, reduce
    (64, 24576, 512, 4, 64, False),      # register-decoded unsplit on 7 waves
    (256, 4096, 1024, 4, 128, True),     # gather + two activation tiles + split-K
])
def test_linear_graph_replays_match_eager(hip, M, N, K, bits, gs, act):
    from distributed_gptq_amd import _ops
    packed, scales, zeros, perm, bias, xs = _inputs(M, N, K, bits, gs, act, M + N + K)

    def op(x, out=None):
        return _ops.linear(x, packed, bits, scales, zeros, K, group_size=gs, bias=bias, perm=perm, out=out)

    eager = [op(x) for x in xs]
    torch.cuda.synchronize()
    x_in = xs[0].clone()
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op(x_in, out=y)  # the stream's workspace is allocated outside the capture
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            op(x_in, out=y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for r in range(6):
        i = r % 3
        x_in.copy_(xs[i])
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        # eager work of the program's own between replays
        other = op(xs[(i + 1) % 3])
        torch.cuda.synchronize()
        assert torch.equal(y, eager[i]), (r, i)
        assert torch.equal(other, eager[(i + 1) % 3]), r


@pytest.mark.parametrize("n,K,dt", [(4096, 768, torch.bfloat16), (3000, 1000, torch.float16),
                                    (32768, 3072, torch.bfloat16)])
def test_hessian_graph_replays_accumulate_like_eager(hip, n, K, dt):
    """H += X^T X captured in a HIP graph: each replay adds exactly what the
    same eager call adds (token splits, partial tiles in the workspace and
    their reduce included), with eager work between the replays."""
    from distributed_gptq_amd import _ops
    g = torch.Generator(device="cuda").manual_seed(n + K)
    X = torch.randn(n, K, generator=g, device="cuda").to(dt)
    X2 = torch.randn(n // 2, K, generator=g, device="cuda").to(dt)
    He = torch.zeros(K, K, device="cuda")
    snaps = []
    for _ in range(3):
        _ops.hessian_accumulate(He, X)
        snaps.append(He.clone())
    Hg = torch.zeros(K, K, device="cuda")
    Hw = torch.zeros(K, K, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _ops.hessian_accumulate(Hw, X)  # the stream's workspace is allocated outside the capture
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            _ops.hessian_accumulate(Hg, X)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    Hg.zero_()
    other = torch.zeros(K, K, device="cuda")
    for r in range(3):
        graph.replay()
        _ops.hessian_accumulate(other, X2)  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(Hg, snaps[r]), r


def test_graph_workspace_survives_a_larger_eager_call(hip):
    """A graph captured with the stream's cached workspace (split-K partial
    sums), then an eager call on the same stream that needs more space and
    so replaces the cached buffer, then other tensors allocated and filled:
    the captured buffer must stay alive, so replays still equal the eager
    result and the other tensors keep their values."""
    from distributed_gptq_amd import _ops
    M, N, K, bits, gs = 64, 4096, 4096, 4, 128         # register kernels, K ranges in the workspace (8.4 MB)
    packed, scales, zeros, perm, bias, xs = _inputs(M, N, K, bits, gs, False, 7)
    big = _inputs(128, 4096, 4096, 3, 128, False, 8)  # twice the partial sums (16.8 MB)
    lib = hip
    assert lib.gptq_linear_workspace_size(128, N, K, 3, gs, 1, 0) > lib.gptq_linear_workspace_size(M, N, K, bits,
                                                                                                   gs, 1, 0) > 0

    def op(x, out=None):
        return _ops.linear(x, packed, bits, scales, zeros, K, group_size=gs, bias=bias, out=out)

    eager = op(xs[0])
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    with torch.cuda.stream(s):
        op(xs[0], out=y)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            op(xs[0], out=y)
        # a larger call on the same stream grows (replaces) its workspace
        bp, bs, bz, _, bb, bx = big
        yb = _ops.linear(bx[0], bp, 3, bs, bz, K, group_size=128, bias=bb)
        s.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    yb_ref = yb.clone()
    fill = [torch.full((1 << 20,), float(i), device="cuda") for i in range(64)]  # 256 MB of other tensors
    for r in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), r
        for i, t in enumerate(fill):
            assert bool((t == float(i)).all()), (r, i)
    assert torch.equal(yb, yb_ref)
