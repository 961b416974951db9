"""The factorisation's and the sweep's fp32 products on bf16 MFMAs (the
three-way split in csrc/gemm.hip) at sizes that put them on 128 x 128 tiles
with partial edge tiles: the bounds-checked staging path of those tiles
(rows past the operand, the transposed B operand in 4 x 4 blocks, the
lower-triangle tile order) runs only there.

K = 6100 (47 full leaves and one of 84 columns) splits at the top into
3072 + 3028, so L21, the Schur update, L21 X11 and X22 T2 are 3028 x 3072
products on 24 x 24 tiles of 128 (>= 512 tiles), the last row and column of
tiles partial.  A 3000-row sweep over it runs its trailing updates as
3000 x (6100 - 512 r) products on 128 x 128 tiles with partial last rows
and columns.

Bars: the factor within 2e-5 of the fp64 factor and U Hd U^T = I to 2e-5
(the real-size tests' bars); every code of the first and the last 40 rows
(the last ones in the partial row tile) the correct rounding of the fp64
replay of the GPU's own trajectory to 1e-3 of a step, the replay's scales
within 1e-5 and its zero points equal (or one apart on a rounding tie)."""
import numpy as np
import pytest
import torch

from oracle import gptq_oracle as O

pytestmark = pytest.mark.gpu

K = 6100


@pytest.fixture(scope="module")
def hess(hip):
    g = torch.Generator(device="cuda").manual_seed(61)
    n = 2 * K + 37
    X = torch.randn(n, K, generator=g, device="cuda")
    X[:, :8] *= 20
    H = (X.t() @ X) * (2.0 / n)
    del X
    torch.cuda.empty_cache()
    return H, n


def test_factor_partial_large_tiles(hess):
    from distributed_gptq_amd import _ops
    H, _ = hess
    perm = torch.argsort(torch.diag(H), descending=True, stable=True).to(torch.int32)
    U, Hd, _, info = _ops.damp_factor(H, 1.0, 0.01, perm=perm, want_hd=True)
    assert int(info.item()) == 0
    Ud, Hdd = U.double(), Hd.double()
    eye = torch.eye(K, device="cuda", dtype=torch.float64)
    resid = (torch.linalg.norm(Ud @ Hdd @ Ud.t() - eye) / K ** 0.5).item()
    ref = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hdd)), upper=True)
    dist = (torch.linalg.norm(Ud - ref) / torch.linalg.norm(ref)).item()
    print(f"K={K}: |U Hd U^T - I|/sqrt(K) {resid:.2e}, distance to the fp64 factor {dist:.2e}")
    assert resid < 2e-5 and dist < 2e-5, (resid, dist)
    # upper triangular, positive diagonal
    assert float(torch.tril(U, -1).abs().max()) == 0.0
    assert bool((torch.diag(U) > 0).all())


def test_sweep_partial_large_tiles(hess):
    from distributed_gptq_amd import GPTQ
    H, n = hess
    rows, bits, gs = 3000, 4, 128
    g = torch.Generator().manual_seed(62)
    lin = torch.nn.Linear(K, rows, bias=False)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02, generator=g)
    lin = lin.to(torch.bfloat16).cuda()
    W0 = lin.weight.data.double().cpu().numpy()
    q = GPTQ(lin, bits=bits, group_size=gs, actorder=True, device="cuda")
    q.H = H.clone()
    q.nsamples = n
    q.fasterquant()
    codes = q.qcodes.cpu().numpy()
    s_gpu, z_gpu = q.scale.double().cpu().numpy(), q.zero.double().cpu().numpy()
    U32 = q.H_inv.cpu().numpy()
    perm = q.perm.cpu().numpy()
    dead = np.diag(H.cpu().numpy()) == 0
    sel = np.r_[0:40, rows - 40:rows]
    rep = O.gptq_canonical_replay(W0[sel], U32, perm, dead, bits, gs, 128, codes[sel], s_gpu[sel], z_gpu[sel])
    print(f"rows {rows} x K {K}: replay margin {rep['margin'].max():.2e}")
    assert rep["margin"].max() < 1e-3, rep["margin"].max()
    np.testing.assert_allclose(s_gpu[sel], rep["scale"], rtol=1e-5)
    tie = rep["zero_margin"] < 1e-3
    dz = np.abs(z_gpu[sel] - rep["zero"])
    assert np.all((dz == 0) | (tie & (dz == 1))), dz.max()
