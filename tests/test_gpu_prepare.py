"""gptq_prepare_weight (the fp32 copy of a weight in sweep order that the
column sweep works on): bit-exact against a torch gather for every dtype,
with and without a column order and dead columns, for row-major and
transposed (Conv1D-layout) weights, strided rows, and rows too long for the
LDS-staged kernel (the element-wise kernel takes those)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(w, perm, dead, transpose):
    ref = (w.t() if transpose else w).float().clone()
    if dead is not None:
        ref[:, dead.bool()] = 0
    if perm is not None:
        ref = ref[:, perm.long()]
    return ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,cols", [(3, 5), (64, 4096), (257, 14336), (4, 40000)])
@pytest.mark.parametrize("use_perm,use_dead", [(False, False), (True, False), (True, True)])
def test_prepare_weight_matches_gather(hip, dtype, rows, cols, use_perm, use_dead):
    from distributed_gptq_amd import _ops
    g = torch.Generator().manual_seed(rows * 7 + cols)
    w = torch.randn(rows, cols, generator=g).to(dtype).cuda()
    perm = torch.randperm(cols, generator=g).to(torch.int32).cuda() if use_perm else None
    dead = (torch.rand(cols, generator=g) < 0.1).to(torch.int32).cuda() if use_dead else None
    out = _ops.prepare_weight(w, perm=perm, dead=dead)
    assert torch.equal(out, _ref(w, perm, dead, False))


@pytest.mark.parametrize("rows,cols", [(48, 768), (5, 33000)])
def test_prepare_weight_transposed_and_strided(hip, rows, cols):
    from distributed_gptq_amd import _ops
    g = torch.Generator().manual_seed(cols)
    perm = torch.randperm(cols, generator=g).to(torch.int32).cuda()
    dead = (torch.rand(cols, generator=g) < 0.1).to(torch.int32).cuda()
    # Conv1D layout: the weight is stored (cols, rows)
    wt = torch.randn(cols, rows, generator=g).to(torch.bfloat16).cuda()
    out = _ops.prepare_weight(wt, perm=perm, dead=dead, transpose=True)
    assert torch.equal(out, _ref(wt, perm, dead, True))
    # rows with a pitch wider than the row (a column slice of a wider tensor)
    wide = torch.randn(rows, cols + 40, generator=g).to(torch.float16).cuda()
    w = wide[:, 8:8 + cols]
    assert w.stride(0) == cols + 40
    out = _ops.prepare_weight(w, perm=perm, dead=dead)
    assert torch.equal(out, _ref(w, perm, dead, False))
