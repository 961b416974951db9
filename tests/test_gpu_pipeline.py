"""The block driver: several layers, two of them sharing one Hessian, each
Hessian's chain on its own stream.  Results must not depend on the number of
streams (bit-identical to one stream) and must match the fp64 oracle to the
north-star bars (codes >= 99.9%, ||WX - QX||^2 within 1%)."""
import numpy as np
import pytest
import torch

from oracle import gptq_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = {"a1": (96, 256), "a2": (64, 256), "b": (80, 384)}
    hkey = {"a1": "A", "a2": "A", "b": "B"}
    weights = {n: (torch.randn(*s, generator=g) * 0.02).cuda() for n, s in shapes.items()}
    hess = {}
    for key, K in (("A", 256), ("B", 384)):
        X = torch.randn(512, K, generator=g)
        X[:, torch.randperm(K, generator=g)[:3]] *= 15
        hess[key] = ((X.T @ X).cuda(), 4)
    return weights, hkey, hess


@pytest.mark.parametrize("actorder", [False, True])
def test_streams_bit_identical_and_oracle(hip, actorder):
    from distributed_gptq_amd import pipeline
    weights, hkey, hess = _inputs(1)
    r4 = pipeline.quantize_layers(weights, hkey, hess, bits=4, group_size=64, actorder=actorder, streams=4)
    r1 = pipeline.quantize_layers(weights, hkey, hess, bits=4, group_size=64, actorder=actorder, streams=1)
    assert list(r4) == list(weights)
    for name in weights:
        for f in ("codes", "qweight", "scale", "zero", "g_idx", "dequant"):
            assert torch.equal(getattr(r4[name], f), getattr(r1[name], f)), (name, f)
        W0 = weights[name].double().cpu().numpy()
        H, ns = hess[hkey[name]]
        Hn = H.double().cpu().numpy()
        ref = O.gptq_canonical(W0, Hn, ns, 4, 64, 128, 0.01, actorder=actorder)
        assert np.mean(r4[name].codes.cpu().numpy() == ref["codes"]) >= 0.999
        np.testing.assert_array_equal(r4[name].g_idx.cpu().numpy(), ref["g_idx"])
        e_gpu = O.layer_error(W0, r4[name].dequant.double().cpu().numpy(), Hn)
        e_ref = O.layer_error(W0, ref["dequant"], Hn)
        assert abs(e_gpu - e_ref) <= 0.01 * e_ref, (name, e_gpu, e_ref)


def test_not_positive_definite_raises(hip):
    from distributed_gptq_amd import pipeline
    weights, hkey, hess = _inputs(2)
    H, ns = hess["B"]
    hess["B"] = (-H, ns)
    with pytest.raises(torch.linalg.LinAlgError):
        pipeline.quantize_layers(weights, hkey, hess, bits=4, group_size=64)
