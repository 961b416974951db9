"""The reference's API wrappers around the per-layer path, on the GPU:
GPTQMultiGPU (core/gptq.py:269-380) as a sequential single-GPU loop,
quantize_layer_gptq (:383-417), quantize_model_simple
(core/quantizer.py:358-383) and GPTQDequantizer / dequantize_model
(core/dequantizer.py:14-163), each against the per-layer GPTQ path or the
oracle."""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import gptq_oracle as O

pytestmark = pytest.mark.gpu


def _model(seed=0):
    torch.manual_seed(seed)
    return nn.Sequential(nn.Linear(256, 128), nn.ReLU(), nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 64)).cuda()


def _data(n=4, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [torch.randn(2, 32, 256, device="cuda", generator=g) for _ in range(n)]


def test_gptq_multi_gpu_sequential_loop(hip):
    from distributed_gptq import GPTQ
    from distributed_gptq.core.gptq import GPTQMultiGPU
    model = _model()
    ref = copy.deepcopy(model)
    X = torch.randn(3, 16, 256, device="cuda")
    mg = GPTQMultiGPU(model, bits=4, group_size=64, actorder=True)
    q = mg.prepare_layer("0", model[0])
    assert q.layer_name == "0" and mg.devices == [torch.device("cuda", 0)]
    mg.add_batch_to_all({"0": X, "missing": X})
    res = mg.quantize_all_layers()
    assert set(res) == {"0"} and q.H is None  # freed after quantization
    g = GPTQ(ref[0], bits=4, group_size=64, actorder=True, device="cuda")
    g.add_batch(X)
    st = g.fasterquant()
    assert torch.equal(model[0].weight, ref[0].weight)
    assert res["0"]["total_error"] == pytest.approx(st["total_error"], rel=1e-6)
    assert mg.get_quantized_model() is model


@pytest.mark.parametrize("canonical", [False, True])
def test_quantize_layer_gptq(hip, canonical):
    from distributed_gptq.core.gptq import quantize_layer_gptq
    lin = nn.Linear(256, 128).cuda()
    W0 = lin.weight.detach().double().cpu().numpy()
    data = [(x,) for x in _data()]
    stats = quantize_layer_gptq(lin, data, bits=4, group_size=64, canonical=canonical, device="cuda")
    Xn = torch.cat([x for (x,) in data]).double().cpu().numpy().reshape(-1, 256)
    H = Xn.T @ Xn
    ns = 4 * 2
    if canonical:
        r = O.gptq_canonical(W0, H, ns, 4, 64, 128, 0.01)
        assert stats["total_error"] == pytest.approx(float(r["losses"].sum()), rel=0.01)
        e = O.layer_error(W0, lin.weight.detach().double().cpu().numpy(), H)
        assert abs(e - O.layer_error(W0, r["dequant"], H)) <= 0.01 * e
    else:
        r = O.gptq_ref(W0, O.full_inverse(O.damp_ref(H, ns, 0.01)), 4, 64, 128)
        assert np.mean(lin.weight.detach().cpu().numpy() == r["codes"]) >= 0.999
        assert stats["total_error"] == pytest.approx(r["total_error"], rel=0.01)


def test_quantize_model_simple_and_dequantize_model(hip):
    from distributed_gptq import quantize_model_simple
    from distributed_gptq.core import GPTQDequantizer, dequantize_model
    from distributed_gptq.models.layers import QuantizedLinear
    base = _model(3).half()
    data = [x.half() for x in _data(3, 5)]
    model = quantize_model_simple(copy.deepcopy(base), data, bits=4)
    qs = [m for m in model.modules() if isinstance(m, QuantizedLinear)]
    assert len(qs) == 3 and all(q.bits == 4 and q.group_size == 128 for q in qs)
    x = torch.randn(5, 256, device="cuda").half()
    with torch.no_grad():
        yq = model(x).float()
        yb = base(x).float()
    assert ((yq - yb).norm() / yb.norm()).item() < 0.2
    # the dequantizer's weights are the layers' own dequantised weights
    dq = GPTQDequantizer(bits=4, group_size=128)
    for q in qs:
        w = dq.dequantize_weight(q.qweight, q.scales, q.zeros, q.g_idx)
        assert torch.equal(w, q.unpack_weights())
        lin = dq.dequantize_layer(q)
        assert isinstance(lin, nn.Linear) and torch.equal(lin.weight, w)
    dense = dequantize_model(copy.deepcopy(model))
    assert not any(isinstance(m, QuantizedLinear) for m in dense.modules())
    with torch.no_grad():
        yd = dense.half()(x).float()
    assert ((yd - yq).norm() / yq.norm()).item() < 1e-2
    # 4-bit unpack: low nibble first (core/dequantizer.py:86-87)
    packed = torch.tensor([[0x21, 0x43]], dtype=torch.uint8, device="cuda")
    assert dq._unpack_4bit(packed).tolist() == [[1.0, 2.0, 3.0, 4.0]]
