"""Quantized-model checkpoints (core/quantizer.py:248-335 of the reference):
safetensors state dict + JSON sidecar, and the pytorch format.

CPU tests: QuantizedLinear buffers are filled with seeded random codes,
scales, zeros and act-order g_idx (no kernel runs), saved, and loaded into a
freshly initialised unquantized model of the same architecture.  The bar is
bit-exact: every tensor of the state dict equal with its dtype, the layer
layouts and the metadata restored.  A sidecar written the reference's way
(three keys, no per-layer layout) is read by inferring the layouts."""
import json

import pytest
import torch
import torch.nn as nn


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = nn.ModuleDict({"q_proj": nn.Linear(64, 48), "o_proj": nn.Linear(48, 64, bias=False)})
        self.norm = nn.LayerNorm(64)
        self.mlp = nn.Sequential(nn.Linear(64, 96), nn.GELU(), nn.Linear(96, 64))


class Model(nn.Module):
    def __init__(self, seed):
        super().__init__()
        torch.manual_seed(seed)
        self.layers = nn.ModuleList([Block(), Block()])
        self.head = nn.Linear(64, 10)


# name -> (bits, group_size, packed, act-order g_idx, bias dtype)
LAYOUT = {
    "layers.0.attn.q_proj": (4, 16, True, False, torch.float32),
    "layers.0.attn.o_proj": (3, 16, True, True, None),
    "layers.0.mlp.0": (2, 32, False, True, torch.bfloat16),
    "layers.1.mlp.2": (8, -1, False, False, torch.float16),
    "layers.1.attn.q_proj": (3, 64, False, False, torch.float32),
}


def _set(model, name, mod):
    parts = name.split(".")
    parent = model
    for p in parts[:-1]:
        parent = getattr(parent, p)
    setattr(parent, parts[-1], mod)


def _get(model, name):
    for p in name.split("."):
        model = getattr(model, p)
    return model


def _quantized(layout=LAYOUT, seed=0):
    from distributed_gptq_amd.models.layers import QuantizedLinear
    model = Model(seed=1)
    g = torch.Generator().manual_seed(seed)
    for name, (bits, gs, packed, act, bdt) in layout.items():
        lin = _get(model, name)
        K, N = lin.in_features, lin.out_features
        q = QuantizedLinear(bits, gs, K, N, bias=lin.bias is not None, packed=packed)
        q.qweight.data = torch.randint(0, 256 if q.packed else 1 << bits, q.qweight.shape, generator=g,
                                       dtype=torch.int32).to(torch.uint8)
        q.scales.data = (torch.rand(q.scales.shape, generator=g) * 0.01 + 1e-3).half()
        q.zeros.data = torch.randint(0, 1 << bits, q.zeros.shape, generator=g).half()
        if act:
            q.g_idx.data = (torch.randperm(K, generator=g) // q.group_size).to(torch.int32)
        if q.bias is not None:
            q.bias.data = torch.randn(N, generator=g).to(bdt)
        _set(model, name, q)
    return model


def _assert_same_state(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert list(sa) == list(sb)
    for k in sa:
        assert sa[k].dtype == sb[k].dtype, k
        assert torch.equal(sa[k], sb[k]), k


def _assert_same_layers(a, b, names):
    from distributed_gptq_amd.models.layers import QuantizedLinear
    for n in names:
        qa, qb = _get(a, n), _get(b, n)
        assert isinstance(qb, QuantizedLinear)
        assert (qa.bits, qa.group_size, qa.packed, qa.num_groups, qa.in_features, qa.out_features) == \
            (qb.bits, qb.group_size, qb.packed, qb.num_groups, qb.in_features, qb.out_features)


@pytest.mark.parametrize("fmt", ["safetensors", "pytorch"])
def test_round_trip_into_unquantized_model(tmp_path, fmt):
    from distributed_gptq_amd import QuantizationConfig, load_quantized_model, save_quantized_model
    src = _quantized()
    cfg = QuantizationConfig(bits=4, group_size=16, actorder=True, percdamp=0.02)
    errs = {n: 0.5 * i for i, n in enumerate(LAYOUT)}
    path = tmp_path / "ckpt" / ("model.safetensors" if fmt == "safetensors" else "model.pt")
    save_quantized_model(src, path, save_format=fmt, quant_config=cfg, quantization_errors=errs)
    dst = Model(seed=7)
    out, meta = load_quantized_model(dst, path, load_format=fmt, return_metadata=True)
    assert out is dst
    _assert_same_state(src, dst)
    _assert_same_layers(src, dst, LAYOUT)
    assert meta["quant_config"] == cfg
    assert sorted(meta["quantized_layers"]) == sorted(LAYOUT)
    assert meta["quantization_errors"] == errs


def test_sidecar_and_state_file_follow_the_reference_layout(tmp_path):
    """The .safetensors file is the plain state dict; the .json sidecar
    carries the reference's three keys (core/quantizer.py:265-279)."""
    from safetensors.torch import load_file

    from distributed_gptq_amd import QuantizationConfig, save_quantized_model
    src = _quantized()
    path = tmp_path / "m.safetensors"
    save_quantized_model(src, path, quant_config=QuantizationConfig(bits=3, group_size=64),
                         quantization_errors={"layers.0.mlp.0": 1.25})
    sd = load_file(str(path))
    assert set(sd) == set(src.state_dict())
    for k, v in src.state_dict().items():
        assert sd[k].dtype == v.dtype and torch.equal(sd[k], v), k
    meta = json.loads(path.with_suffix(".json").read_text())
    assert meta["quantization_config"] == {"bits": 3, "group_size": 64, "actorder": False, "percdamp": 0.01,
                                           "blocksize": 128, "calibration_samples": 128, "use_triton": False,
                                           "save_packed": True}
    assert sorted(meta["quantized_layers"]) == sorted(LAYOUT)
    assert meta["quantization_errors"] == {"layers.0.mlp.0": 1.25}
    assert meta["layers"]["layers.0.attn.o_proj"] == {"bits": 3, "group_size": 16, "packed": True,
                                                      "in_features": 48, "out_features": 64, "bias": False}


@pytest.mark.parametrize("bits,gs,packed", [(4, 16, True), (3, 32, False), (2, -1, False), (3, 16, True)])
def test_reference_written_sidecar(tmp_path, bits, gs, packed):
    """A checkpoint saved the reference's way: save_file(model.state_dict())
    and a sidecar with only quantization_config / quantized_layers /
    quantization_errors (core/quantizer.py:265-283).  Layouts are inferred
    from the buffers and the config's bits."""
    from dataclasses import asdict

    from safetensors.torch import save_file

    from distributed_gptq_amd import QuantizationConfig, load_quantized_model
    layout = {n: (bits, gs, packed, False, torch.float32) for n in
              ("layers.0.attn.q_proj", "layers.1.mlp.0", "head")}
    src = _quantized(layout, seed=3)
    path = tmp_path / "ref.safetensors"
    save_file({k: v.contiguous() for k, v in src.state_dict().items()}, str(path))
    path.with_suffix(".json").write_text(json.dumps({
        "quantization_config": asdict(QuantizationConfig(bits=bits, group_size=gs)),
        "quantized_layers": list(layout), "quantization_errors": {}}))
    dst = load_quantized_model(Model(seed=9), path)
    _assert_same_state(src, dst)
    _assert_same_layers(src, dst, layout)


def test_load_into_already_quantized_model(tmp_path):
    from distributed_gptq_amd import load_quantized_model, save_quantized_model
    src = _quantized(seed=4)
    path = tmp_path / "m.safetensors"
    save_quantized_model(src, path)
    dst = _quantized(seed=5)
    load_quantized_model(dst, path)
    _assert_same_state(src, dst)


def test_errors(tmp_path):
    from distributed_gptq_amd import load_quantized_model, save_quantized_model
    src = _quantized()
    path = tmp_path / "m.safetensors"
    with pytest.raises(ValueError, match="save_format"):
        save_quantized_model(src, path, save_format="npz")
    with pytest.raises(ValueError, match="neither QuantizedLinear"):
        save_quantized_model(src, path, quantized_layers=["layers.0.norm"])
    save_quantized_model(src, path)
    with pytest.raises(ValueError, match="load_format"):
        load_quantized_model(Model(seed=2), path, load_format="npz")

    class Wider(Model):
        def __init__(self):
            super().__init__(seed=2)
            self.layers[0].attn["q_proj"] = nn.Linear(64, 40)

    with pytest.raises(ValueError, match="does not match"):
        load_quantized_model(Wider(), path)
    # a quantized layer whose saved layout differs from the model's
    other = _quantized({"layers.0.attn.q_proj": (3, 16, True, False, torch.float32)})
    with pytest.raises(ValueError, match="differs"):
        load_quantized_model(other, path)

    class Renamed(Model):
        def __init__(self):
            super().__init__(seed=2)
            self.layers[0].attn["q_proj"] = nn.LayerNorm(64)

    with pytest.raises(TypeError, match="expected nn.Linear"):
        load_quantized_model(Renamed(), path)
    # a sidecar naming a layer whose buffers are missing
    meta = json.loads(path.with_suffix(".json").read_text())
    meta["quantized_layers"].append("layers.1.attn.k_proj")
    path.with_suffix(".json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match="no buffers"):
        load_quantized_model(Model(seed=2), path)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["safetensors", "pytorch"])
def test_gptq_layers_round_trip_forward_bit_exact(hip, tmp_path, fmt):
    """GPTQ-quantized layers (act-order, 3/4-bit, fp16) saved and loaded into
    an unquantized model give bit-identical buffers and forward outputs."""
    from distributed_gptq_amd import GPTQ, load_quantized_model, replace_with_quantized_layers, save_quantized_model
    model = Model(seed=3).cuda().half()
    g = torch.Generator(device="cuda").manual_seed(0)
    quantizers = {}
    for name, bits, gs, act in [("layers.0.attn.q_proj", 4, 16, True), ("layers.0.mlp.0", 3, 32, False),
                                ("layers.1.attn.o_proj", 4, 16, False), ("head", 4, 64, True)]:
        lin = _get(model, name)
        q = GPTQ(lin, bits=bits, group_size=gs, actorder=act, device="cuda")
        q.add_batch(torch.randn(2, 32, lin.in_features, device="cuda", generator=g).half())
        q.fasterquant()
        quantizers[name] = q
    replace_with_quantized_layers(model, quantizers)
    errs = {n: float(q.losses.double().sum()) for n, q in quantizers.items()}
    path = tmp_path / ("m.safetensors" if fmt == "safetensors" else "m.pt")
    save_quantized_model(model, path, save_format=fmt, quantization_errors=errs)
    dst, meta = load_quantized_model(Model(seed=8).cuda().half(), path, load_format=fmt, return_metadata=True)
    _assert_same_state(model, dst)
    assert meta["quantization_errors"] == errs
    for name in quantizers:
        a, b = _get(model, name), _get(dst, name)
        assert b.qweight.device.type == "cuda"
        x = torch.randn(5, a.in_features, device="cuda", generator=g).half()
        with torch.no_grad():
            assert torch.equal(a(x), b(x)), name
