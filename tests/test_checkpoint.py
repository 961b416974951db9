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


# ------------------------------------------------ act-order column order --

@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("K", [7, 64, 200])
def test_code_row_packing_matches_the_oracle(bits, K):
    """The byte-level unpack / pack behind the act-order column reorder of a
    checkpoint: LSB-first b-bit rows, as the oracle packs them."""
    from distributed_gptq_amd.models.layers import _pack_rows, _unpack_rows
    from oracle import gptq_oracle as O
    import numpy as np
    codes = np.random.default_rng(bits * K).integers(0, 2 ** bits, (5, K)).astype(np.uint8)
    packed = O.pack_bitstream(codes, bits)
    assert torch.equal(_pack_rows(torch.from_numpy(codes), bits), torch.from_numpy(packed))
    assert torch.equal(_unpack_rows(torch.from_numpy(packed), bits, K), torch.from_numpy(codes))


class RefQuantizedLinear(nn.Module):
    """Only the reference's QuantizedLinear buffers (models/layers.py:49-60):
    qweight, fp16 scales / zeros, int32 g_idx, bias."""

    def __init__(self, row_bytes, K, N, ngroups, bias):
        super().__init__()
        self.register_buffer("qweight", torch.zeros((N, row_bytes), dtype=torch.uint8))
        self.register_buffer("scales", torch.zeros((N, ngroups), dtype=torch.float16))
        self.register_buffer("zeros", torch.zeros((N, ngroups), dtype=torch.float16))
        self.register_buffer("g_idx", torch.arange(K, dtype=torch.int32))
        self.bias = nn.Parameter(torch.zeros(N)) if bias else None


def _actorder_layer(bits, gs, K, N, seed, packed=True):
    """A QuantizedLinear holding act-order codes the way from_gptq stores
    them (columns in perm order, perm = stable sort of g_idx), built on the
    CPU with the oracle's packing; returns it and the input-order codes."""
    import numpy as np

    from distributed_gptq_amd.models.layers import QuantizedLinear
    from oracle import gptq_oracle as O
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    sweep = rng.permutation(K)
    g_idx = np.empty(K, np.int32)
    g_idx[sweep] = np.arange(K) // gs
    perm = np.argsort(g_idx, kind="stable").astype(np.int32)
    q = QuantizedLinear(bits, gs, K, N, bias=True, packed=packed)
    stored = codes[:, perm]
    q.qweight.data = torch.from_numpy(O.pack_bitstream(stored, bits) if q.packed else stored.copy())
    q.scales.data = torch.from_numpy(rng.uniform(1e-3, 1e-2, q.scales.shape)).half()
    q.zeros.data = torch.from_numpy(rng.integers(0, 2 ** bits, q.zeros.shape).astype(np.float64)).half()
    q.g_idx.data = torch.from_numpy(g_idx)
    q.perm.data = torch.from_numpy(perm)
    q.bias.data = torch.randn(N)
    return q, codes


@pytest.mark.parametrize("bits,gs,packed", [(4, 16, True), (3, 32, True), (2, 16, False), (8, 16, False)])
def test_actorder_checkpoint_loads_strictly_into_reference_modules(tmp_path, bits, gs, packed):
    """A saved act-order layer has the reference's keys only (no perm) and its
    codes in input-column order: a strict load_state_dict into modules with
    only the reference's buffers (core/quantizer.py:319-320) takes it and
    decodes the same weights; loading it back into this package's
    QuantizedLinear re-derives perm and the stored order bit for bit."""
    import numpy as np
    from safetensors.torch import load_file

    from distributed_gptq_amd import load_quantized_model, save_quantized_model
    from oracle import gptq_oracle as O
    model = Model(seed=4)
    lin = _get(model, "layers.0.mlp.0")
    q, codes = _actorder_layer(bits, gs, lin.in_features, lin.out_features, seed=bits, packed=packed)
    _set(model, "layers.0.mlp.0", q)
    path = tmp_path / "m.safetensors"
    save_quantized_model(model, path)
    state = load_file(str(path))
    assert "layers.0.mlp.0.perm" not in state
    ref_model = Model(seed=5)
    _set(ref_model, "layers.0.mlp.0", RefQuantizedLinear(q.qweight.shape[1], q.in_features, q.out_features,
                                                         q.num_groups, bias=True))
    ref_model.load_state_dict(state, strict=True)
    rq = _get(ref_model, "layers.0.mlp.0")
    expect = O.pack_bitstream(codes, bits) if q.packed else codes
    np.testing.assert_array_equal(rq.qweight.numpy(), expect)
    got = O.unpack_bitstream(rq.qweight.numpy(), bits, q.in_features) if q.packed else rq.qweight.numpy()
    gi = rq.g_idx.numpy()
    np.testing.assert_array_equal(O.dequant(got, rq.scales.numpy(), rq.zeros.numpy(), gi),
                                  O.dequant(codes, q.scales.numpy(), q.zeros.numpy(), q.g_idx.numpy()))
    # back into this package's layer: perm and the stored order return
    dst = load_quantized_model(Model(seed=6), path)
    back = _get(dst, "layers.0.mlp.0")
    assert torch.equal(back.perm, q.perm) and torch.equal(back.qweight, q.qweight)
    assert torch.equal(back.g_idx, q.g_idx) and torch.equal(back.scales, q.scales)


def test_checkpoint_with_a_perm_key_still_loads(tmp_path):
    """The earlier format (a ``perm`` key, codes in that stored order) loads
    into the same layer."""
    from distributed_gptq_amd.models.layers import QuantizedLinear
    q, _ = _actorder_layer(4, 16, 64, 48, seed=9)
    sd = {k: v.clone() for k, v in q.state_dict().items()}
    sd["qweight"] = q.qweight.clone()
    sd["perm"] = q.perm.clone()
    fresh = QuantizedLinear(4, 16, 64, 48, bias=True)
    fresh.load_state_dict(sd, strict=True)
    assert torch.equal(fresh.perm, q.perm) and torch.equal(fresh.qweight, q.qweight)
