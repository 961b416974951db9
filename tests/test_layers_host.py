"""Host-side logic of QuantizedLinear that needs no GPU: state dicts with and
without the act-order ``perm`` buffer, and the reference's placeholder
g_idx (models/layers.py:60) read as contiguous groups of group_size."""
import pytest
import torch

from distributed_gptq_amd.models.layers import QuantizedLinear


def _state(K, N, gs, g_idx, perm=None):
    ng = -(-K // gs)
    sd = {"qweight": torch.zeros(N, (K + 1) // 2, dtype=torch.uint8),
          "scales": torch.ones(N, ng, dtype=torch.float16), "zeros": torch.zeros(N, ng, dtype=torch.float16),
          "g_idx": g_idx, "bias": torch.zeros(N)}
    if perm is not None:
        sd["perm"] = perm
    return sd


def test_reference_state_dict_without_perm_and_placeholder_g_idx():
    K, N, gs = 200, 8, 128   # K % group_size != 0: ceil(K / groups) = 100 would be wrong
    q = QuantizedLinear(4, gs, K, N)
    q.load_state_dict(_state(K, N, gs, torch.arange(K, dtype=torch.int32)))
    assert q.perm.numel() == 0
    assert torch.equal(q.g_idx, torch.arange(K, dtype=torch.int32) // gs)


def test_state_dict_with_perm_key_loads():
    K, N, gs = 256, 8, 64
    perm = torch.randperm(K).to(torch.int32)
    g_idx = torch.empty(K, dtype=torch.int32)
    g_idx[perm.long()] = torch.arange(K, dtype=torch.int32) // gs
    q = QuantizedLinear(4, gs, K, N)
    q.load_state_dict(_state(K, N, gs, g_idx, perm))
    assert torch.equal(q.perm, perm) and torch.equal(q.g_idx, g_idx)
    # and back to a layer without act-order
    q.load_state_dict(_state(K, N, gs, torch.arange(K, dtype=torch.int32) // gs))
    assert q.perm.numel() == 0
    # perm is never saved: the reference's keys only
    assert set(q.state_dict()) == {"qweight", "scales", "zeros", "g_idx", "bias"}


def test_unexpected_keys_still_reported():
    K, N, gs = 128, 4, 64
    q = QuantizedLinear(4, gs, K, N)
    sd = _state(K, N, gs, torch.arange(K, dtype=torch.int32) // gs)
    sd["bogus"] = torch.zeros(1)
    with pytest.raises(RuntimeError, match="bogus"):
        q.load_state_dict(sd)


def test_group_layout_resolution():
    from distributed_gptq_amd.models.layers import _group_layout
    K = 512
    ar = torch.arange(K, dtype=torch.int32)
    assert _group_layout(ar // 128, K, 4) == (128, None)
    # the placeholder arange(K): groups of ceil(K / ngroups) when they divide K
    assert _group_layout(ar.clone(), K, 4) == (128, None)
    # ... and an error when they do not (K = 200 in 3 groups); the layer
    # itself resolves the placeholder with its group_size when loaded
    with pytest.raises(ValueError, match="ambiguous"):
        _group_layout(torch.arange(200, dtype=torch.int32), 200, 3)
    # act-order: contiguous in perm order -> the group size; else a gather in stored order
    perm = torch.randperm(K).to(torch.int32)
    g_idx = torch.empty(K, dtype=torch.int32)
    g_idx[perm.long()] = ar // 64
    assert _group_layout(g_idx, K, 8, perm) == (64, None)
    gs, gi = _group_layout(g_idx, K, 8)
    assert gs == 64 and torch.equal(gi, g_idx)
    # cached per version: an in-place change is seen
    g2 = ar // 128
    assert _group_layout(g2, K, 4) == (128, None)
    g2[0] = 3
    gs, gi = _group_layout(g2, K, 4)
    assert gi is not None and int(gi[0]) == 3


def test_fused_quantized_linear_rejects_mismatched_layers():
    """Layers fused into one call must agree on in_features, bits, group
    size, storage and column order."""
    from distributed_gptq_amd.models.layers import FusedQuantizedLinear, QuantizedLinear
    a = QuantizedLinear(4, 128, 256, 64, packed=True)
    b = QuantizedLinear(4, 128, 256, 32, packed=True, bias=False)
    f = FusedQuantizedLinear([a, b])
    assert f.splits == [64, 32] and f.qweight.shape == (96, 128) and f.bias.shape == (96,)
    with pytest.raises(ValueError):
        FusedQuantizedLinear([a, QuantizedLinear(4, 64, 256, 32, packed=True)])
    with pytest.raises(ValueError):
        FusedQuantizedLinear([a, QuantizedLinear(3, 128, 256, 32, packed=True)])
    c = QuantizedLinear(4, 128, 256, 32, packed=True)
    c.perm = torch.arange(256, dtype=torch.int32).flip(0)
    with pytest.raises(ValueError):
        FusedQuantizedLinear([a, c])
    with pytest.raises(ValueError):
        FusedQuantizedLinear([])
