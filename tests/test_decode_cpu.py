"""Host-side checks of the decode driver (fast-transformer_amd/decode.py) that need no GPU."""

import pytest
import torch

import qwen3_tiny as Q

import decode as D


def test_cache_layout_is_one_allocation_of_layer_views():
    m = Q.model(layers=3)
    cache = D.KVCache(m.config, 2, 10, "cpu")
    assert cache.store.shape == (2, 3, 2, 4, 10, 128) and cache.store.dtype == torch.bfloat16
    for layer in range(3):
        assert cache.keys[layer].is_contiguous() and cache.values[layer].is_contiguous()
        assert cache.keys[layer].data_ptr() == cache.store[0, layer].data_ptr()
        assert cache.values[layer].data_ptr() == cache.store[1, layer].data_ptr()


def test_packed_layer_stacks_the_reference_rows():
    m = Q.model()
    layer = m.model.layers[1]
    packed = D.PackedLayer(layer)
    a, mlp = layer.self_attn, layer.mlp
    q, k, v = packed.qkv_weight.split((a.q_proj.out_features, a.k_proj.out_features, a.v_proj.out_features))
    assert torch.equal(q, a.q_proj.weight) and torch.equal(k, a.k_proj.weight) and torch.equal(v, a.v_proj.weight)
    gate, up = packed.gate_up_weight.chunk(2)
    assert torch.equal(gate, mlp.gate_proj.weight) and torch.equal(up, mlp.up_proj.weight)
    assert packed.q_heads == 8 and packed.scaling == 128 ** -0.5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_a_model_off_the_gpu_is_refused(dtype):
    m = Q.model().to(dtype)
    with pytest.raises(ValueError):
        D.Decoder(m, 1, 8)
