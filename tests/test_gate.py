"""CompressionGate (gate producer) on the CPU: the reference's module KATs
(tests/test_common.py:24-60 of simple-vsa) and the layout the fused path keys on."""

import pytest
import torch

from vsa_mi355x import CompressionGate
from vsa_mi355x import mi355x as M


def test_compression_gate_shape_and_layout():
    torch.manual_seed(0)
    batch, heads, seq, head_dim = 2, 3, 12, 8
    dim = heads * head_dim
    gate = CompressionGate(dim=dim, num_heads=heads)(torch.randn(batch, seq, dim))
    assert gate.shape == (batch, heads, seq, head_dim)
    # a per-head view of the [B, S, dim] Linear output: consumed in place on the GPU
    assert gate.stride() == (seq * dim, head_dim, dim, 1)
    assert M._token_major(gate)
    assert not M._token_major(gate.contiguous())


def test_compression_gate_rejects_indivisible_dim():
    with pytest.raises(ValueError, match="divisible"):
        CompressionGate(dim=10, num_heads=3)


def test_compression_gate_rejects_bad_rank():
    with pytest.raises(ValueError, match="hidden_states"):
        CompressionGate(dim=8, num_heads=2)(torch.randn(2, 8))


def test_compression_gate_is_the_linear_map():
    torch.manual_seed(2)
    layer = CompressionGate(dim=12, num_heads=3)
    x = torch.randn(2, 5, 12)
    ref = (x @ layer.to_gate_compress.weight.T + layer.to_gate_compress.bias).view(2, 5, 3, 4)
    assert torch.allclose(layer(x), ref.transpose(1, 2), atol=1e-6)
