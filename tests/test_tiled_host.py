"""Host-side checks of mi355x_vsa_tiled (no GPU needed): argument validation
runs before any device work, and CPU tensors are rejected, never computed on
the host."""

import pytest
import torch

from vsa_mi355x import tiled


def _qkv(s, d=64):
    return [torch.zeros(1, 2, s, d) for _ in range(3)]


def test_sequence_length_must_be_the_latent_volume():
    with pytest.raises(ValueError, match=r"is not T\*H\*W"):
        tiled.mi355x_vsa_tiled(*_qkv(100), (4, 5, 6), 2)


def test_q_k_v_must_share_one_shape():
    q, k, v = _qkv(120)
    with pytest.raises(ValueError, match="one shape"):
        tiled.mi355x_vsa_tiled(q, k[:, :, :60], v, (4, 5, 6), 2)


def test_shape_and_tile_must_be_three_positive_sizes():
    with pytest.raises(ValueError, match="three positive sizes"):
        tiled.mi355x_vsa_tiled(*_qkv(120), (4, 5, 6), 2, (4, 4))
    with pytest.raises(ValueError, match="three positive sizes"):
        tiled.mi355x_vsa_tiled(*_qkv(120), (4, 5, 6), 2, (4, 0, 4))


def test_gate_must_broadcast_to_q():
    with pytest.raises(ValueError, match="compress_attn_weight"):
        tiled.mi355x_vsa_tiled(*_qkv(120), (4, 5, 6), 2, (4, 4, 4), torch.zeros(1, 2, 7, 1))


def test_cpu_tensors_are_rejected():
    with pytest.raises(ValueError, match="requires GPU tensors"):
        tiled.mi355x_vsa_tiled(*_qkv(120), (4, 5, 6), 2, (4, 4, 4))


def test_token_major_sequence_length_is_dim_one():
    q, k, v = _qkv(120)
    with pytest.raises(ValueError, match=r"seq_len 2 is not T\*H\*W"):
        tiled.mi355x_vsa_tiled(q, k, v, (4, 5, 6), 2, token_major=True)
    tm = [x.transpose(1, 2).contiguous() for x in (q, k, v)]
    with pytest.raises(ValueError, match="requires GPU tensors"):
        tiled.mi355x_vsa_tiled(*tm, (4, 5, 6), 2, token_major=True)


def test_raster_views_rule():
    """Which [B, H, S, D] inputs mi355x_vsa reads in place as token-major views."""
    from vsa_mi355x import mi355x as M

    def tm(s=256, h=4, d=128, dtype=torch.bfloat16):
        return torch.zeros(1, s, h, d, dtype=dtype).transpose(1, 2)

    q, k, v = tm(), tm(), tm()
    assert M._raster_views(q, k, v, None, 64)
    assert M._raster_views(q, k, v, tm(), 256)
    assert M._raster_views(q, k, v, tm(d=1), 128)                      # per-token gate
    assert M._raster_views(q, k, v, q.contiguous(), 64)                # head-major gate
    assert not M._raster_views(q.contiguous(), k, v, None, 64)         # head-major q
    assert not M._raster_views(q, k, v, tm(dtype=torch.float32), 64)   # fp32 gate
    assert not M._raster_views(q, tm(s=512), tm(s=512), None, 64)      # q / kv lengths differ
    assert not M._raster_views(tm(d=256), tm(d=256), tm(d=256), None, 64)
    assert not M._raster_views(*(tm(dtype=torch.float32) for _ in range(3)), None, 64)
    assert not M._raster_views(q, k, v, None, 32)                      # padded block volume
    assert not M._raster_views(tm(h=1), tm(h=1), tm(h=1), None, 64)    # one head: contiguous
