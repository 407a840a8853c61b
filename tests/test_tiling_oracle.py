"""Pins the tiling oracle (oracle/tiling_oracle.py) on the CPU.

KATs are the reference's own (tests/test_common.py:194-218 of simple-vsa); the
other checks fix the definition from coordinates, independently of how the
oracle builds its indices."""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import tiling_oracle as TO

SHAPES = [((2, 6, 6), (2, 3, 3)), ((3, 5, 5), (2, 4, 4)), ((5, 7, 9), (4, 4, 4)),
          ((1, 1, 1), (4, 4, 4)), ((4, 8, 8), (4, 8, 8)), ((6, 3, 10), (4, 2, 3))]


def test_roundtrip_is_identity_kat():
    # tests/test_common.py:194-209
    meta = TO.build_vsa_metadata((2, 6, 6), tile_size=(2, 3, 3))
    seq = 2 * 6 * 6
    x = torch.arange(seq, dtype=torch.float32).reshape(1, seq, 1)
    tiled = TO.tile(x, meta["tile_partition_indices"], meta["non_pad_index"],
                    math.prod(meta["num_tiles"]), meta["max_block_size"])
    back = TO.untile(tiled, meta["non_pad_index"], meta["reverse_tile_partition_indices"])
    assert torch.equal(back, x)


def test_variable_block_sizes_sum_kat():
    # tests/test_common.py:212-218
    meta = TO.build_vsa_metadata((3, 5, 5), tile_size=(2, 4, 4))
    assert int(meta["variable_block_sizes"].sum()) == 75
    assert meta["non_pad_index"].numel() == 75


@pytest.mark.parametrize("shape,ts", SHAPES)
def test_partition_brute_force_from_coordinates(shape, ts):
    T, H, W = shape
    meta = TO.build_vsa_metadata(shape, ts)
    tpi = meta["tile_partition_indices"].numpy()
    nt = meta["num_tiles"]
    assert nt == tuple(math.ceil(a / b) for a, b in zip(shape, ts))
    # expected: tiles in (t, h, w) order, members row-major inside the box
    expect = []
    sizes = []
    for a, b, c in itertools.product(range(nt[0]), range(nt[1]), range(nt[2])):
        box = [(t, h, w) for t in range(T) for h in range(H) for w in range(W)
               if t // ts[0] == a and h // ts[1] == b and w // ts[2] == c]
        sizes.append(len(box))
        expect += [(t * H + h) * W + w for (t, h, w) in box]
    assert np.array_equal(tpi, np.array(expect))
    assert np.array_equal(meta["variable_block_sizes"].numpy(), np.array(sizes))
    # permutation and inverse
    assert np.array_equal(np.sort(tpi), np.arange(T * H * W))
    rev = meta["reverse_tile_partition_indices"].numpy()
    assert np.array_equal(tpi[rev], np.arange(T * H * W))
    assert np.array_equal(rev, np.argsort(tpi))
    # non-pad slots: exactly the first vbs[n] slots of each padded tile
    be = meta["max_block_size"]
    npi = meta["non_pad_index"].numpy()
    mask = np.zeros(len(sizes) * be, bool)
    mask[npi] = True
    for n, s in enumerate(sizes):
        assert mask[n * be:n * be + s].all() and not mask[n * be + s:(n + 1) * be].any()
    assert np.all(np.diff(npi) > 0)


@pytest.mark.parametrize("shape,ts", SHAPES)
def test_tile_zero_pads_and_places_tokens(shape, ts):
    meta = TO.build_vsa_metadata(shape, ts)
    S = math.prod(shape)
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    x = torch.arange(1, S + 1, dtype=torch.float64).reshape(1, S, 1).repeat(2, 1, 3)
    x[1] *= -1
    out = TO.tile(x, meta["tile_partition_indices"], meta["non_pad_index"], nb, be)
    assert out.shape == (2, nb * be, 3)
    tpi = meta["tile_partition_indices"]
    npi = meta["non_pad_index"]
    # token at padded slot npi[i] is raster token tpi[i]; every other slot is 0
    assert torch.equal(out[:, npi], x[:, tpi])
    pad = torch.ones(nb * be, dtype=torch.bool)
    pad[npi] = False
    assert torch.count_nonzero(out[:, pad]) == 0
    assert torch.equal(TO.untile(out, npi, meta["reverse_tile_partition_indices"]), x)


def test_planted_mistake_transposed_tile_order_is_caught(monkeypatch):
    # a restatement that walks tiles in (w, h, t) order must fail the brute force
    def bad(shape, ts):
        T, H, W = shape
        g = np.arange(T * H * W).reshape(T, H, W)
        out = []
        for w0 in range(0, W, ts[2]):
            for h0 in range(0, H, ts[1]):
                for t0 in range(0, T, ts[0]):
                    out.append(g[t0:t0 + ts[0], h0:h0 + ts[1], w0:w0 + ts[2]].reshape(-1))
        return np.concatenate(out)

    monkeypatch.setattr(TO, "tile_partition_indices", bad)
    with pytest.raises(AssertionError):
        test_partition_brute_force_from_coordinates((3, 5, 5), (2, 4, 4))
