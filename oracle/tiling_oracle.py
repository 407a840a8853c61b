"""CPU restatement of the reference's VSA tiling helpers -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline may
import this module, and only as the checker.  The product path
(``simple-vsa_amd/vsa/tiling.py``) runs the gfx950 kernels and never calls it.

Follows ``vsa/fastvideo_tiling.py`` of ita9naiwa/simple-vsa:

* ``tile_partition_indices``   <- get_tile_partition_indices (fastvideo_tiling.py:22-42)
* ``reverse_indices``          <- get_reverse_tile_partition_indices (45-52)
* ``variable_block_sizes``     <- construct_variable_block_sizes (55-78)
* ``non_pad_index``            <- get_non_pad_index (81-88)
* ``build_vsa_metadata``       <- build_vsa_metadata (91-127)
* ``tile`` / ``untile``        <- tile (130-140) / untile (143-145)

Pinned by tests/test_oracle.py: the reference's own KATs (round trip on a
(2,6,6) grid with (2,3,3) tiles, tests/test_common.py:194-209; valid-token sum
and non-pad length on (3,5,5) with (2,4,4) tiles, 212-218), plus brute-force
checks that fix the definition independently of this code: every tile's
indices are exactly the raster ids whose coordinates fall in that box, in
row-major (t, h, w) order; the partition is a permutation; the reverse is its
inverse; padded slots are the only zero rows of a tiled tensor.
"""

from __future__ import annotations

import math
from typing import Dict, Sequence, Tuple

import numpy as np
import torch


def _extent(length: int, tile: int, index: int) -> int:
    """Tokens of tile ``index`` along one axis (the last tile holds the rest)."""
    return min(tile, length - index * tile)


def tile_partition_indices(shape: Sequence[int], tile_size: Sequence[int]) -> np.ndarray:
    """Raster token ids, tile by tile in (t, h, w) tile order; inside a tile
    row-major over (t, h, w).  fastvideo_tiling.py:22-42."""
    T, H, W = shape
    ts, hs, ws = tile_size
    grid = np.arange(T * H * W, dtype=np.int64).reshape(T, H, W)
    pieces = []
    for t0 in range(0, T, ts):
        for h0 in range(0, H, hs):
            for w0 in range(0, W, ws):
                pieces.append(grid[t0:t0 + ts, h0:h0 + hs, w0:w0 + ws].reshape(-1))
    return np.concatenate(pieces)


def reverse_indices(perm: np.ndarray) -> np.ndarray:
    """Inverse permutation (argsort of a permutation).  fastvideo_tiling.py:45-52."""
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=perm.dtype)
    return inv


def variable_block_sizes(shape: Sequence[int], tile_size: Sequence[int]) -> np.ndarray:
    """Real tokens per tile, (t, h, w) tile order.  fastvideo_tiling.py:55-78."""
    ext = [[_extent(L, s, i) for i in range(math.ceil(L / s))] for L, s in zip(shape, tile_size)]
    return np.array([a * b * c for a in ext[0] for b in ext[1] for c in ext[2]], dtype=np.int64)


def non_pad_index(vbs: np.ndarray, max_block_size: int) -> np.ndarray:
    """Padded-layout slots n*be + p with p < vbs[n], ascending.  fastvideo_tiling.py:81-88."""
    return np.concatenate([n * max_block_size + np.arange(int(c), dtype=np.int64)
                           for n, c in enumerate(vbs)]) if len(vbs) else np.zeros(0, np.int64)


def build_vsa_metadata(shape: Tuple[int, int, int],
                       tile_size: Tuple[int, int, int] = (4, 4, 4)) -> Dict[str, object]:
    """Same keys as the reference's build_vsa_metadata (fastvideo_tiling.py:91-127),
    as CPU int64 tensors."""
    be = math.prod(tile_size)
    nt = tuple(math.ceil(L / s) for L, s in zip(shape, tile_size))
    tpi = tile_partition_indices(shape, tile_size)
    vbs = variable_block_sizes(shape, tile_size)
    return {
        "tile_partition_indices": torch.from_numpy(tpi),
        "reverse_tile_partition_indices": torch.from_numpy(reverse_indices(tpi)),
        "variable_block_sizes": torch.from_numpy(vbs),
        "non_pad_index": torch.from_numpy(non_pad_index(vbs, be)),
        "num_tiles": nt,
        "max_block_size": be,
    }


def tile(x: torch.Tensor, tpi: torch.Tensor, npi: torch.Tensor, num_blocks: int,
         max_block_size: int) -> torch.Tensor:
    """Raster -> zero-padded tile layout along dim 1.  fastvideo_tiling.py:130-140."""
    out = torch.zeros((x.shape[0], num_blocks * max_block_size, *x.shape[2:]), dtype=x.dtype)
    out[:, npi.long()] = x[:, tpi.long()]
    return out


def untile(x: torch.Tensor, npi: torch.Tensor, rev: torch.Tensor) -> torch.Tensor:
    """Tile layout -> raster along dim 1.  fastvideo_tiling.py:143-145."""
    return x[:, npi.long()][:, rev.long()]
