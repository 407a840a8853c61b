"""3-D tile layout of video tokens on MI355X: ``build_vsa_metadata``, ``tile``, ``untile``.

Same names, arguments and results as the reference's ``vsa/fastvideo_tiling.py``
(build_vsa_metadata 91-127, tile 130-140, untile 143-145).  The index tensors
are produced on the GPU by ``vsa_tile_metadata`` (closed form of the raster <->
tile mapping) and the token moves are gfx950 row kernels (``vsa_rows_move``,
``vsa_rows_zero_unmarked``); both are differentiable like the reference's
advanced indexing.  Nothing here runs on the CPU: a CPU tensor or a missing
kernel library raises.
"""

from __future__ import annotations

import functools
import math
from typing import Dict, Optional, Tuple

import torch
from torch import Tensor

from . import _lib

VSA_TILE_SIZE = (4, 4, 4)


def _gpu(device: torch.device) -> torch.device:
    if device.type == "cuda":
        return device
    if not torch.cuda.is_available():
        raise RuntimeError("MI355X tiling builds its metadata on the GPU; no GPU is available")
    return torch.device("cuda", torch.cuda.current_device())


@functools.lru_cache(maxsize=16)
def _metadata(shape: Tuple[int, int, int], tile_size: Tuple[int, int, int],
              device: torch.device) -> Dict[str, object]:
    T, H, W = shape
    ts, hs, ws = tile_size
    if min(shape) <= 0 or min(tile_size) <= 0:
        raise ValueError("dit_seq_shape and tile_size must be positive")
    num_tiles = (math.ceil(T / ts), math.ceil(H / hs), math.ceil(W / ws))
    S, nb = T * H * W, math.prod(num_tiles)
    gdev = _gpu(device)
    tpi = torch.empty(S, dtype=torch.long, device=gdev)
    rev = torch.empty(S, dtype=torch.long, device=gdev)
    npi = torch.empty(S, dtype=torch.long, device=gdev)
    vbs = torch.empty(nb, dtype=torch.long, device=gdev)
    with torch.cuda.device(gdev):
        _lib.call("vsa_tile_metadata", T, H, W, ts, hs, ws, _lib.ptr(tpi), _lib.ptr(rev),
                  _lib.ptr(npi), _lib.ptr(vbs), _lib.stream_of(tpi))
    out = {
        "tile_partition_indices": tpi,
        "reverse_tile_partition_indices": rev,
        "variable_block_sizes": vbs,
        "non_pad_index": npi,
    }
    if device != gdev:
        out = {k: v.to(device) for k, v in out.items()}
    out["num_tiles"] = num_tiles
    out["max_block_size"] = math.prod(tile_size)
    return out


def build_vsa_metadata(dit_seq_shape: Tuple[int, int, int],
                       tile_size: Tuple[int, int, int] = VSA_TILE_SIZE,
                       device: torch.device | str = "cpu") -> Dict[str, object]:
    """Every VSA tiling tensor for a ``(T, H, W)`` latent grid, as the reference's
    build_vsa_metadata (fastvideo_tiling.py:91-127): keys
    ``tile_partition_indices``, ``reverse_tile_partition_indices``,
    ``variable_block_sizes``, ``non_pad_index`` (int64), ``num_tiles``,
    ``max_block_size``.  Built on the GPU and cached per (shape, tile, device);
    for ``device="cpu"`` the tensors are copied back to the host."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    shape = tuple(int(v) for v in dit_seq_shape)
    ts = tuple(int(v) for v in tile_size)
    if len(shape) != 3 or len(ts) != 3:
        raise ValueError("dit_seq_shape and tile_size must have three entries (T, H, W)")
    return dict(_metadata(shape, ts, device))


def _index(t: Tensor, device: torch.device) -> Tensor:
    if t.dtype not in (torch.int64, torch.int32, torch.int16, torch.uint8, torch.int8):
        raise TypeError("tiling indices must be an integer tensor")
    return t.to(device=device, dtype=torch.long).contiguous()


def _rows(x: Tensor) -> Tuple[int, int, int]:
    """(batch, rows, bytes per row) of a [batch, rows, ...] tensor."""
    if x.dim() < 2:
        raise ValueError("expected a [batch, seq_len, ...] tensor")
    row = x.element_size() * math.prod(x.shape[2:])
    return x.shape[0], x.shape[1], row


def _move(x: Tensor, out: Tensor, src: Optional[Tensor], src_outer: Optional[Tensor],
          dst: Optional[Tensor], dst_outer: Optional[Tensor], n: int,
          copy_bytes: Optional[int] = None) -> None:
    """out[b, d(i)] = x[b, s(i)] for i < n (rows along dim 1); with copy_bytes,
    only that prefix of each row is copied and the rest of the out row zeroed."""
    B, xr, xrow = _rows(x)
    _, orow, orb = _rows(out)
    cb = min(xrow, orb) if copy_bytes is None else copy_bytes
    _lib.call("vsa_rows_move", _lib.ptr(x), xr, xrow, _lib.ptr(out), orow, orb, cb, B,
              _lib.ptr(src), src.numel() if src is not None else 0, _lib.ptr(src_outer),
              _lib.ptr(dst), dst.numel() if dst is not None else 0, _lib.ptr(dst_outer), n,
              _lib.stream_of(x))


def _zero_unmarked(out: Tensor, marked: Tensor) -> None:
    B, rows, row = _rows(out)
    mark = torch.empty(max(rows, 1), dtype=torch.uint8, device=out.device)
    _lib.call("vsa_rows_zero_unmarked", _lib.ptr(out), rows, B, row, _lib.ptr(marked),
              marked.numel(), _lib.ptr(mark), _lib.stream_of(out))


def _check(x: Tensor) -> Tensor:
    if x.device.type != "cuda":
        raise ValueError("MI355X tile/untile need a GPU tensor")
    return x.contiguous()


class _Tile(torch.autograd.Function):
    """``out[:, dst] = x[:, src]`` along dim 1 into ``out_rows`` rows, every row
    outside ``dst`` zero.  With unique indices its adjoint is the same move with
    ``src`` and ``dst`` swapped into ``x``'s row count, so the backward applies
    _Tile again and the move differentiates to any order."""

    @staticmethod
    def forward(ctx, x, src, dst, out_rows):
        x = _check(x)
        src, dst = _index(src, x.device), _index(dst, x.device)
        if src.numel() != dst.numel():
            raise ValueError("tile_partition_indices and non_pad_index must have the same length")
        out = torch.empty((x.shape[0], out_rows, *x.shape[2:]), dtype=x.dtype, device=x.device)
        _zero_unmarked(out, dst)
        _move(x, out, src, None, dst, None, src.numel())
        ctx.save_for_backward(src, dst)
        ctx.x_rows = x.shape[1]
        return out

    @staticmethod
    def backward(ctx, g):
        src, dst = ctx.saved_tensors
        return _Tile.apply(g, dst, src, ctx.x_rows), None, None, None


class _Untile(torch.autograd.Function):
    """``out[:, i] = x[:, npi[rev[i]]]`` for i < len(rev); its adjoint is
    _Retile, and the two are each other's backward."""

    @staticmethod
    def forward(ctx, x, npi, rev):
        x = _check(x)
        npi, rev = _index(npi, x.device), _index(rev, x.device)
        out = torch.empty((x.shape[0], rev.numel(), *x.shape[2:]), dtype=x.dtype, device=x.device)
        _move(x, out, npi, rev, None, None, rev.numel())
        ctx.save_for_backward(npi, rev)
        ctx.x_rows = x.shape[1]
        return out

    @staticmethod
    def backward(ctx, g):
        npi, rev = ctx.saved_tensors
        return _Retile.apply(g, npi, rev, ctx.x_rows), None, None


class _Retile(torch.autograd.Function):
    """``out[:, npi[rev[i]]] = x[:, i]`` into ``out_rows`` rows, every row
    outside ``npi`` zero: the adjoint of _Untile."""

    @staticmethod
    def forward(ctx, x, npi, rev, out_rows):
        x = _check(x)
        out = torch.empty((x.shape[0], out_rows, *x.shape[2:]), dtype=x.dtype, device=x.device)
        _zero_unmarked(out, npi)
        _move(x, out, None, None, npi, rev, rev.numel())
        ctx.save_for_backward(npi, rev)
        return out

    @staticmethod
    def backward(ctx, g):
        npi, rev = ctx.saved_tensors
        return _Untile.apply(g, npi, rev), None, None, None


def tile(x: Tensor, tile_partition_indices: Tensor, non_pad_index: Tensor, num_blocks: int,
         max_block_size: int) -> Tensor:
    """Raster-order tokens -> zero-padded tile-contiguous layout along dim 1, as
    the reference's tile (fastvideo_tiling.py:130-140): ``out[:, non_pad_index] =
    x[:, tile_partition_indices]``, every other row zero."""
    return _Tile.apply(x, tile_partition_indices, non_pad_index,
                       int(num_blocks) * int(max_block_size))


def untile(x: Tensor, non_pad_index: Tensor, reverse_tile_partition_indices: Tensor) -> Tensor:
    """Inverse of :func:`tile` (fastvideo_tiling.py:143-145):
    ``x[:, non_pad_index][:, reverse_tile_partition_indices]`` in one pass."""
    return _Untile.apply(x, non_pad_index, reverse_tile_partition_indices)
