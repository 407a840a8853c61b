"""VSA on raster-order video tokens, with tile() / untile() fused into the op.

A video DiT keeps its tokens in raster order (t, h, w) and, for VSA, moves
them into the padded tile-contiguous layout before the op and back after it
(the reference's ``tile`` / ``untile``, fastvideo_tiling.py:130-145): two full
passes over q, k, v and the gate before the op, one over the output after it,
and the same again for the gradients.  ``mi355x_vsa_tiled`` runs the op on
raster-order tensors instead:

* forward: one pass reads raster q, k, v and writes both their tiled copies
  and the block means (``vsa_tile_pool_qkv``); the fine forward writes the
  combined output at raster rows and reads the gate there
  (``vsa_sparse_fwd_tiled``);
* backward: the preprocessing pass reads raster dout and gate, writes d_gate
  at raster rows and the tiled dout the fine kernels consume
  (``vsa_bwd_prep_tiled``); the dQ and dK/dV epilogues store at raster rows.

Every value equals ``untile(mi355x_vsa(tile(q), tile(k), tile(v), ...))`` bit
for bit.  The raster tensors may be head-major ``[B, H, S, D]`` or token-major
``[B, S, H, D]`` (``token_major=True``: the layout a QKV projection writes and
the ``[batch, seq, ...]`` layout tile() itself works on), so a DiT needs no
transpose either side of the op.  Shapes or dtypes without a fused kernel (fp32, head dims other than
64 / 128, tile volumes other than 64 / 128 / 256, a gate that is not
``[B, H, S, D]`` or ``[B, H, S, 1]`` in q's dtype) run that composition.
"""

from __future__ import annotations

import functools
import math
from typing import Optional, Tuple

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import _lib
from . import mi355x as M
from . import tiling

FUSED_BLOCKS = (64, 128, 256)
FUSED_HEAD_DIMS = (64, 128)


@functools.lru_cache(maxsize=16)
def _slot_rows(shape: Tuple[int, int, int], tile_size: Tuple[int, int, int],
               device: torch.device) -> Tensor:
    """int32 [nb * be]: raster token of each padded tile slot, -1 for padding."""
    T, H, W = shape
    ts, hs, ws = tile_size
    nb = math.ceil(T / ts) * math.ceil(H / hs) * math.ceil(W / ws)
    rows = torch.empty(nb * ts * hs * ws, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        _lib.call("vsa_tile_slot_rows", T, H, W, ts, hs, ws, _lib.ptr(rows),
                  _lib.stream_of(rows))
    return rows


def slot_rows(dit_seq_shape, tile_size, device) -> Tensor:
    """The slot -> raster-token table of a latent grid (cached per device)."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return _slot_rows(tuple(int(x) for x in dit_seq_shape), tuple(int(x) for x in tile_size),
                      device)


def _dims(x, token_major):
    """(batch, heads, raster length, head_dim) of a raster q / k / v."""
    if token_major:
        b, s, h, d = x.shape
        return b, h, s, d
    return tuple(x.shape)


def _tile_pool(q, k, v, rows, qvbs, vbs, nb, be, token_major):
    b, h, s_out, d = _dims(q, token_major)
    tiled = (b, h, nb * be, d)
    qt, kt, vt = (torch.empty(tiled, device=q.device, dtype=q.dtype) for _ in range(3))
    qc, kc, vc = (torch.empty((b, h, nb, d), device=q.device, dtype=q.dtype) for _ in range(3))
    _lib.call("vsa_tile_pool_qkv", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(rows),
              _lib.ptr(qvbs), _lib.ptr(vbs), _lib.ptr(qt), _lib.ptr(kt), _lib.ptr(vt), _lib.ptr(qc),
              _lib.ptr(kc), _lib.ptr(vc), b * h, s_out, h if token_major else 0, nb, d, be,
              _lib.dtype_code(q.dtype), _lib.stream_of(q))
    return qt, kt, vt, qc, kc, vc


def _forward(q, k, v, gate, rows, vbs, qvbs, topk, nb, be, scale, want_lse, token_major):
    b, h, s_out, d = _dims(q, token_major)
    qt, kt, vt, qc, kc, vc = _tile_pool(q, k, v, rows, qvbs, vbs, nb, be, token_major)
    _, probs, outc, sel = M.coarse_forward(qc, kc, vc, topk, scale)
    L = nb * be
    out = torch.empty_like(q)
    lse = torch.empty((b, h, L), device=q.device, dtype=torch.float32) if want_lse else None
    fine = torch.empty_like(qt) if want_lse else None
    gmode = M._gate_mode(gate, d, q.dtype)
    _lib.call("vsa_sparse_fwd_tiled", _lib.ptr(qt), _lib.ptr(kt), _lib.ptr(vt), _lib.ptr(sel),
              _lib.ptr(vbs), _lib.ptr(out), _lib.ptr(fine), _lib.ptr(lse), _lib.ptr(outc),
              _lib.ptr(gate), gmode, _lib.ptr(rows), s_out, h if token_major else 0, b * h, L, L,
              d, be, topk, float(scale), _lib.dtype_code(q.dtype), _lib.stream_of(q))
    return out, (qt, kt, vt, qc, kc, vc, probs, outc, sel, fine, lse)


class _VSATiled(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gate, rows, vbs, qvbs, topk_, nb, be, scale, token_major):
        out, saved = _forward(q, k, v, gate, rows, vbs, qvbs, topk_, nb, be, scale, True,
                              token_major)
        ctx.save_for_backward(gate, rows, vbs, qvbs, *saved)
        ctx.dims = (q.shape, _dims(q, token_major), nb, be, scale, token_major)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        gate, rows, vbs, qvbs, qt, kt, vt, qc, kc, vc, probs, outc, sel, fine, lse = \
            ctx.saved_tensors
        shape, (b, h, s_out, d), nb, be, scale, token_major = ctx.dims
        heads = h if token_major else 0
        L = nb * be
        dout = M._aligned16(dout.contiguous())
        code, stream = _lib.dtype_code(dout.dtype), _lib.stream_of(dout)
        delta = torch.empty((b, h, L), device=dout.device, dtype=torch.float32)
        d_outc = torch.empty_like(outc)
        d_gate = torch.empty_like(gate) if gate is not None else None
        dout_t = torch.empty_like(qt)
        gmode = M._gate_mode(gate, d, dout.dtype)
        _lib.call("vsa_bwd_prep_tiled", _lib.ptr(fine), _lib.ptr(dout), _lib.ptr(outc),
                  _lib.ptr(gate), gmode, _lib.ptr(rows), s_out, heads, _lib.ptr(delta),
                  _lib.ptr(d_outc), _lib.ptr(d_gate), _lib.ptr(dout_t), b * h, L, d, be, code,
                  stream)
        dqc, dkc, dvc = M.coarse_backward(qc, kc, vc, probs, d_outc, scale)
        tk = sel.shape[-1]
        dq = torch.empty(shape, device=dout.device, dtype=dout.dtype)
        dk, dv = torch.empty_like(dq), torch.empty_like(dq)
        _lib.call("vsa_sparse_bwd_dq_tiled", _lib.ptr(qt), _lib.ptr(kt), _lib.ptr(vt),
                  _lib.ptr(dout_t), _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(sel), _lib.ptr(vbs),
                  _lib.ptr(dq), _lib.ptr(dqc), _lib.ptr(qvbs), _lib.ptr(rows), s_out, heads, b * h,
                  L, L, d, be, tk, float(scale), code, stream)
        inverse, offsets, counts = M.invert_routes(sel, nb)
        order = M.dkdv_tile_order(counts, b * h, L, d, be)
        _lib.call("vsa_sparse_bwd_dkdv_tiled", _lib.ptr(qt), _lib.ptr(kt), _lib.ptr(vt),
                  _lib.ptr(dout_t), _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(counts),
                  _lib.ptr(offsets), _lib.ptr(inverse), _lib.ptr(vbs), _lib.ptr(dk), _lib.ptr(dv),
                  _lib.ptr(dkc), _lib.ptr(dvc), _lib.ptr(rows), s_out, heads, b * h, L, L, d, be,
                  tk, float(scale), _lib.ptr(order), code, stream)
        return dq, dk, dv, d_gate, None, None, None, None, None, None, None, None


@functools.lru_cache(maxsize=16)
def _identity_rows(n: int, device: torch.device) -> Tensor:
    """int32 [n]: slot s at raster row s (tokens already in block order)."""
    return torch.arange(n, dtype=torch.int32, device=device)


def vsa_token_major_views(q, k, v, gate, vbs, qvbs, topk, be, scale):
    """``mi355x_vsa`` on [B, H, S, D] views of token-major [B, S, H, D] q, k, v:
    the raster kernels with the identity slot table read the token-major
    memory in place and write the output (and dq, dk, dv, d_gate) token-major,
    returned as the same kind of view.  A gate is taken token-major too (free
    for the gate producer's view, one copy for a head-major gate).  The values
    are those of the op on contiguous copies bit for bit: the pool, prep and
    epilogue passes sum in the same order whatever the row addressing."""
    qr, kr, vr = (x.transpose(1, 2) for x in (q, k, v))
    g = None if gate is None else gate.transpose(1, 2).contiguous()
    s = qr.shape[1]
    rows = _identity_rows(s, q.device)
    needs_grad = torch.is_grad_enabled() and (
        q.requires_grad or k.requires_grad or v.requires_grad
        or (g is not None and g.requires_grad))
    if needs_grad:
        out = _VSATiled.apply(qr, kr, vr, g, rows, vbs, qvbs, topk, s // be, be, scale, True)
    else:
        out = _forward(qr, kr, vr, g, rows, vbs, qvbs, topk, s // be, be, scale, False,
                       True)[0]
    return out.transpose(1, 2)


def _composition(q, k, v, meta, nb, be, tile_size, topk, gate, token_major=False):
    """untile(mi355x_vsa(tile(q), tile(k), tile(v), ...)) along the sequence
    dim: head-major tensors with batch and heads folded into tile's batch dim
    (no transposes); token-major ones tiled along dim 1 as they are, then seen
    as [B, H, L, D] by the op."""
    tpi, npi = meta["tile_partition_indices"], meta["non_pad_index"]
    rev, vbs = meta["reverse_tile_partition_indices"], meta["variable_block_sizes"]

    def tl(x):
        if token_major:
            return tiling.tile(x, tpi, npi, nb, be).transpose(1, 2)
        b, h, s, c = x.shape
        return tiling.tile(x.reshape(b * h, s, c), tpi, npi, nb, be).view(b, h, nb * be, c)

    g = None
    if gate is not None:
        per_token = gate.shape[-1] == 1 and q.shape[-1] != 1
        g = tl(torch.broadcast_to(gate, (*q.shape[:3], 1) if per_token else q.shape))
    out = M.mi355x_vsa(tl(q), tl(k), tl(v), vbs, vbs, topk, tile_size, g)
    b, h, _, d = out.shape
    if token_major:
        return tiling.untile(out.transpose(1, 2), npi, rev)
    return tiling.untile(out.reshape(b * h, nb * be, d), npi, rev).view(b, h, -1, d)


def mi355x_vsa_tiled(q: Tensor, k: Tensor, v: Tensor, dit_seq_shape: Tuple[int, int, int],
                     topk: int, tile_size: Tuple[int, int, int] = tiling.VSA_TILE_SIZE,
                     compress_attn_weight: Optional[Tensor] = None,
                     token_major: bool = False) -> Tensor:
    """VSA on raster-order tokens of a ``(T, H, W)`` latent grid: ``[B, H,
    T*H*W, D]``, or ``[B, T*H*W, H, D]`` with ``token_major`` (the gate and the
    result in the same layout).

    Equals ``untile(mi355x_vsa(tile(q), tile(k), tile(v), vbs, vbs, topk,
    tile_size, tile(gate)))`` with tile / untile along the sequence dim and
    ``vbs`` the tiles' real-token counts (build_vsa_metadata), bit for bit;
    the tile and untile passes (fastvideo_tiling.py:130-145) are fused into
    the op's own passes."""
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("mi355x_vsa_tiled expects q, k, v of one shape [batch, heads, seq_len, "
                         "head_dim] ([batch, seq_len, heads, head_dim] with token_major) "
                         "(self-attention over a raster-order video sequence)")
    shape = tuple(int(x) for x in dit_seq_shape)
    ts = tuple(int(x) for x in tile_size)
    if len(shape) != 3 or len(ts) != 3 or min(shape) <= 0 or min(ts) <= 0:
        raise ValueError("dit_seq_shape and tile_size must be three positive sizes (T, H, W)")
    s_out = math.prod(shape)
    seq = q.shape[1] if token_major else q.shape[2]
    if seq != s_out:
        raise ValueError(f"seq_len {seq} is not T*H*W = {s_out} of dit_seq_shape {shape}")
    if compress_attn_weight is not None:
        try:
            ok = torch.broadcast_shapes(compress_attn_weight.shape, q.shape) == q.shape
        except RuntimeError:
            ok = False
        if not ok:
            raise ValueError("compress_attn_weight must have the same shape as q, or a shape "
                             "that broadcasts to it (e.g. [batch, heads, seq_len, 1])")
    be = math.prod(ts)
    nb = math.ceil(shape[0] / ts[0]) * math.ceil(shape[1] / ts[1]) * math.ceil(shape[2] / ts[2])
    # the checks read [B, H, S, D] shapes: token-major tensors as head-major views
    M._check_device_path(*(x.transpose(1, 2) if token_major else x for x in (q, k, v)), be)
    M._check_block_count(nb, q)
    if q.shape[0] * (q.shape[2] if token_major else q.shape[1]) == 0:
        return M._empty_batch(q, k, v, compress_attn_weight)
    gate = compress_attn_weight
    b, h, _, d = _dims(q, token_major)
    full, per_token = ((b, s_out, h, d), (b, s_out, h, 1)) if token_major else \
        ((b, h, s_out, d), (b, h, s_out, 1))
    fused_gate = gate is None or (gate.dtype == q.dtype and gate.device == q.device and
                                  tuple(gate.shape) in (full, per_token))
    fused = (q.dtype in M.MFMA_DTYPES and d in FUSED_HEAD_DIMS and be in FUSED_BLOCKS
             and fused_gate and 1 <= topk <= nb)
    with torch.cuda.device(q.device):
        meta = tiling.build_vsa_metadata(shape, ts, device=q.device)
        if not fused:
            return _composition(q, k, v, meta, nb, be, ts, topk, gate, token_major)
        vbs = meta["variable_block_sizes"].to(torch.int32)
        rows = slot_rows(shape, ts, q.device)
        q, k, v = (M._aligned16(x.contiguous()) for x in (q, k, v))
        if gate is not None:
            gate = M._aligned16(gate.contiguous())
        scale = 1.0 / math.sqrt(d)
        needs_grad = torch.is_grad_enabled() and (
            q.requires_grad or k.requires_grad or v.requires_grad
            or (gate is not None and gate.requires_grad))
        if needs_grad:
            return _VSATiled.apply(q, k, v, gate, rows, vbs, vbs, topk, nb, be, scale,
                                   token_major)
        return _forward(q, k, v, gate, rows, vbs, vbs, topk, nb, be, scale, False,
                        token_major)[0]
