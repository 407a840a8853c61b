"""Host orchestration of the MI355X VSA path (Python over the gfx950 C ABI).

Public entry points keep the reference's operator API:

* ``mi355x_vsa(q, k, v, variable_block_sizes, q_variable_block_sizes, topk,
  block_size=64, compress_attn_weight=None, *, sm_scale=None, return_aux=False)``
  -- drop-in for ``torch_vsa`` / ``triton_vsa`` (torch_impl.py:49-57,
  triton_impl.py:1734-1765) and for ``video_sparse_attn`` (common.py:200-212);
* ``mi355x_sparse_attention(q, k, v, selected, variable_block_sizes, *,
  block_size, sm_scale=None)`` -- drop-in for ``triton_sparse_attention``
  (triton_impl.py:1626-1652).

Both are differentiable (one ``torch.autograd.Function`` each).  Every
compute step is a HIP kernel behind ``_lib``; the host only validates,
allocates outputs/workspace with ``torch.empty`` and launches on the current
stream, with no device synchronisation.

The building blocks (pooling, coarse attention + Top-K, CSR inversion, fine
forward / backward) are exposed as functions so tests can check each kernel.

The kernels exist for block volumes 64 / 128 / 256 and head dims 64 / 128 /
256; bf16 / fp16 run on the MFMA kernels, fp32 on fp32 vector-ALU kernels
(no rounding below fp32 anywhere on its path).  Other shapes the reference accepts on the GPU (volume in [1, 128],
head_dim <= 256; triton_impl.py:379-384) run on the same kernels after a
differentiable zero-padding of each block to the next kernel volume and of
the head dim to the next kernel width (gfx950 row kernels); the softmax scale
stays 1/sqrt(head_dim) of the caller's tensors.  Padded query rows are
computed and dropped, padded keys are masked by the block sizes, padded
channels are zero in every dot product.
"""

from __future__ import annotations

import functools
import math
from typing import Optional, Tuple, Union

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import _lib
from .tiling import _move, _zero_unmarked

SUPPORTED_BLOCKS = (64, 128, 256)
SUPPORTED_HEAD_DIMS = (64, 128, 256)
KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
MFMA_DTYPES = (torch.bfloat16, torch.float16)
# blocks per sequence: the Top-K and the backward's CSR keep one row of blocks
# in LDS; the generic coarse kernels (fp32, head dims above 128) keep two
MAX_ROUTE_BLOCKS = 16000
MAX_COARSE_BLOCKS = 4096
# the per-(batch, head) passes put batch * heads in the grid's y dimension
MAX_BATCH_HEADS = 65535


# ---------------------------------------------------------------------------
# Validation (texts follow common.py:97-134 and triton_impl.py:371-401)
# ---------------------------------------------------------------------------

def as_block_elements(block_size: Union[int, Tuple[int, ...]]) -> int:
    """Block volume: int -> cube, tuple -> product (common.py:39-42)."""
    if isinstance(block_size, int):
        return block_size * block_size * block_size
    return int(math.prod(block_size))


def validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk,
                        block_elements) -> None:
    """Shape contract of ``video_sparse_attn`` (common.py:97-134)."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape [batch, heads, seq_len, dim]")
    batch, heads, q_len, dim = q.shape
    kv_len = k.shape[2]
    if k.shape[0] != batch or v.shape[0] != batch or k.shape[1] != heads or v.shape[1] != heads:
        raise ValueError("q, k, and v must share batch and head dimensions")
    if v.shape[2] != kv_len:
        raise ValueError("k and v must have the same sequence length")
    if k.shape[-1] != dim or v.shape[-1] != dim:
        raise ValueError("q, k, and v must have the same head dimension")
    if q_len % block_elements or kv_len % block_elements:
        raise ValueError(
            f"q/kv sequence lengths must be divisible by block_elements={block_elements}")
    qb, kb = q_len // block_elements, kv_len // block_elements
    if variable_block_sizes.numel() != kb:
        raise ValueError(
            f"variable_block_sizes must have length {kb}, got {variable_block_sizes.numel()}")
    if q_variable_block_sizes.numel() != qb:
        raise ValueError(
            f"q_variable_block_sizes must have length {qb}, got {q_variable_block_sizes.numel()}")
    if not 1 <= topk <= kb:
        raise ValueError(f"topk must be in [1, {kb}]")


def _check_device_path(q, k, v, block_elements, coarse=True) -> None:
    """Constraints of the gfx950 kernels (the reference's GPU checks,
    triton_impl.py:371-384, narrowed to the shapes that have MI355X kernels).
    ``coarse``: the op runs the coarse branch (not the explicit route)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("the MI355X implementation requires GPU tensors")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, and v must be on the same GPU device")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, and v must have the same dtype")
    if q.dtype not in KERNEL_DTYPES:
        raise ValueError("the MI355X kernels support float16, bfloat16 and float32")
    _kernel_block(block_elements)
    _kernel_dim(q.shape[-1])
    if q.ndim == 4 and k.ndim == 4 and block_elements > 0:
        nblocks = max(-(-q.shape[-2] // block_elements), -(-k.shape[-2] // block_elements))
        _check_block_count(nblocks, q, coarse)
    if q.ndim == 4 and q.shape[0] * q.shape[1] > MAX_BATCH_HEADS:
        raise ValueError(f"the MI355X kernels support batch * heads <= {MAX_BATCH_HEADS}")


def _check_block_count(nblocks: int, q: Tensor, coarse: bool = True) -> None:
    """At most MAX_ROUTE_BLOCKS blocks per sequence, MAX_COARSE_BLOCKS where the
    coarse branch runs on its generic kernels (fp32, or head dims above 128)."""
    generic = coarse and not (q.dtype in MFMA_DTYPES and _kernel_dim(q.shape[-1]) <= 128)
    limit = MAX_COARSE_BLOCKS if generic else MAX_ROUTE_BLOCKS
    if nblocks > limit:
        raise ValueError(f"the MI355X kernels support at most {limit} blocks per sequence "
                         f"here ({nblocks} given)")


def _kernel_block(be: int) -> int:
    """Block volume the kernels run for a caller's volume ``be``."""
    if be in SUPPORTED_BLOCKS:
        return be
    if not 1 <= be <= 128:
        raise ValueError("the MI355X kernels support block_size volumes in [1, 128] or 256")
    return 64 if be <= 64 else 128


def _kernel_dim(d: int) -> int:
    """Head dim the kernels run for a caller's head dim ``d``."""
    if d in SUPPORTED_HEAD_DIMS:
        return d
    if not 1 <= d <= 256:
        raise ValueError("the MI355X kernels support head_dim <= 256")
    return 64 if d <= 64 else 128 if d <= 128 else 256


@functools.lru_cache(maxsize=32)
def _block_rows(s: int, be: int, kbe: int, device: torch.device) -> Tensor:
    """Row of token i in the layout padded from blocks of be to blocks of kbe."""
    i = torch.arange(s, device=device, dtype=torch.long)
    return torch.div(i, be, rounding_mode="floor") * kbe + i % be


class _Pad(torch.autograd.Function):
    """[B, H, S, d] -> [B, H, (S/be)*kbe, kd], zero rows and channels added.
    _Pad and _Unpad are each other's adjoint, so each one's backward applies the
    other and both differentiate to any order."""

    @staticmethod
    def forward(ctx, x, rows, out_rows, kd):
        x = x.contiguous()
        b, h, s, d = x.shape
        out = torch.empty((b, h, out_rows, kd), dtype=x.dtype, device=x.device)
        xv, ov = x.view(b * h, s, d), out.view(b * h, out_rows, kd)
        if out_rows != s:
            _zero_unmarked(ov, rows)
        _move(xv, ov, None, None, rows, None, s, copy_bytes=d * x.element_size())
        ctx.save_for_backward(rows)
        ctx.shape = (b, h, s, d)
        return out

    @staticmethod
    def backward(ctx, g):
        (rows,) = ctx.saved_tensors
        return _Unpad.apply(g, rows, ctx.shape), None, None, None


def _unpad(x: Tensor, rows: Tensor, shape) -> Tensor:
    b, h, s, d = shape
    x = x.contiguous()
    out = torch.empty(shape, dtype=x.dtype, device=x.device)
    _move(x.view(b * h, x.shape[2], x.shape[3]), out.view(b * h, s, d), rows, None, None, None,
          s, copy_bytes=d * x.element_size())
    return out


class _Unpad(torch.autograd.Function):
    """Inverse of _Pad: keep the caller's rows and channels."""

    @staticmethod
    def forward(ctx, x, rows, shape):
        ctx.save_for_backward(rows)
        ctx.padded = (x.shape[2], x.shape[3])
        return _unpad(x, rows, shape)

    @staticmethod
    def backward(ctx, g):
        (rows,) = ctx.saved_tensors
        return _Pad.apply(g, rows, *ctx.padded), None, None


def _padded(q, k, be):
    """(kbe, kd, pad_q, pad_k, unpad_out) for a shape without its own kernel,
    or None when the kernels take the tensors as they are."""
    d = q.shape[-1]
    kbe, kd = _kernel_block(be), _kernel_dim(d)
    if kbe == be and kd == d:
        return None
    rq = _block_rows(q.shape[2], be, kbe, q.device)
    rk = _block_rows(k.shape[2], be, kbe, k.device)
    nq, nk = q.shape[2] // be * kbe, k.shape[2] // be * kbe

    def pad_q(x, width=kd):
        return None if x is None else _Pad.apply(x, rq, nq, width)

    def pad_k(x):
        return _Pad.apply(x, rk, nk, kd)

    def unpad_out(x):
        return _Unpad.apply(x, rq, tuple(q.shape))

    return kbe, kd, pad_q, pad_k, unpad_out


def _aligned16(x: Optional[Tensor]) -> Optional[Tensor]:
    """x itself when its data is 16-byte aligned (the kernels read and write
    rows with 16-byte accesses), else a copy with the same strides (a view with
    an odd storage offset)."""
    if x is None or x.data_ptr() % 16 == 0:
        return x
    return x.clone()


def _empty_batch(q: Tensor, *others: Optional[Tensor]) -> Tensor:
    """The op on an empty batch (batch or heads 0): an empty output of q's shape
    that is still in the autograd graph of every input (their gradients are
    empty too), as torch_vsa gives one.  Nothing is launched."""
    out = q * 0
    for x in others:
        if x is not None:
            out = out + x.sum() * 0
    return out


def _i32(x: Tensor, device) -> Tensor:
    return x.to(device=device, dtype=torch.int32).contiguous()


# ---------------------------------------------------------------------------
# Kernel-level building blocks (each one C-ABI call)
# ---------------------------------------------------------------------------

def block_mean_qkv(q, k, v, variable_block_sizes, q_variable_block_sizes, block_elements):
    """Pooled ``(q_c, k_c, v_c)`` in the input dtype (fused_block_mean x3)."""
    b, h, sq, d = q.shape
    skv = k.shape[2]
    qc = torch.empty((b, h, sq // block_elements, d), device=q.device, dtype=q.dtype)
    kc = torch.empty((b, h, skv // block_elements, d), device=q.device, dtype=q.dtype)
    vc = torch.empty_like(kc)
    _lib.call("vsa_pool_qkv", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(_i32(q_variable_block_sizes, q.device)),
              _lib.ptr(_i32(variable_block_sizes, q.device)),
              _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), b * h, sq, skv, d, block_elements,
              _lib.dtype_code(q.dtype), _lib.stream_of(q))
    return qc, kc, vc


def coarse_forward(qc, kc, vc, topk: Optional[int], scale: float):
    """Coarse scores / probabilities (fp32 holding T-rounded values), compact
    ``out_c`` and, if ``topk``, the routed key blocks (int32, ascending)."""
    b, h, qb, d = qc.shape
    kb = kc.shape[2]
    scores = torch.empty((b, h, qb, kb), device=qc.device, dtype=torch.float32)
    probs = torch.empty_like(scores)
    outc = torch.empty_like(qc)
    sel = (torch.empty((b, h, qb, topk), device=qc.device, dtype=torch.int32)
           if topk else None)
    _lib.call("vsa_coarse_fwd", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(scores),
              _lib.ptr(probs), _lib.ptr(outc), _lib.ptr(sel), b * h, qb, kb, d, topk or 0,
              float(scale), _lib.dtype_code(qc.dtype), _lib.stream_of(qc))
    return scores, probs, outc, sel


def topk(scores: Tensor, k: int) -> Tensor:
    """Top-K over the last dim of fp32 scores: ties go to the smaller id; ids
    in ascending order (the routing rule of ``coarse_forward``)."""
    scores = scores.contiguous().float()
    kb = scores.shape[-1]
    rows = scores.numel() // kb
    out = torch.empty((*scores.shape[:-1], k), device=scores.device, dtype=torch.int32)
    _lib.call("vsa_topk", _lib.ptr(scores), _lib.ptr(out), rows, kb, k, _lib.stream_of(scores))
    return out


def invert_routes(selected: Tensor, key_blocks: int):
    """``(inverse, offsets, counts)`` CSR of ``selected`` (triton_impl.py:544-595),
    each segment in ascending query-block order."""
    selected = _i32(selected, selected.device)
    b, h, qb, tk = selected.shape
    counts = torch.empty((b, h, key_blocks), device=selected.device, dtype=torch.int32)
    offsets = torch.empty_like(counts)
    inverse = torch.empty((b, h, qb * tk), device=selected.device, dtype=torch.int32)
    _lib.call("vsa_csr_build", _lib.ptr(selected), _lib.ptr(counts), _lib.ptr(offsets),
              _lib.ptr(inverse), b * h, qb, key_blocks, tk, _lib.stream_of(selected))
    return inverse, offsets, counts


def sparse_forward(q, k, v, selected, variable_block_sizes, block_elements, scale, *,
                   out_c=None, gate=None, want_lse=True, want_fine=False):
    """Fine forward (+ combine when ``out_c`` is given).  Returns (out, lse, fine):
    with the combine and ``want_lse`` (or ``want_fine``), ``fine`` is the fine
    output as stored in T, which the backward's delta needs (triton_impl.py:408,
    598-700) and ``return_aux`` reports; else ``fine`` is ``out`` (no combine,
    ``want_lse``) or None."""
    b, h, sq, d = q.shape
    skv = k.shape[2]
    out = torch.empty_like(q)
    lse = (torch.empty((b, h, sq), device=q.device, dtype=torch.float32) if want_lse else None)
    fine = torch.empty_like(q) if ((want_lse or want_fine) and out_c is not None) else None
    gmode = _gate_mode(gate, d, q.dtype) if out_c is not None else _lib.GATE_NONE
    _lib.call("vsa_sparse_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(selected),
              _lib.ptr(variable_block_sizes), _lib.ptr(out), _lib.ptr(fine), _lib.ptr(lse),
              _lib.ptr(out_c), _lib.ptr(gate if gmode else None), gmode, h, b * h, sq, skv, d,
              block_elements, selected.shape[-1], float(scale), _lib.dtype_code(q.dtype),
              _lib.stream_of(q))
    if out_c is None and want_lse:
        fine = out
    return out, lse, fine


def _token_major(gate: Tensor) -> bool:
    """True when a [B, H, S, D] gate is the per-head transpose of a contiguous
    [B, S, H, D] tensor (the gate producer's Linear output, common.py:326-328)."""
    b, h, s, d = gate.shape
    return gate.stride() == (s * h * d, d, h * d, 1) and not gate.is_contiguous()


def _raster_views(q, k, v, gate, be) -> bool:
    """True when q, k and v are [B, H, S, D] views of token-major [B, S, H, D]
    memory (a DiT's per-head view of its projection output, as the gate
    producer returns one, common.py:326-328) that the raster kernels read and
    write in place: one sequence length for q and kv, bf16 / fp16, head dim 64
    or 128, a block volume with its own kernel and a gate (if any) in q's dtype."""
    if q.shape != k.shape or not all(_token_major(x) for x in (q, k, v)):
        return False
    if q.dtype not in MFMA_DTYPES or q.shape[-1] not in (64, 128) or be not in SUPPORTED_BLOCKS:
        return False
    return gate is None or gate.dtype == q.dtype


def _gate_mode(gate: Optional[Tensor], d: int, dtype: torch.dtype) -> int:
    """C-ABI gate mode: layout, plus the fp32 flag for an fp32 gate beside
    bf16 / fp16 inputs."""
    if gate is None:
        return _lib.GATE_NONE
    if gate.shape[-1] == 1 and d != 1:
        mode = _lib.GATE_PER_TOKEN
    else:
        mode = _lib.GATE_TOKEN_MAJOR if _token_major(gate) else _lib.GATE_FULL
    if gate.dtype != dtype:
        assert gate.dtype == torch.float32, gate.dtype
        mode |= _lib.GATE_F32
    return mode


def backward_prep(fine, dout, block_elements, *, out_c=None, gate=None):
    """delta (fp32, from the fine output ``fine`` as stored in T) and, with the
    combine, (d_out_c, d_gate)."""
    out = fine
    b, h, sq, d = out.shape
    delta = torch.empty((b, h, sq), device=out.device, dtype=torch.float32)
    d_outc = torch.empty_like(out_c) if out_c is not None else None
    gmode = _gate_mode(gate, d, out.dtype) if out_c is not None else _lib.GATE_NONE
    d_gate = None
    if (gmode & ~_lib.GATE_F32) == _lib.GATE_TOKEN_MAJOR:   # the gate's own token-major layout
        d_gate = torch.empty((b, sq, h, d), device=gate.device, dtype=gate.dtype).transpose(1, 2)
    elif gmode:
        d_gate = torch.empty_like(gate, memory_format=torch.contiguous_format)
    _lib.call("vsa_bwd_prep", _lib.ptr(out), _lib.ptr(dout), _lib.ptr(out_c),
              _lib.ptr(gate if gmode else None), gmode, h, _lib.ptr(delta), _lib.ptr(d_outc),
              _lib.ptr(d_gate), b * h, sq, d, block_elements, _lib.dtype_code(out.dtype),
              _lib.stream_of(out))
    return delta, d_outc, d_gate


def coarse_backward(qc, kc, vc, probs, d_outc, scale):
    b, h, qb, d = qc.shape
    kb = kc.shape[2]
    ds = torch.empty_like(probs)
    dqc, dkc, dvc = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
    _lib.call("vsa_coarse_bwd", _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(probs),
              _lib.ptr(d_outc), _lib.ptr(ds), _lib.ptr(dqc), _lib.ptr(dkc), _lib.ptr(dvc),
              b * h, qb, kb, d, float(scale), _lib.dtype_code(qc.dtype), _lib.stream_of(qc))
    return dqc, dkc, dvc


def sparse_backward(q, k, v, dout, lse, delta, selected, variable_block_sizes, block_elements,
                    scale, *, dqc=None, dkc=None, dvc=None, q_variable_block_sizes=None):
    """dQ (query-owned) then dK/dV (KV-owned over the CSR route)."""
    b, h, sq, d = q.shape
    skv = k.shape[2]
    kb = skv // block_elements
    tk = selected.shape[-1]
    inverse, offsets, counts = invert_routes(selected, kb)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    code, stream = _lib.dtype_code(q.dtype), _lib.stream_of(q)
    _lib.call("vsa_sparse_bwd_dq", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(dout),
              _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(selected), _lib.ptr(variable_block_sizes),
              _lib.ptr(dq), _lib.ptr(dqc), _lib.ptr(q_variable_block_sizes), b * h, sq, skv, d,
              block_elements, tk, float(scale), code, stream)
    order = dkdv_tile_order(counts, b * h, skv, d, block_elements) if q.dtype in MFMA_DTYPES \
        else None
    _lib.call("vsa_sparse_bwd_dkdv", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(dout),
              _lib.ptr(lse), _lib.ptr(delta), _lib.ptr(counts), _lib.ptr(offsets),
              _lib.ptr(inverse), _lib.ptr(variable_block_sizes), _lib.ptr(dk), _lib.ptr(dv),
              _lib.ptr(dkc), _lib.ptr(dvc), b * h, sq, skv, d, block_elements, tk, float(scale),
              _lib.ptr(order), code, stream)
    return dq, dk, dv


def dkdv_tile_order(counts, bh, skv, head_dim, block_elements):
    """Scheduling workspace of the bf16/fp16 dK/dV kernel: each XCD's tile
    range longest-first when one key block's in-edge count would otherwise set
    the kernel's end (skewed routes), else in index order with the range's
    smallest tiles last, followed by the counters the persistent workgroups
    take tiles from (see vsa_dkdv_tile_order)."""
    # keys per workgroup: four waves of 64 keys at head_dim 64, of 32 above
    kt = min(block_elements, 256 if head_dim == 64 else 128)
    tiles = bh * (skv // kt) * (2 if head_dim > 128 else 1)
    order = torch.empty(8 * ((tiles + 7) // 8) + 16, device=counts.device, dtype=torch.int32)
    _lib.call("vsa_dkdv_tile_order", _lib.ptr(counts), _lib.ptr(order), order.numel(), bh, skv,
              head_dim, block_elements, _lib.stream_of(counts))
    return order


# ---------------------------------------------------------------------------
# Explicit-route executor (triton_impl.py:1530-1652)
# ---------------------------------------------------------------------------

class _SparseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, selected, vbs, block_elements, scale):
        out, lse, _ = sparse_forward(q, k, v, selected, vbs, block_elements, scale,
                                     want_lse=True)
        ctx.save_for_backward(q, k, v, out, lse, selected, vbs)
        ctx.block_elements, ctx.scale = block_elements, scale
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        q, k, v, out, lse, selected, vbs = ctx.saved_tensors
        dout = _aligned16(dout.contiguous())
        delta, _, _ = backward_prep(out, dout, ctx.block_elements)
        dq, dk, dv = sparse_backward(q, k, v, dout, lse, delta, selected, vbs,
                                     ctx.block_elements, ctx.scale)
        return dq, dk, dv, None, None, None, None


def _validate_route(q, k, selected, variable_block_sizes, be):
    batch, heads, sq, _ = q.shape
    qb, kb = sq // be, k.shape[-2] // be
    if sq % be or k.shape[-2] % be:
        raise ValueError(f"q/kv sequence lengths must be divisible by block_elements={be}")
    if tuple(selected.shape[:3]) != (batch, heads, qb) or selected.ndim != 4:
        raise ValueError("selected must have shape [batch, heads, query_blocks, topk]")
    if not 1 <= selected.shape[-1] <= kb:
        raise ValueError(f"selected topk must be in [1, {kb}]")
    if variable_block_sizes.numel() != kb:
        raise ValueError(
            f"variable_block_sizes must have {kb} entries, got {variable_block_sizes.numel()}")


def mi355x_sparse_attention(q: Tensor, k: Tensor, v: Tensor, selected: Tensor,
                            variable_block_sizes: Tensor, *, block_size, sm_scale=None) -> Tensor:
    """Sparse fine attention on a caller-supplied route ``selected``
    ``[B, H, Qb, topk]`` (any integer dtype).  Route ids outside ``[0, Kb)``
    contribute nothing."""
    be = as_block_elements(block_size)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape [batch, heads, seq_len, dim]")
    _check_device_path(q, k, v, be, coarse=False)
    _validate_route(q, k, selected, variable_block_sizes, be)
    if q.shape[0] * q.shape[1] == 0:
        return _empty_batch(q, k, v)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    pads = _padded(q, k, be)
    if pads is not None:
        kbe, _, pad_q, pad_k, unpad_out = pads
        with torch.cuda.device(q.device):
            out = mi355x_sparse_attention(pad_q(q), pad_k(k), pad_k(v), selected,
                                          variable_block_sizes, block_size=(1, 1, kbe),
                                          sm_scale=scale)
            return unpad_out(out)
    q, k, v = (_aligned16(x.contiguous()) for x in (q, k, v))
    selected = _i32(selected, q.device)
    vbs = _i32(variable_block_sizes, q.device)
    with torch.cuda.device(q.device):
        if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
            return _SparseAttention.apply(q, k, v, selected, vbs, be, float(scale))
        return sparse_forward(q, k, v, selected, vbs, be, scale, want_lse=False)[0]


def mi355x_sparse_executor(block_size):
    """The reference's sparse-executor protocol (triton_impl.py:1711-1718,
    1748-1753): returns ``execute(q, k, v, selected, variable_block_sizes, *,
    sm_scale)``, the callable an orchestrator such as ``_vsa_with_sparse_executor``
    (triton_impl.py:1655-1731) invokes for the fine branch, bound to one block
    volume like the reference's ``execute`` closure."""
    be = as_block_elements(block_size)

    def execute(q, k, v, selected, variable_block_sizes, *, sm_scale=None):
        return mi355x_sparse_attention(q, k, v, selected, variable_block_sizes,
                                       block_size=(1, 1, be), sm_scale=sm_scale)

    return execute


# ---------------------------------------------------------------------------
# Full VSA (torch_vsa / triton_vsa signature)
# ---------------------------------------------------------------------------

class _VSA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gate, vbs, qvbs, topk_, be, scale, aux=None):
        qc, kc, vc = block_mean_qkv(q, k, v, vbs, qvbs, be)
        scores, probs, outc, sel = coarse_forward(qc, kc, vc, topk_, scale)
        out, lse, fine = sparse_forward(q, k, v, sel, vbs, be, scale, out_c=outc, gate=gate,
                                        want_lse=True)
        if aux is not None:
            aux.update(scores=scores, selected=sel, out_c=outc, fine=fine)
        ctx.save_for_backward(q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel, fine, lse)
        ctx.be, ctx.scale = be, scale
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel, fine, lse = ctx.saved_tensors
        dout = _aligned16(dout.contiguous())
        delta, d_outc, d_gate = backward_prep(fine, dout, ctx.be, out_c=outc, gate=gate)
        dqc, dkc, dvc = coarse_backward(qc, kc, vc, probs, d_outc, ctx.scale)
        dq, dk, dv = sparse_backward(q, k, v, dout, lse, delta, sel, vbs, ctx.be, ctx.scale,
                                     dqc=dqc, dkc=dkc, dvc=dvc, q_variable_block_sizes=qvbs)
        return dq, dk, dv, d_gate, None, None, None, None, None, None


def _prepare_gate(gate: Optional[Tensor], q: Tensor) -> Optional[Tensor]:
    """The gate as the kernels read it, by differentiable torch ops (autograd
    takes the gradient back to the caller's shape and dtype).

    torch_vsa multiplies by ``compress_attn_weight.float()`` with broadcasting
    (torch_impl.py:108-113), so any gate that broadcasts to q's shape is
    accepted: one that varies along the head dim is expanded to [B, H, S, D],
    one that does not to [B, H, S, 1].  A gate of q's dtype and of one of those
    shapes is read as it is; any other is promoted with ``.float()`` first, as
    the reference does, so its gradient is reduced over the broadcast dims in
    fp32, and read as fp32 (the combine then runs as its own pass over the
    T-rounded fine output, as the reference's fused combine does)."""
    if gate is None:
        return None
    b, h, s, d = q.shape
    try:
        ok = torch.broadcast_shapes(gate.shape, q.shape) == q.shape
    except RuntimeError:
        ok = False
    if not ok:
        raise ValueError("compress_attn_weight must have the same shape as q, or a shape that "
                         "broadcasts to it (e.g. [batch, heads, seq_len, 1])")
    gate = gate.to(device=q.device)
    per_token = (gate.ndim == 0 or gate.shape[-1] == 1) and d != 1
    full = (b, h, s, 1) if per_token else (b, h, s, d)
    if gate.dtype != q.dtype or tuple(gate.shape) != full:
        gate = gate.float().expand(full)
    # the gate producer's per-head view of its [B, S, H, D] output is consumed in
    # place; a per-token gate is always read as contiguous [B*H, S] (a transposed
    # [B, S, H, 1] view has the token-major strides too, so it must be copied)
    return gate if (not per_token and _token_major(gate)) else gate.contiguous()


def mi355x_vsa(q: Tensor, k: Tensor, v: Tensor, variable_block_sizes: Tensor,
               q_variable_block_sizes: Tensor, topk: int, block_size=64,
               compress_attn_weight: Optional[Tensor] = None, *,
               sm_scale: Optional[float] = None, return_aux: bool = False):
    """Video Sparse Attention on MI355X: ``out = out_c * gate + out_s``
    (torch_impl.py:49-113), coarse routing by Top-K of the pooled scores.

    The keyword-only arguments are those of ``video_sparse_attn``
    (common.py:200-212): ``sm_scale`` (default ``1/sqrt(head_dim)``) scales
    both the coarse scores and the fine branch (common.py:225, 241, 262), and
    ``return_aux`` also returns ``{"coarse_scores", "block_mask",
    "out_compress", "out_sparse"}`` (common.py:277-284): the coarse scores in
    q's dtype ``[B, H, Qb, Kb]``, the routed blocks as a bool mask of that
    shape, the compression output expanded to every token and the fine output
    (both ``[B, H, S, D]`` in q's dtype).  The aux tensors are detached: they
    report what the forward computed and carry no gradient.

    Top-K ties are resolved towards the smaller key-block id.  When q, k and v
    are per-head views of token-major [B, S, H, D] tensors the kernels read
    them in place and the result is the same kind of view (no copies either
    side); values are the same bit for bit."""
    be = as_block_elements(block_size)
    validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, be)
    _check_device_path(q, k, v, be)
    if q.shape[0] * q.shape[1] == 0:
        _prepare_gate(compress_attn_weight, q)  # the same shape checks
        out = _empty_batch(q, k, v, compress_attn_weight)
        return (out, _empty_aux(q, k, be)) if return_aux else out
    gate = _aligned16(_prepare_gate(compress_attn_weight, q))
    q, k, v = (_aligned16(x) for x in (q, k, v))
    scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    vbs = _i32(variable_block_sizes, q.device)
    qvbs = _i32(q_variable_block_sizes, q.device)
    aux = {} if return_aux else None
    with torch.cuda.device(q.device):
        if aux is None and _raster_views(q, k, v, gate, be):
            from . import tiled
            return tiled.vsa_token_major_views(q, k, v, gate, vbs, qvbs, topk, be, scale)
        pads = _padded(q, k, be)
        if pads is not None:
            kbe, kd, pad_q, pad_k, unpad_out = pads
            gate = pad_q(gate, kd if gate is not None and gate.shape[-1] == q.shape[-1] else 1)
            out = unpad_out(_vsa(pad_q(q), pad_k(k), pad_k(v), gate, vbs, qvbs, topk, kbe,
                                 scale, aux))
            if aux is not None:
                aux["fine"] = _unpad(aux["fine"], _block_rows(q.shape[2], be, kbe, q.device),
                                     tuple(q.shape))
                aux["out_c"] = aux["out_c"][..., :q.shape[-1]]
        else:
            out = _vsa(q.contiguous(), k.contiguous(), v.contiguous(), gate, vbs, qvbs, topk,
                       be, scale, aux)
    return (out, _aux_dict(aux, q, be)) if return_aux else out


def _aux_dict(aux: dict, q: Tensor, be: int) -> dict:
    """``video_sparse_attn``'s aux outputs (common.py:277-284) from the forward's
    own intermediates: scores (fp32 holding T values) rounded to T exactly, the
    route scattered into a mask, ``out_c`` expanded to every token of its block
    (padding tokens included, common.py:192-196) and the stored fine output."""
    b, h, sq, d = q.shape
    scores, sel = aux["scores"], aux["selected"]
    mask = torch.zeros(scores.shape, dtype=torch.bool, device=q.device)
    mask.scatter_(-1, sel.long(), True)
    outc = aux["out_c"]
    expanded = outc.unsqueeze(3).expand(b, h, sq // be, be, d).reshape(b, h, sq, d)
    return {"coarse_scores": scores.to(q.dtype), "block_mask": mask,
            "out_compress": expanded, "out_sparse": aux["fine"].detach()}


def _empty_aux(q: Tensor, k: Tensor, be: int) -> dict:
    b, h, sq, d = q.shape
    kb = k.shape[2] // be
    return {"coarse_scores": q.new_empty((b, h, sq // be, kb)),
            "block_mask": torch.zeros((b, h, sq // be, kb), dtype=torch.bool, device=q.device),
            "out_compress": q.new_empty(q.shape), "out_sparse": q.new_empty(q.shape)}


def _vsa(q, k, v, gate, vbs, qvbs, topk, be, scale, aux=None):
    """The op on kernel-native shapes (contiguous, be and head dim supported).
    With ``aux`` (a dict) the forward's scores, route, ``out_c`` and fine output
    are put into it."""
    needs_grad = torch.is_grad_enabled() and (
        q.requires_grad or k.requires_grad or v.requires_grad
        or (gate is not None and gate.requires_grad))
    if needs_grad:
        return _VSA.apply(q, k, v, gate, vbs, qvbs, topk, be, scale, aux)
    qc, kc, vc = block_mean_qkv(q, k, v, vbs, qvbs, be)
    scores, _, outc, sel = coarse_forward(qc, kc, vc, topk, scale)
    out, _, fine = sparse_forward(q, k, v, sel, vbs, be, scale, out_c=outc, gate=gate,
                                  want_lse=False, want_fine=aux is not None)
    if aux is not None:
        aux.update(scores=scores, selected=sel, out_c=outc, fine=fine)
    return out


def mi355x_route(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, block_size=64):
    """The routing ``mi355x_vsa`` would use: ``(scores, selected)`` with scores
    as fp32 holding input-dtype values.  For inspection and parity tests."""
    be = as_block_elements(block_size)
    validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, be)
    _check_device_path(q, k, v, be)
    scale = 1.0 / math.sqrt(q.shape[-1])
    vbs = _i32(variable_block_sizes, q.device)
    qvbs = _i32(q_variable_block_sizes, q.device)
    with torch.cuda.device(q.device), torch.no_grad():
        pads = _padded(q, k, be)
        if pads is not None:
            be, _, pad_q, pad_k, _ = pads
            q, k, v = pad_q(q), pad_k(k), pad_k(v)
        qc, kc, vc = block_mean_qkv(q.contiguous(), k.contiguous(), v.contiguous(), vbs, qvbs,
                                    be)
        scores, _, _, sel = coarse_forward(qc, kc, vc, topk, scale)
    return scores, sel
