"""The MI355X VSA path as torch.library custom ops, for torch.compile.

``vsa_mi355x.mi355x_vsa`` is an autograd Function whose forward and backward
call the C ABI through ctypes, which torch.compile cannot trace (it breaks the
graph there).  The same computation is registered here as opaque custom ops
with fake (shape-only) implementations and an autograd formula, so a compiled
model keeps the op inside its graph:

* ``vsa_mi355x::vsa_fwd`` / ``vsa_mi355x::vsa_bwd`` -- the full op
  (``torch_vsa`` / ``triton_vsa``, torch_impl.py:49-113);
* ``vsa_mi355x::sparse_fwd`` / ``vsa_mi355x::sparse_bwd`` -- the explicit-route
  fine branch (``triton_sparse_attention``, triton_impl.py:1626-1652).

``mi355x_vsa`` and ``mi355x_sparse_attention`` below keep the reference
signatures and validation and give the same values as the eager functions of
the same name, bit for bit.  Shapes without a kernel of their own (block
volumes other than 64 / 128 / 256, head dims other than 64 / 128 / 256) run
the eager functions (a graph break under torch.compile).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import mi355x as M


def _empty(like: Tensor, dtype=None) -> Tensor:
    return like.new_empty((0,), dtype=dtype or like.dtype)


# ---------------------------------------------------------------------------
# Full op
# ---------------------------------------------------------------------------

@torch.library.custom_op("vsa_mi355x::vsa_fwd", mutates_args=(), device_types="cuda")
def vsa_fwd(q: Tensor, k: Tensor, v: Tensor, gate: Optional[Tensor], vbs: Tensor, qvbs: Tensor,
            topk: int, be: int, scale: float, save: bool
            ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(out, q_c, k_c, v_c, probs, out_c, selected, fine, lse); with ``save``
    false everything after ``out`` is an empty placeholder."""
    q, k, v, gate = (M._aligned16(x) for x in (q, k, v, gate))
    with torch.cuda.device(q.device):
        qc, kc, vc = M.block_mean_qkv(q, k, v, vbs, qvbs, be)
        _, probs, outc, sel = M.coarse_forward(qc, kc, vc, topk, scale)
        out, lse, fine = M.sparse_forward(q, k, v, sel, vbs, be, scale, out_c=outc, gate=gate,
                                          want_lse=save)
    if not save:
        return (out, _empty(q), _empty(q), _empty(q), _empty(q, torch.float32), _empty(q),
                _empty(q, torch.int32), _empty(q), _empty(q, torch.float32))
    return out, qc, kc, vc, probs, outc, sel, fine, lse


@vsa_fwd.register_fake
def _(q, k, v, gate, vbs, qvbs, topk, be, scale, save):
    b, h, sq, d = q.shape
    qb, kb = sq // be, k.shape[2] // be
    out = torch.empty_like(q)
    if not save:
        return (out, _empty(q), _empty(q), _empty(q), _empty(q, torch.float32), _empty(q),
                _empty(q, torch.int32), _empty(q), _empty(q, torch.float32))
    blocks = q.new_empty((b, h, qb, d))
    return (out, blocks, q.new_empty((b, h, kb, d)), q.new_empty((b, h, kb, d)),
            q.new_empty((b, h, qb, kb), dtype=torch.float32), torch.empty_like(blocks),
            q.new_empty((b, h, qb, topk), dtype=torch.int32), torch.empty_like(q),
            q.new_empty((b, h, sq), dtype=torch.float32))


@torch.library.custom_op("vsa_mi355x::vsa_bwd", mutates_args=(), device_types="cuda")
def vsa_bwd(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, gate: Optional[Tensor], vbs: Tensor,
            qvbs: Tensor, qc: Tensor, kc: Tensor, vc: Tensor, probs: Tensor, outc: Tensor,
            sel: Tensor, fine: Tensor, lse: Tensor, be: int, scale: float
            ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, dv, d_gate); d_gate is an empty placeholder without a gate."""
    q, k, v, gate = (M._aligned16(x) for x in (q, k, v, gate))
    with torch.cuda.device(q.device):
        dout = M._aligned16(dout.contiguous())
        delta, d_outc, d_gate = M.backward_prep(fine, dout, be, out_c=outc, gate=gate)
        dqc, dkc, dvc = M.coarse_backward(qc, kc, vc, probs, d_outc, scale)
        dq, dk, dv = M.sparse_backward(q, k, v, dout, lse, delta, sel, vbs, be, scale,
                                       dqc=dqc, dkc=dkc, dvc=dvc, q_variable_block_sizes=qvbs)
    return dq, dk, dv, (d_gate if d_gate is not None else _empty(q))


@vsa_bwd.register_fake
def _(dout, q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel, fine, lse, be, scale):
    d_gate = (torch.empty(gate.shape, dtype=gate.dtype, device=gate.device) if gate is not None
              else _empty(q))
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), d_gate


def _vsa_setup(ctx, inputs, output):
    q, k, v, gate, vbs, qvbs, topk, be, scale, save = inputs
    _, qc, kc, vc, probs, outc, sel, fine, lse = output
    ctx.save_for_backward(q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel, fine, lse)
    ctx.be, ctx.scale, ctx.has_gate = be, scale, gate is not None


def _vsa_backward(ctx, dout, *_):
    q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel, fine, lse = ctx.saved_tensors
    dq, dk, dv, d_gate = vsa_bwd(dout, q, k, v, gate, vbs, qvbs, qc, kc, vc, probs, outc, sel,
                                 fine, lse, ctx.be, ctx.scale)
    return (dq, dk, dv, d_gate if ctx.has_gate else None, None, None, None, None, None, None)


vsa_fwd.register_autograd(_vsa_backward, setup_context=_vsa_setup)


def mi355x_vsa(q: Tensor, k: Tensor, v: Tensor, variable_block_sizes: Tensor,
               q_variable_block_sizes: Tensor, topk: int, block_size=64,
               compress_attn_weight: Optional[Tensor] = None, *,
               sm_scale: Optional[float] = None, return_aux: bool = False):
    """``vsa_mi355x.mi355x_vsa`` (torch_impl.py:49-57, common.py:200-212) through
    the custom ops: the same checks, values and gradients, traceable by
    torch.compile.  ``return_aux`` runs the eager function (a graph break)."""
    be = M.as_block_elements(block_size)
    M.validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, be)
    M._check_device_path(q, k, v, be)
    if (return_aux or q.shape[0] * q.shape[1] == 0 or M._padded(q, k, be) is not None):
        return M.mi355x_vsa(q, k, v, variable_block_sizes, q_variable_block_sizes, topk,
                            block_size, compress_attn_weight, sm_scale=sm_scale,
                            return_aux=return_aux)
    # contiguous gate: d_gate then has the strides the fake implementation
    # gives it (the eager op returns a token-major gate's gradient as a view)
    gate = M._prepare_gate(compress_attn_weight, q)
    gate = gate.contiguous() if gate is not None else None
    q, k, v = (x.contiguous() for x in (q, k, v))
    vbs = M._i32(variable_block_sizes, q.device)
    qvbs = M._i32(q_variable_block_sizes, q.device)
    save = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad or
                                        (gate is not None and gate.requires_grad))
    scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    return vsa_fwd(q, k, v, gate, vbs, qvbs, topk, be, scale, save)[0]


# ---------------------------------------------------------------------------
# Explicit route
# ---------------------------------------------------------------------------

@torch.library.custom_op("vsa_mi355x::sparse_fwd", mutates_args=(), device_types="cuda")
def sparse_fwd(q: Tensor, k: Tensor, v: Tensor, selected: Tensor, vbs: Tensor, be: int,
               scale: float, save: bool) -> Tuple[Tensor, Tensor]:
    """(out, lse); lse is an empty placeholder without ``save``."""
    q, k, v = (M._aligned16(x) for x in (q, k, v))
    with torch.cuda.device(q.device):
        out, lse, _ = M.sparse_forward(q, k, v, selected, vbs, be, scale, want_lse=save)
    return out, (lse if save else _empty(q, torch.float32))


@sparse_fwd.register_fake
def _(q, k, v, selected, vbs, be, scale, save):
    b, h, sq, _ = q.shape
    lse = (q.new_empty((b, h, sq), dtype=torch.float32) if save else _empty(q, torch.float32))
    return torch.empty_like(q), lse


@torch.library.custom_op("vsa_mi355x::sparse_bwd", mutates_args=(), device_types="cuda")
def sparse_bwd(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor,
               selected: Tensor, vbs: Tensor, be: int, scale: float
               ) -> Tuple[Tensor, Tensor, Tensor]:
    q, k, v = (M._aligned16(x) for x in (q, k, v))
    with torch.cuda.device(q.device):
        dout = M._aligned16(dout.contiguous())
        delta, _, _ = M.backward_prep(out, dout, be)
        return M.sparse_backward(q, k, v, dout, lse, delta, selected, vbs, be, scale)


@sparse_bwd.register_fake
def _(dout, q, k, v, out, lse, selected, vbs, be, scale):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _sparse_setup(ctx, inputs, output):
    q, k, v, selected, vbs, be, scale, save = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, selected, vbs)
    ctx.be, ctx.scale = be, scale


def _sparse_backward(ctx, dout, _):
    q, k, v, out, lse, selected, vbs = ctx.saved_tensors
    dq, dk, dv = sparse_bwd(dout, q, k, v, out, lse, selected, vbs, ctx.be, ctx.scale)
    return dq, dk, dv, None, None, None, None, None


sparse_fwd.register_autograd(_sparse_backward, setup_context=_sparse_setup)


def mi355x_sparse_attention(q: Tensor, k: Tensor, v: Tensor, selected: Tensor,
                            variable_block_sizes: Tensor, *, block_size,
                            sm_scale: Optional[float] = None) -> Tensor:
    """``vsa_mi355x.mi355x_sparse_attention`` (triton_impl.py:1626-1652) through
    the custom ops: the same checks, values and gradients."""
    be = M.as_block_elements(block_size)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape [batch, heads, seq_len, dim]")
    M._check_device_path(q, k, v, be, coarse=False)
    M._validate_route(q, k, selected, variable_block_sizes, be)
    if q.shape[0] * q.shape[1] == 0 or M._padded(q, k, be) is not None:
        return M.mi355x_sparse_attention(q, k, v, selected, variable_block_sizes,
                                         block_size=block_size, sm_scale=sm_scale)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    q, k, v = (x.contiguous() for x in (q, k, v))
    sel = M._i32(selected, q.device)
    vbs = M._i32(variable_block_sizes, q.device)
    save = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    return sparse_fwd(q, k, v, sel, vbs, be, float(scale), save)[0]
