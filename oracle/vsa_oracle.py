"""CPU oracle for the MI355X VSA hot path.  TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``vsa_mi355x.mi355x_vsa`` / ``vsa_mi355x.mi355x_sparse_attention``)
runs the HIP kernels and fails loudly when they are missing.

It restates, in plain PyTorch (fp32 math on the CPU unless the input dtype says
otherwise), the semantics of the reference ``ita9naiwa/simple-vsa``:

* ``vsa/common.py``        block volume, valid mask, block mean, validation,
                           coarse branch, Top-K mask, masked-fill dense oracle
* ``vsa/torch_impl.py``    the gather oracle ``torch_vsa``
* ``vsa/triton_impl.py``   the explicit-route contract (int32 routes, base-2 LSE)
                           and the compact CSR inverse routing

Every function cites the reference lines it follows.  How each is pinned
(independently of retyping its own formula) is listed in ``PINNING`` below and
exercised by ``tests/test_oracle.py``.

Extra hooks that the reference does not have, for parity testing only:

* ``torch_vsa(..., selected=...)`` overrides the Top-K route so the oracle can be
  driven by exactly the route the GPU chose (Top-K ties are resolved by a
  documented rule on the GPU, while ``torch.topk`` leaves tie order open);
* ``torch_vsa(..., head_chunk=h)`` evaluates the fine branch ``h`` heads at a
  time so large configurations fit in host memory (heads are independent);
* ``video_sparse_attn(..., selected=...)`` does for the dense oracle what
  ``selected`` does for ``torch_vsa``;
* ``gather=`` on ``torch_vsa`` / ``sparse_attention`` picks the fine branch's
  gather (below).

One deliberate precision difference from ``torch_impl.py``: the fine branch
gathers from fp32 copies of k and v by default, so gradients of a key block
shared by many query blocks are summed in fp32 and rounded once (see
``_fine_branch``); ``gather="as_written"`` restates torch_impl.py's own
``torch.gather`` over the broadcast block view instead, and the tests hold the
GPU gradients to both.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple, Union

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

# Which independent check pins each function (tests/test_oracle.py and
# tests/test_oracle_rounding.py hold them).  No golden vectors of the reference
# exist (its tests hold none), so every pin is a known answer from the
# reference's own tests, a textbook identity or a brute force; each check also
# catches at least one planted mistake.
PINNING = {
    "as_block_elements": "closed form; int -> cube (tests/test_torch_vsa.py:59-72 KAT)",
    "valid_token_mask": "closed form pos < vbs; brute force loop",
    "block_mean": "KAT [2.0, 2.0] ignoring padding 999 (tests/test_common.py:81-88); "
                  "explicit per-block mean (tests/test_common.py:63-78); bf16 / fp16: "
                  "T(fp64 sum / count) brute force (planted: fp32 result, padded divisor)",
    "validate_vsa_inputs": "error-text KATs (tests/test_torch_vsa.py:112-130)",
    "coarse_branch_compact": "fp64: equals F.scaled_dot_product_attention on pooled tokens; "
                             "compact == expanded (tests/test_common.py:91-112); bf16 / fp16: "
                             "scores T(T(dot) * scale), P = T(softmax), out_c = T(P v_c) by fp64 "
                             "brute force from the T operands (planted: fp32 scores, fp32 "
                             "softmax, fp32 out_c, one rounding of the scores)",
    "topk_reference": "brute-force full sort; torch.topk on tie-free rows; exactly tk per row "
                      "(tests/test_common.py:165-172)",
    "video_sparse_attn": "topk = Kb with full blocks == SDPA (tests/test_common.py:115-130); "
                         "gate 0 / gate 2 (tests/test_common.py:145-162); out == compress + "
                         "sparse; bf16 / fp16 route == torch.topk of the brute-force T scores, "
                         "ties included (planted: routing on fp32 scores)",
    "torch_vsa": "== masked-fill video_sparse_attn at 1e-5, full / padded / gate / int block "
                 "(tests/test_torch_vsa.py:12-72); unselected blocks get gradient (89-109); "
                 "fp64 gradcheck; bf16 / fp16 output == T(float(out_c) * float(gate) + out_s) "
                 "by fp64 brute force (planted: out_c kept in fp32); fp32 gather and "
                 "the as-written torch.gather of torch_impl.py measured against fp64 on a "
                 "Zipf hot-key route (planted: an indexing gather that sums in T)",
    "sparse_attention_reference": "hot-KV dense per-block softmax (tests/test_helion_vsa.py:332-403); "
                                  "all blocks selected == SDPA; LSE2 == log2 sum exp2 brute force",
    "sparse_attention": "fp64 gradcheck; == torch_vsa fine branch with the same route",
    "csr_reference": "brute force selected.eq(kv).nonzero() (tests/test_triton_vsa.py:163-196)",
}


# ----------------------------------------------------------------------------
# Block bookkeeping (vsa/common.py:39-52)
# ----------------------------------------------------------------------------

def as_block_elements(block_size: Union[int, Sequence[int]]) -> int:
    """Block volume: an int is a cube edge, a tuple is multiplied (common.py:39-42)."""
    if isinstance(block_size, int):
        return block_size * block_size * block_size
    return int(math.prod(block_size))


def valid_token_mask(variable_block_sizes: Tensor, block_elements: int) -> Tensor:
    """``[nb, be]`` bool, True where ``slot < vbs[block]`` (common.py:45-52)."""
    pos = torch.arange(block_elements, device=variable_block_sizes.device)
    return pos[None, :] < variable_block_sizes[:, None]


def block_mean(x: Tensor, variable_block_sizes: Tensor, block_elements: int) -> Tensor:
    """Mean over the valid tokens of each block, fp32 sum, stored in x.dtype
    (common.py:55-82)."""
    b, h, s, d = x.shape
    nb = s // block_elements
    blocks = _acc(x.reshape(b, h, nb, block_elements, d))
    valid = valid_token_mask(variable_block_sizes, block_elements).view(1, 1, nb, block_elements, 1)
    summed = (blocks * valid).sum(dim=3)
    counts = variable_block_sizes.clamp(min=1).to(summed.dtype).view(1, 1, nb, 1)
    return (summed / counts).to(x.dtype)


def validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, block_elements):
    """Shape / length contract with the reference's error texts (common.py:97-134)."""
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


# ----------------------------------------------------------------------------
# Coarse (compression) branch (vsa/common.py:137-197)
# ----------------------------------------------------------------------------

def _acc(x: Tensor) -> Tensor:
    """The reference's ``.float()`` promotion (fp32 accumulation type).  fp64
    inputs stay fp64 so ``torch.autograd.gradcheck`` can pin the backward; the
    reference itself never sees fp64."""
    return x if x.dtype == torch.float64 else x.float()


def _mT(x: Tensor) -> Tensor:
    # Materialise transposes before batched products (keeps every matmul operand
    # contiguous, which is also what the GPU box needs for bf16 bmm).
    return x.transpose(-2, -1).contiguous()


def coarse_branch_compact(q, k, v, variable_block_sizes, q_variable_block_sizes,
                          block_elements, scale) -> Tuple[Tensor, Tensor]:
    """Pooled scores and one compression vector per query block, all in the input
    dtype: ``scores = T(T(q_c k_c^T) * scale)``, ``P = softmax(scores)`` in T,
    ``out_c = T(P v_c)`` (common.py:137-167)."""
    q_c = block_mean(q, q_variable_block_sizes, block_elements)
    k_c = block_mean(k, variable_block_sizes, block_elements)
    v_c = block_mean(v, variable_block_sizes, block_elements)
    scores = torch.matmul(q_c, _mT(k_c)) * scale
    attn = torch.softmax(scores, dim=-1)
    out_c_blocks = torch.matmul(attn, v_c)
    return scores, out_c_blocks


def coarse_branch(q, k, v, variable_block_sizes, q_variable_block_sizes, block_elements, scale):
    """Coarse branch with the compact output expanded to every token, padding
    included (common.py:170-197)."""
    b, h, sq, d = q.shape
    qb = sq // block_elements
    scores, out_c_blocks = coarse_branch_compact(
        q, k, v, variable_block_sizes, q_variable_block_sizes, block_elements, scale)
    out_c = out_c_blocks.view(b, h, qb, 1, d).expand(b, h, qb, block_elements, d).reshape(b, h, sq, d)
    return scores, out_c


def topk_block_mask(scores: Tensor, topk: int) -> Tensor:
    """Exactly ``topk`` True per row, via ``torch.topk`` + scatter (common.py:85-94)."""
    topk = min(topk, scores.shape[-1])
    idx = torch.topk(scores, topk, dim=-1).indices
    return torch.zeros_like(scores, dtype=torch.bool).scatter_(-1, idx, True)


def topk_reference(scores, topk: int) -> np.ndarray:
    """Top-K ids per row with a fixed tie rule: larger score first, then the
    smaller key-block id.  Returns int32 ``[..., topk]`` in that order.

    The reference calls ``scores.topk(topk)`` (torch_impl.py:85,
    triton_impl.py:1710), whose tie order is implementation-defined; on rows
    without a tie at the k-th value both agree on the selected set."""
    s = scores.detach().float().cpu().numpy() if isinstance(scores, Tensor) else np.asarray(scores, np.float32)
    lead = s.shape[:-1]
    kb = s.shape[-1]
    flat = s.reshape(-1, kb)
    out = np.empty((flat.shape[0], topk), dtype=np.int32)
    ids = np.arange(kb)
    for r in range(flat.shape[0]):
        # lexsort: last key is primary -> (-value) primary, id secondary.
        order = np.lexsort((ids, -flat[r].astype(np.float64)))
        out[r] = order[:topk]
    return out.reshape(*lead, topk)


# ----------------------------------------------------------------------------
# Dense masked-fill oracle (vsa/common.py:200-285)
# ----------------------------------------------------------------------------

def video_sparse_attn(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, *,
                      block_size=64, compress_attn_weight=None, sm_scale=None, return_aux=False,
                      selected: Optional[Tensor] = None):
    """Full ``q k^T`` masked to the Top-K blocks and valid keys (common.py:200-285).

    ``selected`` (test hook, ``[B, H, Qb, topk]``) replaces the Top-K of the
    coarse scores (common.py:85-94, 250) so the oracle can follow a route the
    GPU chose; the block mask is then that route scattered into a bool grid."""
    be = as_block_elements(block_size)
    validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, be)
    b, h, sq, d = q.shape
    skv = k.shape[2]
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(d)
    vbs = variable_block_sizes.to(q.device)
    qvbs = q_variable_block_sizes.to(q.device)
    coarse_scores, out_c = coarse_branch(q, k, v, vbs, qvbs, be, scale)
    if selected is None:
        block_mask = topk_block_mask(coarse_scores, topk)
    else:
        block_mask = torch.zeros_like(coarse_scores, dtype=torch.bool).scatter_(
            -1, selected.to(q.device).long(), True)
    token_sel = block_mask.repeat_interleave(be, dim=2).repeat_interleave(be, dim=3)
    kv_valid = valid_token_mask(vbs, be).reshape(skv)
    allowed = token_sel & kv_valid.view(1, 1, 1, skv)
    fine = torch.matmul(_acc(q), _mT(_acc(k))) * scale
    fine = fine.masked_fill(~allowed, float("-inf"))
    out_s = torch.matmul(torch.softmax(fine, dim=-1), _acc(v))
    if compress_attn_weight is not None:
        out = out_c * _acc(compress_attn_weight) + out_s
    else:
        out = out_c + out_s
    out = out.to(q.dtype)
    if return_aux:
        return out, {"coarse_scores": coarse_scores, "block_mask": block_mask,
                     "out_compress": out_c.to(q.dtype), "out_sparse": out_s.to(q.dtype)}
    return out


# ----------------------------------------------------------------------------
# Gather oracle torch_vsa (vsa/torch_impl.py:33-113)
# ----------------------------------------------------------------------------

def _gather_blocks(x: Tensor, block_ids: Tensor, be: int) -> Tensor:
    """``[B,H,Qb,tk,be,D]`` copy of the selected blocks (torch_impl.py:33-46)."""
    b, h, s, d = x.shape
    blocks = x.reshape(b, h, s // be, be, d)
    bi = torch.arange(b, device=x.device).view(b, 1, 1, 1)
    hi = torch.arange(h, device=x.device).view(1, h, 1, 1)
    return blocks[bi, hi, block_ids.long()]


def _gather_blocks_as_written(x: Tensor, block_ids: Tensor, be: int) -> Tensor:
    """The same ``[B,H,Qb,tk,be,D]`` blocks by the reference's own mechanism
    (torch_impl.py:33-46): ``torch.gather`` along the key-block axis of the
    block view broadcast over the query blocks.  Its backward scatters each
    query block's gradient into that broadcast view in x's dtype, and the
    expand's backward then sums over the query blocks (fp32 accumulation
    inside torch's reduction, one rounding to x's dtype at the end)."""
    b, h, s, d = x.shape
    qb, tk = block_ids.shape[-2:]
    blocks = x.reshape(b, h, s // be, be, d)
    source = blocks.unsqueeze(2).expand(b, h, qb, s // be, be, d)
    index = block_ids.long().view(b, h, qb, tk, 1, 1).expand(b, h, qb, tk, be, d)
    return torch.gather(source, 3, index)


def _fine_branch(q, k, v, selected, vbs, be, scale, gather: str = "fp32"):
    """Sparse fine branch in fp32 over the valid keys of the selected blocks
    (torch_impl.py:86-106).  Returns ``(out_s fp32 [B,H,Sq,D], lse2 [B,H,Sq])``.

    ``gather="fp32"`` (the default) gathers from fp32 copies of k and v;
    ``gather="as_written"`` gathers in T and then promotes, as torch_impl.py:86-87
    does.  Forward values are identical; the backward differs in where a shared
    key block's per-query-block gradients are rounded (see below)."""
    b, h, sq, d = q.shape
    qb = sq // be
    tk = selected.shape[-1]
    # Gather from fp32 copies by default: the backward then sums the
    # per-query-block gradients of a shared key block in fp32 and rounds once.
    # The reference's gather (torch_impl.py:43-46, then .float()) rounds each
    # query block's contribution to T before that sum; on a Zipf(1.2) route
    # with a key block of 191 in-edges this puts dk / dv at relative L2 2.4e-3
    # from fp64 against 1.7e-3 for the fp32 gather
    # (tests/test_oracle_rounding.py), both far inside the 1e-2 parity bar.
    if gather == "as_written":
        sel_k = _acc(_gather_blocks_as_written(k, selected, be))
        sel_v = _acc(_gather_blocks_as_written(v, selected, be))
    elif gather == "fp32":
        sel_k = _gather_blocks(_acc(k), selected, be)
        sel_v = _gather_blocks(_acc(v), selected, be)
    else:
        raise ValueError(f"gather must be 'fp32' or 'as_written', got {gather!r}")
    valid_sel = valid_token_mask(vbs, be)[selected.long()]          # [B,H,Qb,tk,be]
    query = _acc(q.reshape(b, h, qb, be, d))
    keys = sel_k.reshape(b, h, qb, tk * be, d)
    s = torch.matmul(query, _mT(keys)) * scale                       # [B,H,Qb,be,tk*be]
    s = s.masked_fill(~valid_sel.reshape(b, h, qb, 1, tk * be), float("-inf"))
    p = torch.softmax(s, dim=-1)
    out_s = torch.matmul(p, sel_v.reshape(b, h, qb, tk * be, d)).reshape(b, h, sq, d)
    lse2 = (torch.logsumexp(s, dim=-1) * (1.0 / math.log(2.0))).reshape(b, h, sq)
    return out_s, lse2


def torch_vsa(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, block_size=64,
              compress_attn_weight=None, *, selected: Optional[Tensor] = None,
              head_chunk: Optional[int] = None, gather: str = "fp32"):
    """VSA forward, differentiable (torch_impl.py:49-113).

    ``selected`` (test hook) replaces the ``scores.topk`` route (torch_impl.py:85);
    ``head_chunk`` evaluates the fine branch a few heads at a time; ``gather``
    picks the fine branch's gather (``_fine_branch``)."""
    be = as_block_elements(block_size)
    validate_vsa_inputs(q, k, v, variable_block_sizes, q_variable_block_sizes, topk, be)
    b, h, sq, d = q.shape
    scale = 1.0 / math.sqrt(d)
    vbs = variable_block_sizes.to(q.device)
    qvbs = q_variable_block_sizes.to(q.device)
    scores, out_c = coarse_branch(q, k, v, vbs, qvbs, be, scale)
    if selected is None:
        selected = scores.topk(topk, dim=-1).indices
    selected = selected.to(q.device).long()
    if head_chunk is None or head_chunk >= h:
        out_s, _ = _fine_branch(q, k, v, selected, vbs, be, scale, gather)
    else:
        parts = [
            _fine_branch(q[:, i:i + head_chunk], k[:, i:i + head_chunk], v[:, i:i + head_chunk],
                         selected[:, i:i + head_chunk], vbs, be, scale, gather)[0]
            for i in range(0, h, head_chunk)
        ]
        out_s = torch.cat(parts, dim=1)
    if compress_attn_weight is not None:
        out = out_c * _acc(compress_attn_weight) + out_s
    else:
        out = out_c + out_s
    return out.to(q.dtype)


# ----------------------------------------------------------------------------
# Explicit-route sparse executor contract (vsa/triton_impl.py:358-473, 1583-1652)
# ----------------------------------------------------------------------------

def sparse_attention_reference(q, k, v, selected, variable_block_sizes, block_elements, scale,
                               gather: str = "fp32"):
    """Fine branch only, on a caller-supplied route; fp32 output and the base-2
    log-sum-exp ``lse2 = m + log2(l)`` the fine kernels save
    (triton_impl.py:189-192, 352-355)."""
    return _fine_branch(q, k, v, selected.long(), variable_block_sizes.to(q.device),
                        block_elements, scale, gather)


def sparse_attention(q, k, v, selected, variable_block_sizes, *, block_size, sm_scale=None,
                     gather: str = "fp32"):
    """Differentiable explicit-route oracle, output in the input dtype
    (triton_sparse_attention, triton_impl.py:1626-1652)."""
    be = as_block_elements(block_size)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    out, _ = sparse_attention_reference(q, k, v, selected, variable_block_sizes, be, scale,
                                        gather)
    return out.to(q.dtype)


# ----------------------------------------------------------------------------
# CSR inverse routing (vsa/triton_impl.py:544-595)
# ----------------------------------------------------------------------------

def csr_reference(selected, key_blocks: int):
    """KV-block -> query-block CSR per (batch, head), canonical order.

    ``counts[bh, kv]`` = number of (q-block, slot) edges naming ``kv``;
    ``offsets`` = exclusive prefix sum of ``counts`` per (b, h);
    ``inverse[bh, offsets[kv]:offsets[kv]+counts[kv]]`` = the q-blocks that chose
    ``kv``, ascending (the reference's atomic-cursor scatter leaves this order
    open; its own test sorts each segment, tests/test_triton_vsa.py:190-195).
    Storage is exactly ``Qb*tk`` edges per (b, h) (triton_impl.py:577-582)."""
    sel = selected.detach().cpu().numpy() if isinstance(selected, Tensor) else np.asarray(selected)
    sel = sel.astype(np.int64)
    b, h, qb, tk = sel.shape
    counts = np.zeros((b, h, key_blocks), np.int32)
    offsets = np.zeros((b, h, key_blocks), np.int32)
    inverse = np.zeros((b, h, qb * tk), np.int32)
    qids = np.repeat(np.arange(qb), tk)
    for bi in range(b):
        for hi in range(h):
            kv = sel[bi, hi].reshape(-1)
            counts[bi, hi] = np.bincount(kv, minlength=key_blocks)
            offsets[bi, hi] = np.concatenate(([0], np.cumsum(counts[bi, hi])[:-1]))
            order = np.lexsort((qids, kv))        # by kv, then ascending q-block
            inverse[bi, hi] = qids[order]
    return inverse, offsets, counts
