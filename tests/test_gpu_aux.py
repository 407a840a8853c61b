"""GPU parity of ``video_sparse_attn``'s keyword surface on ``mi355x_vsa``:
``sm_scale`` (one scale for the coarse scores and the fine branch,
common.py:225, 241, 262) and ``return_aux`` (``coarse_scores``,
``block_mask``, ``out_compress``, ``out_sparse``, common.py:277-284).

The oracle is the dense masked-fill ``video_sparse_attn`` restatement, driven
by the GPU's own route for the tensors (Top-K ties are resolved by a fixed rule
on the GPU and left open by ``torch.topk``) and by its own Top-K for the mask
comparison on rows without a tie.  Bars: the north star's max-abs 2e-2 and
relative L2 1e-2 for bf16 tensors, bit-exact masks and routes."""

import pytest
import torch

from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, REL_L2 = 2e-2, 1e-2
AUX_KEYS = ("coarse_scores", "block_mask", "out_compress", "out_sparse")


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _close(actual, expected, what, max_abs=MAX_ABS, rel_l2=REL_L2):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{what}: non-finite"
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    print(f"  {what}: max-abs {diff:.2e} rel-L2 {rel:.2e}", flush=True)
    assert diff <= max_abs and rel <= rel_l2, f"{what}: max-abs {diff:.3e}, rel-L2 {rel:.3e}"


def _case(seed, nb, be, d, qvbs, kvbs, gate="full", h=2, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    shape = (1, h, nb * be, d)
    q, k, v, do = (torch.randn(shape, generator=g).to(dtype) for _ in range(4))
    gt = None
    if gate == "full":
        gt = torch.rand(shape, generator=g).to(dtype)
    elif gate == "token":
        gt = torch.rand((1, h, nb * be, 1), generator=g).to(dtype)
    return q, k, v, do, gt, torch.tensor(qvbs), torch.tensor(kvbs)


def _gpu_run(q, k, v, gate, qvbs, kvbs, topk, block, sm_scale, do=None):
    from vsa_mi355x import mi355x as M
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    g = gate.to(DEV).requires_grad_() if gate is not None else None
    out, aux = M.mi355x_vsa(*leaves, kvbs.to(DEV), qvbs.to(DEV), topk, block, g,
                            sm_scale=sm_scale, return_aux=True)
    grads = None
    if do is not None:
        grads = torch.autograd.grad(out, leaves + ([g] if g is not None else []), do.to(DEV))
    torch.cuda.synchronize()
    return out, aux, grads


def _untied_rows(scores, topk):
    """Rows whose topk-th and (topk+1)-th largest scores differ."""
    s = scores.float().sort(dim=-1, descending=True).values
    if topk == s.shape[-1]:
        return torch.ones(s.shape[:-1], dtype=torch.bool)
    return s[..., topk - 1] != s[..., topk]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_aux_and_sm_scale_match_the_dense_oracle_padded_gated_block_256(dtype):
    """Padded, gated block-256 case at sm_scale 0.07: output, gradients and
    every aux entry against video_sparse_attn(..., sm_scale=0.07,
    return_aux=True) on the GPU's route; the block mask bit-exact against the
    oracle's own Top-K on every untied row."""
    qvbs = [256, 256, 200, 256, 131, 256]
    kvbs = [256, 97, 256, 256, 256, 180]
    q, k, v, do, gate, qv, kv = _case(3, 6, 256, 128, qvbs, kvbs, dtype=dtype)
    topk, block, scale = 3, (4, 8, 8), 0.07
    out, aux, grads = _gpu_run(q, k, v, gate, qv, kv, topk, block, scale, do)

    assert set(aux) == set(AUX_KEYS)
    b, h, s, d = q.shape
    assert aux["coarse_scores"].shape == (b, h, 6, 6) and aux["coarse_scores"].dtype == dtype
    assert aux["block_mask"].shape == (b, h, 6, 6) and aux["block_mask"].dtype == torch.bool
    for key in ("out_compress", "out_sparse"):
        assert aux[key].shape == q.shape and aux[key].dtype == dtype, key
    for t in aux.values():
        assert not t.requires_grad and t.device.type == "cuda"
    assert (aux["block_mask"].sum(-1) == topk).all()

    # the route the GPU used is the mask's True entries (ids ascending)
    sel = aux["block_mask"].cpu().nonzero()[:, -1].view(b, h, 6, topk)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, gate)]
    ref, raux = O.video_sparse_attn(*leaves[:3], kv, qv, topk, block_size=block,
                                    compress_attn_weight=leaves[3], sm_scale=scale,
                                    return_aux=True, selected=sel)
    ref_grads = torch.autograd.grad(ref, leaves, do)
    _close(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv", "dgate"), grads, ref_grads):
        _close(a, e, n)
    assert torch.equal(aux["block_mask"].cpu(), raux["block_mask"])
    for key in ("coarse_scores", "out_compress", "out_sparse"):
        assert raux[key].dtype == dtype
        _close(aux[key], raux[key], key)

    # the oracle's own Top-K: same mask on every row whose scores are tied
    # nowhere near the cut and agree bit for bit with the GPU's
    _, own = O.video_sparse_attn(q, k, v, kv, qv, topk, block_size=block,
                                 compress_attn_weight=gate, sm_scale=scale, return_aux=True)
    same = (aux["coarse_scores"].cpu() == own["coarse_scores"]).all(-1)
    rows = same & _untied_rows(own["coarse_scores"], topk)
    assert rows.float().mean() >= 0.5, rows
    assert torch.equal(aux["block_mask"].cpu()[rows], own["block_mask"][rows])


def test_sm_scale_changes_both_branches():
    """sm_scale reaches the coarse scores (scores scale by it exactly up to
    T rounding) and the fine branch (out_sparse differs from the default)."""
    q, k, v, _, gate, qv, kv = _case(7, 4, 64, 64, [64] * 4, [64, 64, 33, 64], gate=None)
    _, a1, _ = _gpu_run(q, k, v, None, qv, kv, 2, (1, 1, 64), None)
    _, a2, _ = _gpu_run(q, k, v, None, qv, kv, 2, (1, 1, 64), 0.5)
    s1, s2 = a1["coarse_scores"].float(), a2["coarse_scores"].float()
    _close(s2, s1 * (0.5 * 64 ** 0.5), "scaled scores", max_abs=4e-2, rel_l2=1e-2)
    assert not torch.equal(a1["out_sparse"], a2["out_sparse"])
    _, ref = O.video_sparse_attn(q, k, v, kv, qv, 2, block_size=(1, 1, 64), sm_scale=0.5,
                                 return_aux=True,
                                 selected=a2["block_mask"].cpu().nonzero()[:, -1].view(1, 2, 4, 2))
    _close(a2["out_sparse"], ref["out_sparse"], "out_sparse at sm_scale 0.5")
    _close(a2["out_compress"], ref["out_compress"], "out_compress at sm_scale 0.5")


def test_aux_is_the_same_with_and_without_grad_and_for_every_gate_kind():
    """The no-grad forward reports the same aux bit for bit; out_sparse does
    not depend on the gate (bf16, per-token, fp32 and no gate), out_compress
    neither."""
    from vsa_mi355x import mi355x as M
    q, k, v, _, gate, qv, kv = _case(11, 5, 128, 128, [128, 128, 77, 128, 128],
                                     [128, 5, 128, 128, 128])
    block = (1, 1, 128)
    _, a_grad, _ = _gpu_run(q, k, v, gate, qv, kv, 2, block, None)
    with torch.no_grad():
        out_ng, a_ng = M.mi355x_vsa(q.to(DEV), k.to(DEV), v.to(DEV), kv.to(DEV), qv.to(DEV), 2,
                                    block, gate.to(DEV), return_aux=True)
    for key in AUX_KEYS:
        assert torch.equal(a_grad[key], a_ng[key]), key
    plain = M.mi355x_vsa(q.to(DEV), k.to(DEV), v.to(DEV), kv.to(DEV), qv.to(DEV), 2, block,
                         gate.to(DEV))
    assert torch.equal(out_ng, plain)
    for g in (gate[..., :1].contiguous(), gate.float(), None):
        _, a, _ = _gpu_run(q, k, v, g, qv, kv, 2, block, None)
        for key in AUX_KEYS:
            assert torch.equal(a[key], a_grad[key]), (key, None if g is None else g.dtype)


def test_aux_on_the_padding_path_and_on_token_major_views():
    """Block volume 48 and head dim 80 run padded kernels: the aux entries come
    back at the caller's shapes and match the oracle.  Token-major views give
    the same aux as contiguous inputs."""
    from vsa_mi355x import mi355x as M
    q, k, v, do, gate, qv, kv = _case(13, 5, 48, 80, [48, 48, 20, 48, 48], [48, 31, 48, 48, 48])
    block = (3, 4, 4)
    out, aux, grads = _gpu_run(q, k, v, gate, qv, kv, 2, block, 0.11, do)
    assert aux["out_sparse"].shape == q.shape and aux["out_compress"].shape == q.shape
    assert aux["coarse_scores"].shape == (1, 2, 5, 5)
    sel = aux["block_mask"].cpu().nonzero()[:, -1].view(1, 2, 5, 2)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, gate)]
    ref, raux = O.video_sparse_attn(*leaves[:3], kv, qv, 2, block_size=block,
                                    compress_attn_weight=leaves[3], sm_scale=0.11,
                                    return_aux=True, selected=sel)
    ref_grads = torch.autograd.grad(ref, leaves, do)
    _close(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv", "dgate"), grads, ref_grads):
        _close(a, e, n)
    for key in ("coarse_scores", "out_compress", "out_sparse"):
        _close(aux[key], raux[key], key)

    # token-major views (the in-place raster path without aux) report the aux
    # of the contiguous op
    q2, k2, v2, _, g2, qv2, kv2 = _case(17, 4, 256, 128, [256] * 4, [256, 256, 100, 256])
    tm = [t.transpose(1, 2).contiguous().transpose(1, 2).to(DEV) for t in (q2, k2, v2, g2)]
    assert all(M._token_major(t) for t in tm)
    o_tm, a_tm = M.mi355x_vsa(*tm[:3], kv2.to(DEV), qv2.to(DEV), 2, (4, 8, 8), tm[3],
                              return_aux=True)
    o_c, a_c = M.mi355x_vsa(q2.to(DEV), k2.to(DEV), v2.to(DEV), kv2.to(DEV), qv2.to(DEV), 2,
                            (4, 8, 8), g2.to(DEV), return_aux=True)
    assert torch.equal(o_tm.contiguous(), o_c)
    for key in AUX_KEYS:
        assert torch.equal(a_tm[key], a_c[key]), key


def test_custom_op_path_takes_sm_scale():
    """vsa_mi355x.ops.mi355x_vsa: sm_scale gives the eager op's values bit for
    bit; return_aux runs the eager op."""
    from vsa_mi355x import mi355x as M
    from vsa_mi355x import ops
    q, k, v, do, gate, qv, kv = _case(19, 4, 128, 64, [128] * 4, [128, 128, 64, 128])
    args = [t.to(DEV) for t in (q, k, v)]
    a = ops.mi355x_vsa(*args, kv.to(DEV), qv.to(DEV), 2, (1, 1, 128), gate.to(DEV), sm_scale=0.2)
    e = M.mi355x_vsa(*args, kv.to(DEV), qv.to(DEV), 2, (1, 1, 128), gate.to(DEV), sm_scale=0.2)
    assert torch.equal(a, e)
    o1, x1 = ops.mi355x_vsa(*args, kv.to(DEV), qv.to(DEV), 2, (1, 1, 128), gate.to(DEV),
                            sm_scale=0.2, return_aux=True)
    assert torch.equal(o1, e) and set(x1) == set(AUX_KEYS)
