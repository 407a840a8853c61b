"""Shapes without a kernel of their own (block volume not in {64, 128, 256},
head_dim not in {64, 128, 256}) run on the kernels after zero padding, and the
head_dim 256 kernels directly; checked against the oracle on the caller's
shapes."""

import math

import pytest
import torch

from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [((1, 1, 16), 64, 8, 3, "full"), ((3, 3, 3), 32, 6, 2, "token"),
         ((1, 1, 100), 128, 6, 3, None), ((2, 4, 4), 80, 10, 4, "full"),
         ((4, 4, 4), 48, 8, 3, "token"), ((4, 8, 8), 96, 4, 2, "full"),
         ((1, 1, 128), 40, 5, 2, None),
         # head_dim 256 kernels (dK/dV split over two workgroups per key tile),
         # natively and for head dims padded up to 256
         ((4, 8, 8), 256, 4, 2, "full"), ((2, 8, 8), 256, 6, 3, "token"),
         ((1, 1, 64), 192, 8, 3, None), ((3, 3, 3), 200, 6, 2, "full")]


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


# bf16 bar of the north star: max-abs 2e-2 and relative L2 1e-2 (inputs kept at
# magnitudes where one bf16 ulp of an output is below the max-abs bar)
def _check(a, e, what, max_abs=2e-2, rel_l2=1e-2):
    a, e = a.detach().float().cpu(), e.detach().float().cpu()
    assert torch.isfinite(a).all(), what
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    assert diff <= max_abs and rel <= rel_l2, f"{what}: max-abs {diff:.3e} rel-L2 {rel:.3e}"


@pytest.mark.parametrize("block,D,nb,topk,gate_kind", CASES)
def test_padded_shapes_match_oracle(block, D, nb, topk, gate_kind):
    _full_op_case(block, D, nb, topk, gate_kind)


# An int block_size is the edge of a cube of tokens (tests/test_torch_vsa.py:59-72):
# 2 -> 8 tokens (with head_dim 8, as there), 4 -> 64 (a kernel of its own), 5 -> 125.
@pytest.mark.parametrize("block,D,nb,topk,gate_kind", [(2, 8, 3, 2, None), (4, 64, 6, 3, "full"),
                                                       (5, 32, 4, 2, "token")])
def test_int_block_size_is_a_cube(block, D, nb, topk, gate_kind):
    _full_op_case(block, D, nb, topk, gate_kind)


def _full_op_case(block, D, nb, topk, gate_kind):
    from vsa_mi355x import mi355x as M
    be = M.as_block_elements(block)
    B, H, S = 1, 2, be * nb
    g = torch.Generator(device=DEV).manual_seed(be * 1000 + D)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = None
    if gate_kind == "full":
        gate = torch.rand(B, H, S, D, generator=g, device=DEV, dtype=torch.bfloat16)
    elif gate_kind == "token":
        gate = torch.rand(B, H, S, 1, generator=g, device=DEV, dtype=torch.bfloat16)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = max(1, be - 5)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    gl = gate.clone().requires_grad_() if gate is not None else None
    out = M.mi355x_vsa(*leaves, vbs, vbs, topk, block, gl)
    assert out.shape == q.shape
    wrt = leaves + ([gl] if gl is not None else [])
    grads = torch.autograd.grad(out, wrt, do)
    _, sel = M.mi355x_route(q, k, v, vbs, vbs, topk, block)
    assert sel.shape == (B, H, nb, topk)
    rl = [t.cpu().clone().requires_grad_() for t in (q, k, v)]
    rg = gate.cpu().clone().requires_grad_() if gate is not None else None
    ref = O.torch_vsa(*rl, vbs.cpu(), vbs.cpu(), topk, block, rg, selected=sel.cpu().long())
    rgrads = torch.autograd.grad(ref, rl + ([rg] if rg is not None else []), do.cpu())
    _check(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv", "dgate"), grads, rgrads):
        _check(a, e, n)


@pytest.mark.parametrize("be,D", [(16, 64), (100, 40), (64, 96)])
def test_padded_explicit_route_matches_oracle(be, D):
    from vsa_mi355x import mi355x as M
    B, H, nb, topk = 1, 2, 7, 3
    S = be * nb
    g = torch.Generator(device=DEV).manual_seed(be + D)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    sel = torch.stack([torch.randperm(nb, generator=torch.Generator().manual_seed(i))[:topk]
                       for i in range(B * H * nb)]).reshape(B, H, nb, topk)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[2] = be // 2
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be),
                                    sm_scale=0.1)
    grads = torch.autograd.grad(out, leaves, do)
    rl = [t.cpu().clone().requires_grad_() for t in (q, k, v)]
    ref = O.sparse_attention(*rl, sel, vbs, block_size=(1, 1, be), sm_scale=0.1)
    rgrads = torch.autograd.grad(ref, rl, do.cpu())
    _check(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv"), grads, rgrads):
        _check(a, e, n)
