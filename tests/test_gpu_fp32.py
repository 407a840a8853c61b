"""fp32 inputs on the GPU (the reference's GPU path accepts fp32,
triton_impl.py:375-376): pooling, coarse attention, Top-K, the fp32 fine
kernels and the backward, checked against the oracle at the north star's fp32
bar (max-abs and relative L2 1e-4).  The oracle computes in fp32 on the CPU and
is driven by the GPU's own route, so the only differences left are fp32
summation orders."""

import math

import pytest
import torch

from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = torch.float32

# (block, head_dim, blocks, topk, gate): every (block volume, head dim) kernel
# pair, the three gate layouts, and shapes padded onto the kernels
CASES = [((1, 1, 64), 64, 12, 3, None), ((1, 1, 64), 128, 9, 4, "full"),
         ((1, 1, 64), 256, 6, 2, "token"), ((2, 8, 8), 64, 7, 3, "token"),
         ((2, 8, 8), 128, 8, 3, None), ((2, 8, 8), 256, 5, 2, "full"),
         ((4, 8, 8), 64, 5, 2, "full"), ((4, 8, 8), 128, 6, 3, "token"),
         ((4, 8, 8), 256, 4, 2, None), ((3, 3, 3), 80, 9, 3, "full"),
         ((1, 1, 100), 40, 6, 2, "token"), ((2, 4, 4), 192, 7, 3, "tokmaj")]


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _check(a, e, what, max_abs=1e-4, rel_l2=1e-4):
    a, e = a.detach().float().cpu(), e.detach().float().cpu()
    assert a.dtype == e.dtype == torch.float32
    assert torch.isfinite(a).all(), what
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    print(f"  {what}: max-abs {diff:.2e} rel-L2 {rel:.2e}", flush=True)
    assert diff <= max_abs and rel <= rel_l2, f"{what}: max-abs {diff:.3e} rel-L2 {rel:.3e}"


def _gate(kind, B, H, S, D, g):
    if kind == "full":
        return torch.rand(B, H, S, D, generator=g, device=DEV, dtype=F32)
    if kind == "token":
        return torch.rand(B, H, S, 1, generator=g, device=DEV, dtype=F32)
    if kind == "tokmaj":  # the gate producer's [B, S, H, D] output seen per head
        return torch.rand(B, S, H, D, generator=g, device=DEV, dtype=F32).transpose(1, 2)
    return None


@pytest.mark.parametrize("block,D,nb,topk,gate_kind", CASES)
def test_fp32_vsa_matches_oracle(block, D, nb, topk, gate_kind):
    from vsa_mi355x import mi355x as M
    be = math.prod(block)
    B, H, S = 1, 2, be * nb
    print(f"fp32 vsa block={block} D={D} nb={nb} topk={topk} gate={gate_kind}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(be * 1000 + D + nb)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=DEV, dtype=F32)
                   for _ in range(4))
    gate = _gate(gate_kind, B, H, S, D, g)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = max(1, be - 5)
    vbs[1] = 1                                  # a block holding a single token
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    gl = gate.detach().clone().requires_grad_() if gate is not None else None
    out = M.mi355x_vsa(*leaves, vbs, vbs, topk, block, gl)
    assert out.dtype == F32 and out.shape == q.shape
    wrt = leaves + ([gl] if gl is not None else [])
    grads = torch.autograd.grad(out, wrt, do)
    _, sel = M.mi355x_route(q, k, v, vbs, vbs, topk, block)
    rl = [t.cpu().clone().requires_grad_() for t in (q, k, v)]
    rg = gate.detach().cpu().clone().requires_grad_() if gate is not None else None
    ref = O.torch_vsa(*rl, vbs.cpu(), vbs.cpu(), topk, block, rg, selected=sel.cpu().long())
    rgrads = torch.autograd.grad(ref, rl + ([rg] if rg is not None else []), do.cpu())
    _check(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv", "dgate"), grads, rgrads):
        _check(a, e, n)
    # deterministic: no atomics anywhere on the path
    leaves2 = [t.clone().requires_grad_() for t in (q, k, v)]
    gl2 = gate.detach().clone().requires_grad_() if gate is not None else None
    out2 = M.mi355x_vsa(*leaves2, vbs, vbs, topk, block, gl2)
    grads2 = torch.autograd.grad(out2, leaves2 + ([gl2] if gl2 is not None else []), do)
    assert torch.equal(out, out2)
    for a, b_ in zip(grads, grads2):
        assert torch.equal(a, b_)


@pytest.mark.parametrize("be,D,scale", [(64, 64, None), (256, 128, -0.05), (128, 256, 0.2),
                                        (16, 96, None)])
def test_fp32_explicit_route_matches_oracle(be, D, scale):
    from vsa_mi355x import mi355x as M
    B, H, nb, topk = 2, 2, 9, 4
    S = be * nb
    print(f"fp32 explicit route be={be} D={D} scale={scale}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(be + D)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g, device=DEV, dtype=F32)
                   for _ in range(4))
    sel = torch.stack([torch.randperm(nb, generator=torch.Generator().manual_seed(i))[:topk]
                       for i in range(B * H * nb)]).reshape(B, H, nb, topk).to(torch.int32)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[2] = be // 2
    vbs[5] = 0      # an empty key block contributes nothing (routes hold 4 distinct blocks)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be),
                                    sm_scale=scale)
    grads = torch.autograd.grad(out, leaves, do)
    rl = [t.cpu().clone().requires_grad_() for t in (q, k, v)]
    ref = O.sparse_attention(*rl, sel, vbs, block_size=(1, 1, be), sm_scale=scale)
    rgrads = torch.autograd.grad(ref, rl, do.cpu())
    _check(out, ref, "out")
    for n, a, e in zip(("dq", "dk", "dv"), grads, rgrads):
        _check(a, e, n)


def test_fp32_lse_matches_oracle():
    """The saved base-2 log-sum-exp of the fp32 forward (used by both backward
    kernels) against the oracle's m + log2(l)."""
    from vsa_mi355x import mi355x as M
    be, D, nb, topk = 128, 128, 6, 3
    S = be * nb
    g = torch.Generator(device=DEV).manual_seed(7)
    q, k, v = (torch.randn(1, 3, S, D, generator=g, device=DEV, dtype=F32) for _ in range(3))
    sel = torch.stack([torch.randperm(nb, generator=torch.Generator().manual_seed(i))[:topk]
                       for i in range(3 * nb)]).reshape(1, 3, nb, topk).to(torch.int32)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[0] = 77
    scale = 1.0 / math.sqrt(D)
    out, lse, _ = M.sparse_forward(q, k, v, sel.to(DEV), vbs.to(DEV), be, scale, want_lse=True)
    ref_out, ref_lse = O.sparse_attention_reference(q.cpu(), k.cpu(), v.cpu(), sel, vbs, be, scale)
    _check(out, ref_out, "out")
    _check(lse, ref_lse, "lse")
