"""Query and key/value sequences of different lengths (the reference's checks
only ask both to be multiples of the block volume, common.py:97-134): the full
op and the explicit-route executor against the oracle, for shorter and longer
key sequences, bf16 and fp32, native and padded block volumes and head dims."""

import math

import pytest
import torch

from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _check(a, e, what, dtype):
    # north_star bars: bf16 max-abs 2e-2 / rel-L2 1e-2, fp32 1e-4 / 1e-4
    tol = (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 1e-2)
    a, e = a.detach().float().cpu(), e.detach().float().cpu()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    assert torch.isfinite(a).all(), what
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    print(f"  {what}: max-abs {diff:.2e} rel-L2 {rel:.2e}", flush=True)
    assert diff <= tol[0] and rel <= tol[1], f"{what}: max-abs {diff:.3e} rel-L2 {rel:.3e}"


CASES = [((4, 8, 8), 128, 3, 7, 2, torch.bfloat16, "full"),
         ((4, 8, 8), 128, 9, 4, 3, torch.bfloat16, None),
         ((1, 1, 64), 64, 6, 11, 4, torch.bfloat16, "token"),
         ((1, 1, 128), 256, 5, 3, 2, torch.bfloat16, None),
         ((3, 3, 3), 80, 7, 5, 3, torch.bfloat16, "full"),
         ((2, 8, 8), 128, 4, 9, 3, torch.float32, "full"),
         ((1, 1, 64), 256, 8, 3, 2, torch.float32, None)]


@pytest.mark.parametrize("block,D,nq,nk,topk,dtype,gate_kind", CASES)
def test_full_op_with_different_query_and_key_lengths(block, D, nq, nk, topk, dtype, gate_kind):
    from vsa_mi355x import mi355x as M
    be = math.prod(block)
    B, H = 1, 2
    print(f"cross-length block={block} D={D} Sq={nq * be} Skv={nk * be} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(nq * 100 + nk + D)
    q = torch.randn(B, H, nq * be, D, generator=g, device=DEV, dtype=dtype)
    k, v = (torch.randn(B, H, nk * be, D, generator=g, device=DEV, dtype=dtype) for _ in range(2))
    do = torch.randn_like(q)
    gate = None
    if gate_kind == "full":
        gate = torch.rand(B, H, nq * be, D, generator=g, device=DEV, dtype=dtype)
    elif gate_kind == "token":
        gate = torch.rand(B, H, nq * be, 1, generator=g, device=DEV, dtype=dtype)
    kvbs = torch.full((nk,), be, dtype=torch.int32, device=DEV)
    kvbs[-1] = max(1, be - 9)
    qvbs = torch.full((nq,), be, dtype=torch.int32, device=DEV)
    qvbs[0] = max(1, be - 3)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    gl = gate.clone().requires_grad_() if gate is not None else None
    out = M.mi355x_vsa(*leaves, kvbs, qvbs, topk, block, gl)
    assert out.shape == q.shape
    wrt = leaves + ([gl] if gl is not None else [])
    grads = torch.autograd.grad(out, wrt, do)
    _, sel = M.mi355x_route(q, k, v, kvbs, qvbs, topk, block)
    assert tuple(sel.shape) == (B, H, nq, topk)
    rl = [t.cpu().clone().requires_grad_() for t in (q, k, v)]
    rg = gate.cpu().clone().requires_grad_() if gate is not None else None
    ref = O.torch_vsa(*rl, kvbs.cpu(), qvbs.cpu(), topk, block, rg, selected=sel.cpu().long())
    rgrads = torch.autograd.grad(ref, rl + ([rg] if rg is not None else []), do.cpu())
    _check(out, ref, "out", dtype)
    for n, a, e in zip(("dq", "dk", "dv", "dgate"), grads, rgrads):
        _check(a, e, n, dtype)


# (B, H, be, D, nq, nk); the last two run the 8-wave forward and dQ (>= 256 query blocks)
@pytest.mark.parametrize("B,H,be,D,nq,nk", [(2, 2, 256, 128, 2, 6), (2, 2, 64, 64, 12, 5),
                                           (2, 2, 128, 256, 3, 4), (1, 64, 256, 128, 4, 6),
                                           (1, 32, 256, 64, 8, 3)])
def test_explicit_route_with_different_query_and_key_lengths(B, H, be, D, nq, nk):
    from vsa_mi355x import mi355x as M
    topk = 3
    g = torch.Generator().manual_seed(be + nq + nk)
    q = torch.randn(B, H, nq * be, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(B, H, nk * be, D, generator=g).to(torch.bfloat16) for _ in range(2))
    do = torch.randn(q.shape, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(nk, generator=g)[:topk] for _ in range(B * H * nq)])
    sel = sel.reshape(B, H, nq, topk).to(torch.int32)
    vbs = torch.full((nk,), be, dtype=torch.int32)
    vbs[1] = be // 3
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be))
    grads = torch.autograd.grad(out, leaves, do.to(DEV))
    rl = [t.clone().requires_grad_() for t in (q, k, v)]
    ref = O.sparse_attention(*rl, sel, vbs, block_size=(1, 1, be))
    rgrads = torch.autograd.grad(ref, rl, do)
    _check(out, ref, "out", torch.bfloat16)
    for n, a, e in zip(("dq", "dk", "dv"), grads, rgrads):
        _check(a, e, n, torch.bfloat16)
