"""Known answers the reference's own tests pin, run on the MI355X kernels:
* all key blocks selected with full blocks => the fine branch is dense softmax
  attention (tests/test_common.py:115-130), checked against fp32 SDPA on the CPU;
* gate 0 => out = out_s, gate 2 => out = 2 out_c + out_s (tests/test_common.py:145-162);
* key blocks no query block routes to still get gradient through the coarse
  branch (tests/test_torch_vsa.py:89-109)."""

import math

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


@pytest.mark.parametrize("be,D,nb,dtype", [(256, 128, 3, torch.bfloat16), (64, 64, 5, torch.bfloat16),
                                          (128, 256, 2, torch.bfloat16), (64, 128, 4, torch.float32)])
def test_all_blocks_selected_is_dense_attention(be, D, nb, dtype):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(be + D)
    B, H, S = 1, 2, nb * be
    q, k, v, do = (torch.randn(B, H, S, D, generator=g).to(dtype) for _ in range(4))
    sel = torch.arange(nb, dtype=torch.int32).expand(B, H, nb, nb).contiguous()
    vbs = torch.full((nb,), be, dtype=torch.int32)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be))
    grads = torch.autograd.grad(out, leaves, do.to(DEV))
    rl = [t.float().requires_grad_() for t in (q, k, v)]
    ref = F.scaled_dot_product_attention(*rl)          # fp32, CPU, scale 1/sqrt(D)
    rgrads = torch.autograd.grad(ref, rl, do.float())
    tol = (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 1e-2)
    for n, a, e in zip(("out", "dq", "dk", "dv"), (out,) + tuple(grads), (ref,) + tuple(rgrads)):
        a = a.detach().float().cpu()
        diff = (a - e).abs().max().item()
        rel = ((a - e).norm() / e.norm()).item()
        assert diff <= tol[0] and rel <= tol[1], (n, diff, rel)


def test_gate_zero_and_two():
    from vsa_mi355x import mi355x as M
    g = torch.Generator(device=DEV).manual_seed(3)
    be, D, nb, topk = 256, 128, 4, 2
    q, k, v = (torch.randn(1, 2, nb * be, D, generator=g, device=DEV, dtype=torch.bfloat16)
               for _ in range(3))
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = 200
    scale = 1.0 / math.sqrt(D)
    _, sel = M.mi355x_route(q, k, v, vbs, vbs, topk, (4, 8, 8))
    qc, kc, vc = M.block_mean_qkv(q, k, v, vbs, vbs, be)
    _, _, outc, _ = M.coarse_forward(qc, kc, vc, topk, scale)
    fine = M.mi355x_sparse_attention(q, k, v, sel, vbs, block_size=(4, 8, 8))
    zero = M.mi355x_vsa(q, k, v, vbs, vbs, topk, (4, 8, 8), torch.zeros_like(q))
    assert torch.equal(zero, fine)                     # 0 * out_c + out_s, exactly
    two = M.mi355x_vsa(q, k, v, vbs, vbs, topk, (4, 8, 8), torch.full_like(q, 2.0))
    expect = (2.0 * outc.float().repeat_interleave(be, dim=2) + fine.float()).to(torch.bfloat16)
    diff = (two.float() - expect.float()).abs().max().item()
    assert diff <= 2e-2, diff                          # one bf16 rounding apart at most


def test_unrouted_key_blocks_still_get_gradient():
    from vsa_mi355x import mi355x as M
    g = torch.Generator(device=DEV).manual_seed(5)
    be, D, nb, topk = 64, 64, 8, 1
    q, k, v = (torch.randn(1, 1, nb * be, D, generator=g, device=DEV, dtype=torch.bfloat16)
               for _ in range(3))
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    _, sel = M.mi355x_route(q, k, v, vbs, vbs, topk, (1, 1, be))
    unrouted = sorted(set(range(nb)) - set(sel.flatten().tolist()))
    assert unrouted, "route selects every block; pick another seed"
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    out = M.mi355x_vsa(*leaves, vbs, vbs, topk, (1, 1, be))
    dq, dk, dv = torch.autograd.grad(out, leaves, torch.ones_like(out))
    for blk in unrouted:                               # pooled-key gradient reaches every token
        rows = slice(blk * be, (blk + 1) * be)
        assert (dk[0, 0, rows].abs().sum(-1) > 0).all()
        assert (dv[0, 0, rows].abs().sum(-1) > 0).all()
