"""Routes longer than 64 slots on the GPU kernels.

The forward and dQ kernels hold a query block's route in registers 64 slots at
a time and reload it past slot 63.  A route whose first 64 slots point at empty
key blocks (valid size 0) and whose last slots hold real blocks visits exactly
the chunks of the short route made of those real blocks, in the same order, so
outputs and gradients must be bit-identical to the short route's; the short
route is checked against the oracle.  Block 256 at >= 256 query blocks runs the
8-wave forward, block 64 the 2-wave one."""

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
    from vsa import _lib
    _lib.load()
    yield


def _run(q, k, v, sel, vbs, be, do):
    from vsa import mi355x as M
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel, vbs, block_size=(1, 1, be))
    grads = torch.autograd.grad(out, leaves, do)
    return out.detach(), grads


@pytest.mark.parametrize("be,H,D,nb,n_real", [(256, 16, 128, 70, 2), (256, 4, 64, 80, 3),
                                              (64, 2, 64, 140, 2), (64, 3, 128, 70, 5)])
def test_long_route_equals_short_route(be, H, D, nb, n_real):
    g = torch.Generator().manual_seed(nb + D)
    S = nb * be
    n_empty = 64 if nb - n_real >= 64 else nb - n_real
    assert n_empty + n_real <= nb
    q, k, v, do = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16) for _ in range(4))
    vbs = torch.full((nb,), be, dtype=torch.int32)
    empty = torch.arange(n_real, n_real + n_empty)            # blocks with no valid token
    vbs[empty] = 0
    real = torch.stack([torch.randperm(n_real, generator=g) for _ in range(H * nb)])
    real = real.view(1, H, nb, n_real).to(torch.int32)        # each query block: all real blocks
    long_sel = torch.cat([empty.to(torch.int32).expand(1, H, nb, n_empty), real], dim=-1)
    assert long_sel.shape[-1] > 64 or be == 64
    q, k, v, do, vbs = (t.to(DEV) for t in (q, k, v, do, vbs))
    out_l, gr_l = _run(q, k, v, long_sel.to(DEV), vbs, be, do)
    out_s, gr_s = _run(q, k, v, real.to(DEV), vbs, be, do)
    assert torch.equal(out_l, out_s)
    for a, b_ in zip(gr_l, gr_s):
        assert torch.equal(a, b_)
    # and the short route against the oracle, on the first head
    ref = O.sparse_attention(q[:, :1].cpu(), k[:, :1].cpu(), v[:, :1].cpu(), real[:, :1],
                             vbs.cpu(), block_size=(1, 1, be))
    a, e = out_s[:, :1].float().cpu(), ref.float()
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm()).item()
    assert diff <= 2e-2 and rel <= 1e-2, (diff, rel)
