"""GPU gradients against torch_vsa's fine branch as written.

The oracle gathers key / value blocks from fp32 copies, so a key block's
per-query-block gradients are summed in fp32; torch_impl.py:43-46, 86-87
gathers in T with ``torch.gather`` over the block view broadcast across query
blocks and promotes afterwards, so each contribution is rounded to T before
the sum.  On skewed routes a key block collects hundreds of such terms.  Here
the HIP dq / dk / dv must be within relative L2 1e-2 of both restatements (and
within the north star's max-abs 2e-2 of the fp32 one) on Zipf(1.2) routes."""

import numpy as np
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


def _zipf_routes(h, qb, kb, tk, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, kb + 1) ** 1.2
    p /= p.sum()
    perm = rng.permutation(kb)
    sel = np.stack([np.stack([perm[rng.choice(kb, tk, replace=False, p=p)] for _ in range(qb)])
                    for _ in range(h)])
    return torch.from_numpy(sel[None].astype(np.int32))


def _rel(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return ((a - e).norm() / e.norm()).item()


@pytest.mark.parametrize("S,D,be,tk,vbs_last,heads", [
    (16384, 64, 64, 32, 64, [1]),         # c5's block, head dim and topk, 256 blocks
    (40960, 128, 256, 20, 256, [7]),      # c3's shape with a skewed route
    (8192, 128, 256, 8, 131, [0]),        # a padded last key block
])
def test_hot_key_gradients_match_both_gathers(S, D, be, tk, vbs_last, heads):
    from vsa_mi355x import mi355x as M
    H, nb = max(heads) + 1, S // be
    sel = _zipf_routes(H, nb, nb, tk, 5)
    counts = np.bincount(sel[0, heads[0]].flatten().numpy(), minlength=nb)
    print(f"  hottest key block: {counts.max()} in-edges of {nb} query blocks", flush=True)
    assert counts.max() >= nb // 2
    g = torch.Generator().manual_seed(21)
    q, k, v, do = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16) for _ in range(4))
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[-1] = vbs_last
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v)]
    out = M.mi355x_sparse_attention(*leaves, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be))
    grads = torch.autograd.grad(out, leaves, do.to(DEV))
    torch.cuda.synchronize()

    sl = lambda t: t[:, heads].clone().requires_grad_()
    for gather in ("fp32", "as_written"):
        qr, kr, vr = sl(q), sl(k), sl(v)
        ref = O.sparse_attention(qr, kr, vr, sel[:, heads], vbs, block_size=(1, 1, be),
                                 gather=gather)
        ref_grads = torch.autograd.grad(ref, (qr, kr, vr), do[:, heads])
        for n, a, e in zip(("dq", "dk", "dv"), grads, ref_grads):
            a = a[:, heads]
            rel = _rel(a, e)
            diff = (a.detach().float().cpu() - e.float()).abs().max().item()
            print(f"  {gather} {n}: rel-L2 {rel:.2e} max-abs {diff:.2e}", flush=True)
            assert rel <= 1e-2, (gather, n, rel)
            if gather == "fp32":
                assert diff <= 2e-2, (n, diff)
