"""Routes longer than 64 slots on the GPU kernels.

The forward and dQ kernels hold a query block's route in registers 64 slots at
a time and reload it past slot 63.  A route whose first 64 slots point at empty
key blocks (valid size 0) and whose last slots hold real blocks visits exactly
the chunks of the short route made of those real blocks, in the same order, so
outputs and gradients must be bit-identical to the short route's; the short
route is checked against the oracle.  Block 256 at >= 256 query blocks runs the
8-wave forward, block 64 the 2-wave one."""

import math
import numpy

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


def _run(q, k, v, sel, vbs, be, do):
    from vsa_mi355x import mi355x as M
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


def _order_case(H, nb, be, D, hot):
    """Inputs for the dK/dV dispatch-order checks: `hot` key blocks chosen by
    every query block (a skewed route), the other slots spread uniformly."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(nb * 7 + hot)
    S, tk = nb * be, 4
    q, k, v, do = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16).to(DEV)
                   for _ in range(4))
    rest = torch.stack([hot + torch.randperm(nb - hot, generator=g)[:tk - hot]
                        for _ in range(H * nb)]).view(1, H, nb, tk - hot)
    sel = torch.cat([torch.arange(hot).expand(1, H, nb, hot), rest], -1).to(torch.int32).to(DEV)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out, lse, _ = M.sparse_forward(q, k, v, sel, vbs, be, scale)
    delta, _, _ = M.backward_prep(out, do, be)
    inv, off, cnt = M.invert_routes(sel, nb)
    return M, q, k, v, do, lse, delta, sel, vbs, inv, off, cnt, scale, tk


@pytest.mark.parametrize("H,nb,be,D,hot", [(4, 160, 64, 64, 2), (2, 60, 256, 128, 1),
                                           (3, 40, 128, 256, 2), (16, 160, 256, 128, 0),
                                           (3, 48, 256, 64, 1), (2, 64, 128, 64, 0)])
def test_dkdv_tile_order_is_a_permutation_and_keeps_results(H, nb, be, D, hot):
    from vsa_mi355x import _lib
    M, q, k, v, do, lse, delta, sel, vbs, inv, off, cnt, scale, tk = _order_case(H, nb, be, D, hot)
    S = nb * be
    order = M.dkdv_tile_order(cnt, H, S, D, be)
    kw = 64 if D == 64 else 32                                # keys per wave
    kt = min(be, 4 * kw)                                      # keys per workgroup
    nsplit = 2 if D > 128 else 1
    tiles = H * (S // kt) * nsplit
    per = (tiles + 7) // 8
    assert order.numel() == 8 * per + 16
    assert (order[8 * per:8 * per + 9] == 0).all()           # scheduling counters, reset
    raw = order[:8 * per].cpu().numpy()
    tag = 1 << 30                                             # entries of a longest-first range
    o = raw & (tag - 1)
    real = o[o < tiles]
    assert sorted(real.tolist()) == list(range(tiles))        # every tile exactly once
    assert (o[o >= tiles] == tiles).all()                     # the rest are the sentinel
    nedge = cnt.cpu().reshape(H, nb).repeat_interleave(be // kt, 1).reshape(-1)
    nedge = nedge.repeat_interleave(nsplit)
    slots = 32 * (4 // (kt // kw))                            # concurrent workgroups per XCD
    sorted_ranges = 0
    for x in range(8):                                        # each XCD keeps its own range
        ids = o[x::8]
        tagged = (raw[x::8] & tag) != 0
        assert tagged.all() or not tagged.any()               # one kind per range
        ids = ids[ids < tiles]
        assert ((ids >= x * per) & (ids < (x + 1) * per)).all()
        rng = nedge[x * per:min((x + 1) * per, tiles)]
        if len(rng) and int(rng.max()) * slots * 4 > int(rng.sum()):   # skewed: longest first
            e = nedge[torch.from_numpy(ids.astype('int64'))]
            assert (e[:-1] >= e[1:]).all()
            assert tagged.all()
            sorted_ranges += 1
        else:   # balanced: index order, with the smallest tiles (<= 4 per slot) moved last
            r = rng.clamp(max=1023).numpy()
            cut = max([c for c in set(r.tolist()) if (r <= c).sum() <= 4 * slots], default=-1)
            idx = numpy.arange(x * per, x * per + len(r))
            want = numpy.concatenate([idx[r > cut], idx[r <= cut]])
            assert (ids == want).all()
            assert not tagged.any()
    assert sorted_ranges > 0 if hot else True
    # the dispatch order does not reach the results
    P = lambda t: _lib.ptr(t)
    res = []
    for tord in (None, order):
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        _lib.call("vsa_sparse_bwd_dkdv", P(q), P(k), P(v), P(do), P(lse), P(delta), P(cnt),
                  P(off), P(inv), P(vbs), P(dk), P(dv), None, None, H, S, S, D, be, tk,
                  float(scale), P(tord), _lib.dtype_code(q.dtype), _lib.stream_of(q))
        res.append((dk, dv))
    torch.cuda.synchronize()
    for a, b_ in zip(*res):
        assert torch.equal(a, b_)
    assert (order[8 * per:8 * per + 9] == 0).all()           # left reset for the next launch
