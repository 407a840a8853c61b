"""GPU: the no-allocation dK/dV entry point equals the workspace one.

``vsa_sparse_bwd_dkdv_noalloc`` keeps the dK/dV tile order and scheduling
counters in the library's static device scratch instead of a caller buffer.
Its results must be bit for bit those of ``vsa_sparse_bwd_dkdv`` given a
``vsa_dkdv_tile_order`` workspace (the tile order only changes the dispatch
order, never a value).  Two calls in a row, the second on a smaller input, so
the second runs on a scratch that still holds the first call's order.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _problem(seed, be, d, h, nb, tk, dtype):
    """Inputs of one dK/dV call: a route with one hot key block, a ragged block
    and pooled gradients to fold in."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(seed)
    shape = (1, h, nb * be, d)
    q, k, v, do = (torch.randn(shape, generator=g).to(dtype).to(DEV) for _ in range(4))
    rows = []
    for r in range(h * nb):   # every other query block also chooses the hot key block 0
        if r % 2:
            rows.append(torch.randperm(nb, generator=g)[:tk])
        else:
            rows.append(torch.cat([torch.zeros(1, dtype=torch.long),
                                   1 + torch.randperm(nb - 1, generator=g)[:tk - 1]]))
    sel = torch.stack(rows).sort(-1).values.view(1, h, nb, tk).to(torch.int32).to(DEV)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[nb // 3] = be - 5
    vbs = vbs.to(DEV)
    dkc = torch.randn((1, h, nb, d), generator=g).to(dtype).to(DEV)
    dvc = torch.randn((1, h, nb, d), generator=g).to(dtype).to(DEV)
    scale = d ** -0.5
    with torch.no_grad():
        out, lse, _ = M.sparse_forward(q, k, v, sel, vbs, be, scale)
        delta, _, _ = M.backward_prep(out, do, be)
        inverse, offsets, counts = M.invert_routes(sel, nb)
    return dict(q=q, k=k, v=v, do=do, lse=lse, delta=delta, counts=counts, offsets=offsets,
                inverse=inverse, vbs=vbs, dkc=dkc, dvc=dvc, bh=h, s=nb * be, d=d, be=be, tk=tk,
                scale=scale)


def _args(p, dk, dv):
    from vsa_mi355x import _lib
    P = _lib.ptr
    return [P(p["q"]), P(p["k"]), P(p["v"]), P(p["do"]), P(p["lse"]), P(p["delta"]),
            P(p["counts"]), P(p["offsets"]), P(p["inverse"]), P(p["vbs"]), P(dk), P(dv),
            P(p["dkc"]), P(p["dvc"]), p["bh"], p["s"], p["s"], p["d"], p["be"], p["tk"],
            p["scale"]]


def _with_workspace(p):
    from vsa_mi355x import _lib
    from vsa_mi355x import mi355x as M
    dk, dv = torch.empty_like(p["k"]), torch.empty_like(p["v"])
    order = M.dkdv_tile_order(p["counts"], p["bh"], p["s"], p["d"], p["be"])
    _lib.call("vsa_sparse_bwd_dkdv", *_args(p, dk, dv), _lib.ptr(order),
              _lib.dtype_code(p["q"].dtype), _lib.stream_of(p["q"]))
    return dk, dv


def _no_alloc(p):
    from vsa_mi355x import _lib
    dk = torch.full_like(p["k"], float("nan"))
    dv = torch.full_like(p["v"], float("nan"))
    _lib.call("vsa_sparse_bwd_dkdv_noalloc", *_args(p, dk, dv), _lib.dtype_code(p["q"].dtype),
              _lib.stream_of(p["q"]))
    return dk, dv


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_no_alloc_dkdv_equals_workspace_entry_point_two_calls(dtype):
    big = _problem(71, be=256, d=128, h=8, nb=40, tk=8, dtype=dtype)
    small = _problem(72, be=64, d=64, h=2, nb=24, tk=5, dtype=dtype)
    for p in (big, small):          # the second call is smaller than the first
        print(f"no-alloc dK/dV: be {p['be']} d {p['d']} heads {p['bh']} seq {p['s']}", flush=True)
        dk, dv = _no_alloc(p)
        ek, ev = _with_workspace(p)
        torch.cuda.synchronize()
        assert torch.equal(dk, ek) and torch.equal(dv, ev)


def test_no_alloc_dkdv_fp32_runs_the_fp32_kernel():
    p = _problem(73, be=64, d=64, h=2, nb=8, tk=3, dtype=torch.float32)
    dk, dv = _no_alloc(p)
    ek, ev = _with_workspace(p)
    torch.cuda.synchronize()
    assert torch.equal(dk, ek) and torch.equal(dv, ev)


def test_no_alloc_dkdv_head_dim_256_two_calls():
    """Head dim 256 splits each key tile over two workgroups and takes its tiles
    from the order by workgroup index (no counters): the same bit-for-bit bar,
    the second call smaller than the first."""
    big = _problem(74, be=128, d=256, h=4, nb=24, tk=6, dtype=torch.bfloat16)
    small = _problem(75, be=256, d=256, h=2, nb=6, tk=3, dtype=torch.bfloat16)
    for p in (big, small):
        print(f"no-alloc dK/dV: be {p['be']} d {p['d']} heads {p['bh']} seq {p['s']}", flush=True)
        dk, dv = _no_alloc(p)
        ek, ev = _with_workspace(p)
        torch.cuda.synchronize()
        assert torch.equal(dk, ek) and torch.equal(dv, ev)
