"""GPU: the torch.library custom-op form of the op (``vsa_mi355x.ops``).

Its output and gradients equal the eager autograd Function's bit for bit; a
model around it compiles with ``torch.compile(fullgraph=True)`` (the op stays
in the graph, no break) and gives the eager model's values; and
``torch.library.opcheck`` accepts the schemas, fake implementations and
autograd registration."""

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


def _inputs(b, h, nb, d, be, gate, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    s = nb * be
    q, k, v, do = (torch.randn(b, h, s, d, generator=g, device=DEV, dtype=dtype)
                   for _ in range(4))
    gt = None
    if gate == "full":
        gt = torch.rand(b, h, s, d, generator=g, device=DEV, dtype=dtype)
    elif gate == "token":
        gt = torch.rand(b, h, s, 1, generator=g, device=DEV, dtype=dtype)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = be - 37
    return q, k, v, do, gt, vbs


def _run(fn, q, k, v, do, gt):
    leaves = [x.detach().clone().requires_grad_() for x in (q, k, v)]
    gl = gt.detach().clone().requires_grad_() if gt is not None else None
    out = fn(*leaves, gl)
    wrt = leaves + ([gl] if gl is not None else [])
    return [out.detach()] + list(torch.autograd.grad(out, wrt, do))


@pytest.mark.parametrize("b,h,nb,d,be,gate,topk", [(1, 4, 6, 128, 256, "full", 3),
                                                   (2, 3, 8, 64, 64, "token", 4),
                                                   (1, 2, 5, 128, 128, None, 2)])
def test_custom_op_equals_eager_bit_for_bit(b, h, nb, d, be, gate, topk):
    from vsa_mi355x import mi355x as M, ops
    q, k, v, do, gt, vbs = _inputs(b, h, nb, d, be, gate, seed=nb + d)
    blk = (1, 1, be)
    ref = _run(lambda q_, k_, v_, g_: M.mi355x_vsa(q_, k_, v_, vbs, vbs, topk, blk, g_),
               q, k, v, do, gt)
    got = _run(lambda q_, k_, v_, g_: ops.mi355x_vsa(q_, k_, v_, vbs, vbs, topk, blk, g_),
               q, k, v, do, gt)
    for name, a, e in zip(["out", "dq", "dk", "dv", "dgate"], got, ref):
        assert torch.equal(a, e), name
    with torch.no_grad():
        assert torch.equal(ops.mi355x_vsa(q, k, v, vbs, vbs, topk, blk, gt), ref[0])


def test_explicit_route_custom_op_equals_eager():
    from vsa_mi355x import mi355x as M, ops
    q, k, v, do, _, vbs = _inputs(1, 3, 10, 64, 64, None, seed=4)
    g = torch.Generator(device=DEV).manual_seed(5)
    sel = torch.stack([torch.randperm(10, generator=g, device=DEV)[:4]
                       for _ in range(30)]).view(1, 3, 10, 4).to(torch.int32)
    blk = (1, 1, 64)
    ref = _run(lambda q_, k_, v_, _g: M.mi355x_sparse_attention(q_, k_, v_, sel, vbs,
                                                                 block_size=blk), q, k, v, do, None)
    got = _run(lambda q_, k_, v_, _g: ops.mi355x_sparse_attention(q_, k_, v_, sel, vbs,
                                                                   block_size=blk), q, k, v, do, None)
    for name, a, e in zip(["out", "dq", "dk", "dv"], got, ref):
        assert torch.equal(a, e), name


def test_compiled_model_keeps_the_op_in_its_graph():
    """A block with projections around the op compiles as one graph
    (fullgraph=True raises on any break) and matches the eager block (the
    projections in fp32; AOT autograd may reorder the loss reduction, so the
    block is compared at fp32 rounding; the op itself is checked bit for bit
    above)."""
    from vsa_mi355x import ops
    torch._dynamo.reset()
    b, h, nb, d, be, topk = 1, 4, 6, 128, 256, 3
    s, dim = nb * be, h * d
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(b, s, dim, generator=g, device=DEV)
    w = [torch.randn(dim, dim, generator=g, device=DEV) * dim ** -0.5 for _ in range(4)]
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)

    def block(x, wq, wk, wv, wg):
        q, k, v, gate = ((x @ w_).to(torch.bfloat16).view(b, s, h, d).transpose(1, 2)
                         for w_ in (wq, wk, wv, wg))
        out = ops.mi355x_vsa(q, k, v, vbs, vbs, topk, (1, 1, be), gate)
        return out.transpose(1, 2).reshape(b, s, dim).float().square().mean()

    def grads(fn):
        leaves = [t.detach().clone().requires_grad_() for t in [x] + w]
        loss = fn(*leaves)
        return [loss.detach()] + list(torch.autograd.grad(loss, leaves))

    compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    for name, a, e in zip(["loss", "dx", "dwq", "dwk", "dwv", "dwg"], grads(compiled),
                          grads(block)):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-6, msg=name)


def test_opcheck_accepts_the_registrations():
    from vsa_mi355x import ops  # noqa: F401
    q, k, v, do, gt, vbs = _inputs(1, 2, 4, 64, 64, "full", seed=2)
    args = [x.clone().requires_grad_() for x in (q, k, v, gt)]
    torch.library.opcheck(torch.ops.vsa_mi355x.vsa_fwd.default,
                          (*args[:3], args[3], vbs, vbs, 2, 64, 0.125, True),
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))
    sel = torch.tensor([[[[0, 1], [1, 2], [2, 3], [3, 0]]] * 2], dtype=torch.int32, device=DEV)
    torch.library.opcheck(torch.ops.vsa_mi355x.sparse_fwd.default,
                          (*args[:3], sel, vbs, 64, 0.125, True),
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))
