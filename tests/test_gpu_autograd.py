"""GPU: the autograd contract of the public functions.

The row moves (tile, untile and the zero-padding of odd block volumes / head
dims) are linear, and each one's backward is its adjoint move, itself
differentiable: gradcheck and gradgradcheck (fast mode: random projections
of the Jacobian) hold in float64.  The attention
functions compute their gradients in hand-written kernels and define no
second derivative (nor does the reference's Triton backward, whose gradients
carry no graph); they are marked differentiable once, so a second derivative
through them raises instead of silently leaving their term out."""

import math

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


@pytest.mark.parametrize("shape,ts", [((3, 5, 5), (2, 4, 4)), ((2, 6, 6), (2, 3, 3))])
def test_tile_untile_gradgradcheck(shape, ts):
    from vsa_mi355x import tiling
    meta = tiling.build_vsa_metadata(shape, ts, device=DEV)
    S = math.prod(shape)
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    tpi, npi = meta["tile_partition_indices"], meta["non_pad_index"]
    rev = meta["reverse_tile_partition_indices"]
    x = torch.randn(2, S, 3, device=DEV, dtype=torch.float64, requires_grad=True)
    y = torch.randn(2, nb * be, 3, device=DEV, dtype=torch.float64, requires_grad=True)
    t = lambda a: tiling.tile(a, tpi, npi, nb, be)
    u = lambda a: tiling.untile(a, npi, rev)
    for f, a in ((t, x), (u, y), (lambda a: u(t(a)), x)):
        assert torch.autograd.gradcheck(f, (a,), fast_mode=True)
        assert torch.autograd.gradgradcheck(f, (a,), fast_mode=True)


def test_tile_second_derivative_is_the_move_itself():
    """d/dg <tile^T g, w> = tile(w): the second derivative through tile's
    backward is tile again, bit-exact."""
    from vsa_mi355x import tiling
    meta = tiling.build_vsa_metadata((5, 7, 9), (4, 4, 4), device=DEV)
    S = math.prod((5, 7, 9))
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    tpi, npi = meta["tile_partition_indices"], meta["non_pad_index"]
    x = torch.randn(2, S, 8, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    g = torch.randn(2, nb * be, 8, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = torch.randn(2, S, 8, device=DEV, dtype=torch.bfloat16)
    (dx,) = torch.autograd.grad(tiling.tile(x, tpi, npi, nb, be), x, g, create_graph=True)
    (dg,) = torch.autograd.grad(dx, g, w)
    assert torch.equal(dg, tiling.tile(w, tpi, npi, nb, be))


@pytest.mark.parametrize("s,be,d", [(2 * 27, 27, 40), (2 * 100, 100, 72)])
def test_pad_unpad_gradgradcheck(s, be, d):
    from vsa_mi355x import mi355x as M
    kbe, kd = M._kernel_block(be), M._kernel_dim(d)
    rows = M._block_rows(s, be, kbe, torch.device(DEV))
    out_rows = (s // be) * kbe
    x = torch.randn(1, 2, s, d, device=DEV, dtype=torch.float64, requires_grad=True)
    y = torch.randn(1, 2, out_rows, kd, device=DEV, dtype=torch.float64, requires_grad=True)
    pad = lambda a: M._Pad.apply(a, rows, out_rows, kd)
    unpad = lambda a: M._Unpad.apply(a, rows, (1, 2, s, d))
    for f, a in ((pad, x), (unpad, y)):
        assert torch.autograd.gradcheck(f, (a,), fast_mode=True)
        assert torch.autograd.gradgradcheck(f, (a,), fast_mode=True)


def _qkv(shape, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(5)
    return [torch.randn(shape, generator=g).to(dtype).to(DEV).requires_grad_()
            for _ in range(3)]


def _second_derivative_raises(out, leaves):
    do = torch.randn_like(out).requires_grad_()
    grads = torch.autograd.grad(out, leaves, do, create_graph=True)
    assert all(torch.isfinite(g).all() for g in grads)
    # the gradients hang off once_differentiable's error node, not off the
    # leaves: a backward through them reaches that node and raises
    with pytest.raises(RuntimeError, match="differentiate twice"):
        sum(g.float().sum() for g in grads).backward()


@pytest.mark.parametrize("be,d", [(64, 64), (27, 40)])
def test_vsa_second_derivative_raises(be, d):
    from vsa_mi355x import mi355x as M
    nb = 4
    q, k, v = _qkv((1, 2, nb * be, d))
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    out = M.mi355x_vsa(q, k, v, vbs, vbs, 2, (1, 1, be))
    _second_derivative_raises(out, (q, k, v))


def test_sparse_attention_second_derivative_raises():
    from vsa_mi355x import mi355x as M
    nb, be = 4, 64
    q, k, v = _qkv((1, 2, nb * be, 64))
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    sel = torch.tensor([[0, 1], [1, 2], [2, 3], [3, 0]], dtype=torch.int32,
                       device=DEV).expand(1, 2, nb, 2).contiguous()
    out = M.mi355x_sparse_attention(q, k, v, sel, vbs, block_size=(1, 1, be))
    _second_derivative_raises(out, (q, k, v))


def test_tiled_second_derivative_raises():
    from vsa_mi355x import tiled
    q, k, v = _qkv((1, 2, 4 * 5 * 6, 64))
    out = tiled.mi355x_vsa_tiled(q, k, v, (4, 5, 6), 2, (4, 4, 4))
    _second_derivative_raises(out, (q, k, v))


def test_custom_op_second_derivative_raises():
    from vsa_mi355x import ops
    nb, be = 4, 64
    q, k, v = _qkv((1, 2, nb * be, 64))
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    out = ops.mi355x_vsa(q, k, v, vbs, vbs, 2, (1, 1, be))
    do = torch.randn_like(out).requires_grad_()
    grads = torch.autograd.grad(out, (q, k, v), do, create_graph=True)
    with pytest.raises(RuntimeError, match="no autograd formula"):
        torch.autograd.grad(sum(g.float().sum() for g in grads), (q, k, v))
