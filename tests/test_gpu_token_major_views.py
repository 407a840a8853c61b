"""GPU: ``mi355x_vsa`` on per-head views of token-major [B, S, H, D] tensors.

A DiT produces q, k, v (and the gate, common.py:326-328) as
``x.view(B, S, H, D).transpose(1, 2)``.  The op reads such views in place
through the raster kernels with the identity slot table and returns the same
kind of view; the output and every gradient must equal the op on contiguous
copies bit for bit, with separate q and kv block sizes."""

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


CASES = [
    # batch, heads, blocks, head_dim, block, dtype, gate, topk
    (2, 3, 4, 64, 64, torch.bfloat16, "full_tm", 2),     # block 64, token-major gate
    (1, 22, 6, 128, 256, torch.float16, "token", 3),     # ping-pong kernels, per-token gate
    (1, 2, 5, 128, 128, torch.bfloat16, None, 2),        # block 128, no gate
    (1, 2, 6, 64, 256, torch.bfloat16, "full_hm", 4),    # 4-wave kernels, head-major gate
]


def _counts(n, be, g):
    c = torch.randint(1, be + 1, (n,), generator=g, dtype=torch.int32)
    c[0] = be
    return c


def _leaves(b, h, s, d, dtype, g):
    """Token-major leaves [B, S, H, D] and their [B, H, S, D] views."""
    base = [torch.randn(b, s, h, d, generator=g).to(dtype).to(DEV).requires_grad_()
            for _ in range(3)]
    return base, [x.transpose(1, 2) for x in base]


def _gate(kind, b, h, s, d, dtype, g):
    if kind is None:
        return None, None
    if kind == "full_tm":
        base = (2.0 * torch.rand(b, s, h, d, generator=g)).to(dtype).to(DEV).requires_grad_()
        return base, base.transpose(1, 2)
    if kind == "token":
        base = (2.0 * torch.rand(b, s, h, 1, generator=g)).to(dtype).to(DEV).requires_grad_()
        return base, base.transpose(1, 2)
    base = (2.0 * torch.rand(b, h, s, d, generator=g)).to(dtype).to(DEV).requires_grad_()
    return base, base


def _as_leaf(x):
    return x.detach().clone().requires_grad_()


@pytest.mark.parametrize("b,h,nb,d,be,dtype,gate,topk", CASES)
def test_token_major_views_equal_contiguous_op_bit_for_bit(b, h, nb, d, be, dtype, gate, topk):
    from vsa_mi355x import mi355x as M
    s = nb * be
    print(f"case b={b} h={h} nb={nb} d={d} be={be} {dtype} gate={gate} topk={topk}", flush=True)
    g = torch.Generator().manual_seed(nb * 131 + h + d)
    vbs, qvbs = _counts(nb, be, g), _counts(nb, be, g)
    base, views = _leaves(b, h, s, d, dtype, g)
    gbase, gview = _gate(gate, b, h, s, d, dtype, g)
    dout = torch.randn(b, h, s, d, generator=g).to(dtype).to(DEV)
    assert M._raster_views(*views, gview, be)

    out = M.mi355x_vsa(*views, vbs, qvbs, topk, (1, 1, be), gview)
    assert out.shape == (b, h, s, d) and out.dtype == dtype
    assert out.transpose(1, 2).is_contiguous() and not out.is_contiguous()
    out.backward(dout)

    ref_leaves = [_as_leaf(x.transpose(1, 2).contiguous()) for x in base]
    ref_gate = None if gbase is None else _as_leaf(gview.contiguous())
    ref = M.mi355x_vsa(*ref_leaves, vbs, qvbs, topk, (1, 1, be), ref_gate)
    assert ref.is_contiguous()
    ref.backward(dout)

    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, ref), (out.float() - ref.float()).abs().max().item()
    for name, x, r in zip("qkv", base, ref_leaves):
        assert torch.equal(x.grad.transpose(1, 2), r.grad), name
    if gbase is not None:
        got = gbase.grad.transpose(1, 2) if gate in ("full_tm", "token") else gbase.grad
        assert torch.equal(got, ref_gate.grad), "gate"


def test_token_major_views_no_grad_and_shared_q_k():
    """Inference (no autograd) on views, and one tensor passed as both q and k
    with different q and kv block sizes (each mean uses its own counts)."""
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be = 1, 4, 6, 128, 64
    s = nb * be
    g = torch.Generator().manual_seed(17)
    vbs, qvbs = _counts(nb, be, g), _counts(nb, be, g)
    qk = torch.randn(b, s, h, d, generator=g).to(torch.bfloat16).to(DEV).transpose(1, 2)
    v = torch.randn(b, s, h, d, generator=g).to(torch.bfloat16).to(DEV).transpose(1, 2)
    with torch.no_grad():
        out = M.mi355x_vsa(qk, qk, v, vbs, qvbs, 3, (1, 1, be))
        c = qk.contiguous()
        ref = M.mi355x_vsa(c, c, v.contiguous(), vbs, qvbs, 3, (1, 1, be))
    assert torch.equal(out, ref)


def test_views_without_a_raster_kernel_take_the_contiguous_path():
    """fp32, an fp32 gate beside bf16 inputs, and q / kv of different lengths
    are copied to contiguous first; the result is the contiguous op's."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(5)
    b, h, d, be = 1, 2, 64, 64
    blk = (1, 1, be)

    def view(s, dtype):
        return torch.randn(b, s, h, d, generator=g).to(dtype).to(DEV).transpose(1, 2)

    q, k, v = view(3 * be, torch.float32), view(3 * be, torch.float32), view(3 * be,
                                                                              torch.float32)
    vbs = torch.tensor([64, 30, 64], dtype=torch.int32)
    assert not M._raster_views(q, k, v, None, be)
    assert torch.equal(M.mi355x_vsa(q, k, v, vbs, vbs, 2, blk),
                       M.mi355x_vsa(q.contiguous(), k.contiguous(), v.contiguous(), vbs, vbs,
                                    2, blk))

    q, k, v = (view(3 * be, torch.bfloat16) for _ in range(3))
    gate = torch.rand(b, h, 3 * be, d, generator=g).to(DEV)
    gate32 = M._prepare_gate(gate, q)
    assert not M._raster_views(q, k, v, gate32, be)
    assert torch.equal(M.mi355x_vsa(q, k, v, vbs, vbs, 2, blk, gate),
                       M.mi355x_vsa(q.contiguous(), k.contiguous(), v.contiguous(), vbs, vbs,
                                    2, blk, gate))

    q = view(2 * be, torch.bfloat16)
    assert not M._raster_views(q, k, v, None, be)
    qvbs = torch.tensor([64, 40], dtype=torch.int32)
    assert torch.equal(M.mi355x_vsa(q, k, v, vbs, qvbs, 2, blk),
                       M.mi355x_vsa(q.contiguous(), k.contiguous(), v.contiguous(), vbs, qvbs,
                                    2, blk))


def test_inputs_off_16_byte_alignment_give_the_same_result():
    """q, k, v, gate and dout whose data starts 2 bytes past a 16-byte boundary
    (contiguous views with an odd storage offset): the host copies them before
    the kernels, whose rows are read and written 16 bytes at a time."""
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be = 1, 3, 4, 128, 64
    s = nb * be
    g = torch.Generator().manual_seed(23)
    vbs = _counts(nb, be, g)

    def odd(x):
        buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=DEV)
        y = buf[1:].view(x.shape)
        y.copy_(x)
        assert y.data_ptr() % 16 != 0
        return y

    src = [torch.randn(b, h, s, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]
    gate = (2.0 * torch.rand(b, h, s, d, generator=g)).to(torch.bfloat16).to(DEV)
    res = []
    for make in (lambda x: x.clone(), odd):
        leaves = [make(x).requires_grad_() for x in src[:3]]
        gl = make(gate).requires_grad_()
        out = M.mi355x_vsa(*leaves, vbs, vbs, 2, (1, 1, be), gl)
        out.backward(make(src[3]))
        res.append([out.detach()] + [x.grad for x in leaves] + [gl.grad])
    for name, a, b_ in zip(["out", "dq", "dk", "dv", "dgate"], *res):
        assert torch.equal(a, b_), name


@pytest.mark.parametrize("shape", [(0, 3, 256, 64), (2, 0, 256, 64)])
def test_empty_batch_gives_an_empty_differentiable_output(shape):
    """batch or heads 0: an empty output of q's shape and empty gradients, as
    torch_vsa returns, for the full op, the explicit-route op and the tiled op."""
    from vsa_mi355x import mi355x as M, tiled
    b, h, s, d = shape
    vbs = torch.full((s // 64,), 64, dtype=torch.int32, device=DEV)
    leaves = [torch.randn(*shape, device=DEV, dtype=torch.bfloat16).requires_grad_()
              for _ in range(3)]
    gate = torch.rand(*shape, device=DEV, dtype=torch.bfloat16).requires_grad_()
    sel = torch.zeros(b, h, s // 64, 2, dtype=torch.int32, device=DEV)
    for out, wrt in ((M.mi355x_vsa(*leaves, vbs, vbs, 2, (1, 1, 64), gate), leaves + [gate]),
                     (M.mi355x_sparse_attention(*leaves, sel, vbs, block_size=(1, 1, 64)),
                      leaves),
                     (tiled.mi355x_vsa_tiled(*leaves, (1, 4, 64), 2, (1, 1, 64), gate),
                      leaves + [gate])):
        assert out.shape == shape and out.dtype == torch.bfloat16
        grads = torch.autograd.grad(out, wrt, torch.ones_like(out))
        assert all(g_.shape == x.shape for g_, x in zip(grads, wrt))
