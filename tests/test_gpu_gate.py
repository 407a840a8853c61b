"""GPU parity of the gate-producer row: the token-major gate path of
mi355x_vsa (gate read and its gradient written in the Linear's own layout)."""

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


def _grads(q, k, v, gate, vbs, topk, block, do):
    from vsa_mi355x import mi355x as M
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    g = gate.detach().clone() if gate.is_contiguous() else \
        gate.detach().transpose(1, 2).clone().transpose(1, 2)
    g.requires_grad_()
    out = M.mi355x_vsa(*leaves, vbs, vbs, topk, block, g)
    grads = torch.autograd.grad(out, leaves + [g], do)
    return out.detach(), grads


@pytest.mark.parametrize("B,H,S,D,be,topk", [(2, 3, 1024, 64, 64, 4), (1, 4, 2048, 128, 256, 3),
                                              (1, 40, 40960, 128, 256, 20)])
def test_token_major_gate_is_bit_identical_to_contiguous_gate(B, H, S, D, be, topk):
    gen = torch.Generator(device=DEV).manual_seed(5)
    q, k, v, do = (torch.randn(B, H, S, D, generator=gen, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    # the producer's layout: [B, S, H, D] contiguous, viewed per head
    g_tm = torch.rand(B, S, H, D, generator=gen, device=DEV, dtype=torch.bfloat16).transpose(1, 2)
    from vsa_mi355x import mi355x as M
    assert M._token_major(g_tm)
    vbs = torch.full((S // be,), be, device=DEV, dtype=torch.int32)
    vbs[-1] = be - 7
    out_a, gr_a = _grads(q, k, v, g_tm, vbs, topk, (1, 1, be), do)
    out_b, gr_b = _grads(q, k, v, g_tm.contiguous(), vbs, topk, (1, 1, be), do)
    assert torch.equal(out_a, out_b)
    for a, b in zip(gr_a, gr_b):
        assert torch.equal(a.contiguous(), b.contiguous())
    # the gate gradient keeps the producer's layout (no transpose copy)
    assert M._token_major(gr_a[3])


def test_gate_producer_trains_end_to_end_against_oracle():
    from vsa_mi355x import CompressionGate
    from vsa_mi355x import mi355x as M
    torch.manual_seed(1)
    B, H, D, be, nb = 1, 2, 64, 64, 6
    S, dim = be * nb, H * D
    hidden = torch.randn(B, S, dim)
    q, k, v = (torch.randn(B, H, S, D) for _ in range(3))
    layer = CompressionGate(dim=dim, num_heads=H)
    vbs = torch.full((nb,), be, dtype=torch.int32)
    # GPU: bf16 Linear (hipBLASLt) + mi355x_vsa, token-major gate
    lg = CompressionGate(dim=dim, num_heads=H).to(DEV, torch.bfloat16)
    lg.load_state_dict(layer.state_dict())
    gate = lg(hidden.to(DEV, torch.bfloat16))
    assert M._token_major(gate)
    out = M.mi355x_vsa(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16),
                       v.to(DEV, torch.bfloat16), vbs.to(DEV), vbs.to(DEV), 2, (1, 1, be), gate)
    out.float().square().mean().backward()
    gw = lg.to_gate_compress.weight.grad
    assert gw is not None and torch.isfinite(gw).all() and gw.abs().sum() > 0
    # oracle: same weights in fp32 on the CPU, bf16 inputs, the GPU's route
    _, sel = M.mi355x_route(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16),
                            v.to(DEV, torch.bfloat16), vbs.to(DEV), vbs.to(DEV), 2, (1, 1, be))
    rg = layer(hidden.to(torch.bfloat16).float())
    ro = O.torch_vsa(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), vbs, vbs,
                     2, (1, 1, be), rg.to(torch.bfloat16), selected=sel.cpu().long())
    ro.float().square().mean().backward()
    rw = layer.to_gate_compress.weight.grad
    rel = ((gw.float().cpu() - rw).norm() / rw.norm()).item()
    assert rel < 3e-2, rel


# ---------------------------------------------------------------------------
# Gates of another dtype or shape: torch_vsa multiplies by
# compress_attn_weight.float() with broadcasting (torch_impl.py:108-113)
# ---------------------------------------------------------------------------

def _gate_case(gate_shape, gate_dtype, seed, tm=False, be=256, nb=4, h=3, d=128):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(seed)
    shape = (1, h, nb * be, d)
    q, k, v, do = (torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(4))
    gate = torch.rand(gate_shape, generator=g).to(gate_dtype)
    if tm:   # the producer's token-major layout, in fp32
        gate = gate.transpose(1, 2).contiguous().transpose(1, 2)
    vbs = torch.full((nb,), be)
    vbs[1] = be - 19
    leaves = [x.to(DEV).requires_grad_() for x in (q, k, v)]
    gd = gate.to(DEV)
    if tm:
        gd = gd.transpose(1, 2).contiguous().transpose(1, 2)
    gd.requires_grad_()
    out = M.mi355x_vsa(*leaves, vbs.to(DEV), vbs.to(DEV), 2, (1, 1, be), gd)
    grads = torch.autograd.grad(out, leaves + [gd], do.to(DEV))
    _, sel = M.mi355x_route(*(x.detach() for x in leaves), vbs.to(DEV), vbs.to(DEV), 2,
                            (1, 1, be))
    ref_leaves = [x.clone().requires_grad_() for x in (q, k, v, gate)]
    ref = O.torch_vsa(*ref_leaves[:3], vbs, vbs, 2, (1, 1, be), ref_leaves[3],
                      selected=sel.cpu().long())
    ref_grads = torch.autograd.grad(ref, ref_leaves, do)
    assert grads[3].dtype == gate_dtype and grads[3].shape == gate.shape
    for name, a, e in zip(("out", "dq", "dk", "dv", "dgate"), [out] + list(grads),
                          [ref] + list(ref_grads)):
        a, e = a.detach().float().cpu(), e.detach().float().cpu()
        diff = (a - e).abs().max().item()
        rel = ((a - e).norm() / e.norm()).item()
        assert diff <= 2e-2 and rel <= 1e-2, f"{name}: max-abs {diff:.3e}, rel-L2 {rel:.3e}"
    return gd, grads


@pytest.mark.parametrize("kind", ["full", "token", "token_major"])
def test_fp32_gate_beside_bf16_inputs(kind):
    """The gate stays fp32 (the reference promotes it, it does not round it to
    bf16) and its gradient comes back in fp32."""
    shape = (1, 3, 1024, 1) if kind == "token" else (1, 3, 1024, 128)
    _gate_case(shape, torch.float32, 81, tm=kind == "token_major")


@pytest.mark.parametrize("shape", [(1, 1, 1024, 1), (1, 3, 1, 128), (1024, 128), (128,),
                                   (1, 3, 1024, 1)])
def test_broadcast_gate_shapes(shape):
    """Any gate shape that broadcasts to [B, H, S, D]; the gradient is reduced
    back to the gate's own shape."""
    _gate_case(shape, torch.bfloat16, 83)


def test_fp32_gate_no_grad_forward_equals_grad_forward():
    from vsa_mi355x import mi355x as M
    g = torch.Generator(device=DEV).manual_seed(85)
    q, k, v = (torch.randn(1, 2, 1024, 128, generator=g, device=DEV, dtype=torch.bfloat16)
               for _ in range(3))
    gate = torch.rand(1, 2, 1024, 128, generator=g, device=DEV, dtype=torch.float32)
    vbs = torch.full((4,), 256, device=DEV, dtype=torch.int32)
    with torch.no_grad():
        a = M.mi355x_vsa(q, k, v, vbs, vbs, 2, (4, 8, 8), gate)
    b = M.mi355x_vsa(q.requires_grad_(), k, v, vbs, vbs, 2, (4, 8, 8), gate)
    assert torch.equal(a, b.detach())


def test_gate_that_does_not_broadcast_is_rejected():
    from vsa_mi355x import mi355x as M
    q = torch.randn(1, 2, 512, 64, device=DEV, dtype=torch.bfloat16)
    vbs = torch.full((2,), 256, device=DEV, dtype=torch.int32)
    with pytest.raises(ValueError, match="compress_attn_weight"):
        M.mi355x_vsa(q, q, q, vbs, vbs, 1, (4, 8, 8), torch.rand(1, 2, 512, 32, device=DEV))


@pytest.mark.parametrize("heads", [3, 22])
def test_per_token_gate_as_a_transposed_view_is_read_by_its_values(heads):
    """A [B, H, S, 1] gate that is the transpose of a contiguous [B, S, H, 1]
    tensor has the strides of a token-major full gate; it must still be read
    as the per-token gate it is (regression: it used to be passed through
    uncopied and read as if contiguous)."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator(device=DEV).manual_seed(87 + heads)
    q, k, v = (torch.randn(1, heads, 1024, 128, generator=g, device=DEV, dtype=torch.bfloat16)
               for _ in range(3))
    base = 2.0 * torch.rand(1, 1024, heads, 1, generator=g, device=DEV, dtype=torch.bfloat16)
    view = base.transpose(1, 2)
    assert not view.is_contiguous()
    vbs = torch.full((4,), 256, device=DEV, dtype=torch.int32)
    with torch.no_grad():
        a = M.mi355x_vsa(q, k, v, vbs, vbs, 2, (4, 8, 8), view)
        b = M.mi355x_vsa(q, k, v, vbs, vbs, 2, (4, 8, 8), view.contiguous())
    assert torch.equal(a, b)
