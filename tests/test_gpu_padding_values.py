"""GPU: values held in padding tokens never reach the results.

A token at or past its block's valid count (``variable_block_sizes``) is
padding.  The reference's block mean multiplies it by a zero mask
(common.py:78-80; tests/test_common.py:81-88 puts 999 there), and its fine
branch fills the scores of padding keys with -inf before the softmax
(common.py:259-264), so a padding key gets probability 0 and no gradient.

Here the padding of q, k and v holds U(-200, 200): scores against it spread
over about +-100 nats, enough to overflow an exponential taken before the
mask or to swamp a running max that saw an unmasked key.  Against the same inputs with
zero padding, and with dO zero on padding query rows (their outputs are
defined, but depend on their own q), the following must hold bit for bit:
the output and dQ of every valid query row, dK and dV of every valid key, and
the gate gradient; dK and dV of padding keys must be exactly zero; and
everything must be finite."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
POISON = 200.0


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _valid(vbs, be):
    """[nb * be] bool: token t of block n is valid when t % be < vbs[n]."""
    pos = torch.arange(be, device=DEV)
    return (pos.view(1, be) < vbs.to(DEV).view(-1, 1)).reshape(-1)


def _poison(x, valid, g):
    noise = (torch.rand(x.shape, generator=g, device=DEV) * 2 - 1) * POISON
    return torch.where(valid.view(1, 1, -1, 1), x, noise.to(x.dtype))


def _run(fn, q, k, v, gate, do):
    leaves = [x.detach().clone().requires_grad_() for x in (q, k, v)]
    gl = gate.detach().clone().requires_grad_() if gate is not None else None
    out = fn(*leaves, gl)
    wrt = leaves + ([gl] if gl is not None else [])
    return [out.detach()] + list(torch.autograd.grad(out, wrt, do))


CASES = [
    # batch, heads, blocks, head_dim, block, dtype, gate, topk
    (1, 3, 5, 64, 64, torch.bfloat16, "full", 2),      # 4-wave kernels, block 64
    (1, 32, 8, 128, 256, torch.bfloat16, "token", 3),  # 8-wave ping-pong forward / dQ
    (2, 2, 6, 128, 128, torch.float16, None, 4),       # block 128, fp16
    (1, 2, 4, 64, 64, torch.float32, "full", 2),       # fp32 kernels
    (1, 2, 4, 256, 64, torch.bfloat16, None, 2),       # head_dim 256 kernels
]


@pytest.mark.parametrize("b,h,nb,d,be,dtype,gate,topk", CASES)
def test_poisoned_padding_leaves_the_full_op_unchanged(b, h, nb, d, be, dtype, gate, topk):
    from vsa_mi355x import mi355x as M
    print(f"case b={b} h={h} nb={nb} d={d} be={be} {dtype} gate={gate} topk={topk}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(nb * 7 + d)
    s = nb * be
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[1], vbs[-1] = be // 2 + 3, 5       # a half-full block and an almost empty last block
    qvbs = vbs.roll(1)
    kvalid, qvalid = _valid(vbs, be), _valid(qvbs, be)
    q, k, v = (torch.randn(b, h, s, d, generator=g, device=DEV).to(dtype) for _ in range(3))
    q = torch.where(qvalid.view(1, 1, -1, 1), q, torch.zeros_like(q))
    k = torch.where(kvalid.view(1, 1, -1, 1), k, torch.zeros_like(k))
    v = torch.where(kvalid.view(1, 1, -1, 1), v, torch.zeros_like(v))
    gt = None
    if gate == "full":
        gt = torch.rand(b, h, s, d, generator=g, device=DEV).to(dtype)
    elif gate == "token":
        gt = torch.rand(b, h, s, 1, generator=g, device=DEV).to(dtype)
    do = torch.randn(b, h, s, d, generator=g, device=DEV).to(dtype)
    do = torch.where(qvalid.view(1, 1, -1, 1), do, torch.zeros_like(do))

    def op(q_, k_, v_, g_):
        return M.mi355x_vsa(q_, k_, v_, vbs, qvbs, topk, (1, 1, be), g_)

    clean = _run(op, q, k, v, gt, do)
    dirty = _run(op, _poison(q, qvalid, g), _poison(k, kvalid, g), _poison(v, kvalid, g), gt, do)
    for name, a in zip(["out", "dq", "dk", "dv", "dgate"], dirty):
        assert torch.isfinite(a.float()).all(), name
    qrows, krows = qvalid.view(1, 1, -1, 1), kvalid.view(1, 1, -1, 1)
    for name, a, e, rows in zip(["out", "dq", "dk", "dv"], dirty, clean,
                                [qrows, qrows, krows, krows]):
        assert torch.equal(torch.where(rows, a, 0), torch.where(rows, e, 0)), name
    for name, a in zip(["dk", "dv"], dirty[2:4]):
        assert not torch.where(krows, 0, a).any(), f"{name} of padding keys"
    if gt is not None:
        assert torch.equal(torch.where(qrows, dirty[4], 0), torch.where(qrows, clean[4], 0)), \
            "dgate"


def test_poisoned_padding_leaves_the_explicit_route_unchanged():
    """mi355x_sparse_attention with an explicit route that selects the
    half-full and the almost empty key block for every query block."""
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be = 1, 4, 6, 128, 64
    g = torch.Generator(device=DEV).manual_seed(3)
    s = nb * be
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[1], vbs[-1] = 35, 5
    kvalid = _valid(vbs, be)
    krows = kvalid.view(1, 1, -1, 1)
    q = torch.randn(b, h, s, d, generator=g, device=DEV).to(torch.bfloat16)
    k, v = (torch.where(krows, torch.randn(b, h, s, d, generator=g, device=DEV), 0.0)
            .to(torch.bfloat16) for _ in range(2))
    do = torch.randn(b, h, s, d, generator=g, device=DEV).to(torch.bfloat16)
    sel = torch.tensor([1, nb - 1, 0], dtype=torch.int32, device=DEV).expand(b, h, nb, 3)
    sel = sel.contiguous()

    def op(q_, k_, v_, _g):
        return M.mi355x_sparse_attention(q_, k_, v_, sel, vbs, block_size=(1, 1, be))

    clean = _run(op, q, k, v, None, do)
    dirty = _run(op, q, _poison(k, kvalid, g), _poison(v, kvalid, g), None, do)
    for name, a, e in zip(["out", "dq"], dirty[:2], clean[:2]):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, e), name
    for name, a, e in zip(["dk", "dv"], dirty[2:], clean[2:]):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(torch.where(krows, a, 0), torch.where(krows, e, 0)), name
        assert not torch.where(krows, 0, a).any(), f"{name} of padding keys"


@pytest.mark.parametrize("h,nb,be", [(4, 5, 64), (32, 8, 256)])
def test_poisoned_padding_leaves_token_major_views_unchanged(h, nb, be):
    """The same check on per-head views of token-major [B, S, H, D] tensors,
    which run the kernels' raster instantiations."""
    from vsa_mi355x import mi355x as M
    b, d, topk = 1, 128, 2
    g = torch.Generator(device=DEV).manual_seed(h + nb)
    s = nb * be
    vbs = torch.full((nb,), be, dtype=torch.int32)
    vbs[1], vbs[-1] = be // 2 + 3, 5
    qvbs = vbs.roll(1)
    kvalid, qvalid = _valid(vbs, be), _valid(qvbs, be)
    # [B, S, H, D] with the padding tokens zeroed (clean) or poisoned (dirty)
    tok = [torch.randn(b, s, h, d, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3)]
    masks = [qvalid, kvalid, kvalid]
    clean_tm = [torch.where(m.view(1, -1, 1, 1), x, 0) for x, m in zip(tok, masks)]
    dirty_tm = [_poison(x.transpose(1, 2), m, g).transpose(1, 2).contiguous()
                for x, m in zip(clean_tm, masks)]
    do = torch.randn(b, h, s, d, generator=g, device=DEV).to(torch.bfloat16)
    do = torch.where(qvalid.view(1, 1, -1, 1), do, 0)

    def run(tensors):
        leaves = [x.detach().clone().requires_grad_() for x in tensors]
        views = [x.transpose(1, 2) for x in leaves]
        assert M._raster_views(*views, None, be)
        out = M.mi355x_vsa(*views, vbs, qvbs, topk, (1, 1, be))
        grads = torch.autograd.grad(out, leaves, do)
        return [out.detach()] + [gr.transpose(1, 2) for gr in grads]

    clean, dirty = run(clean_tm), run(dirty_tm)
    qrows, krows = qvalid.view(1, 1, -1, 1), kvalid.view(1, 1, -1, 1)
    for name, a, e, rows in zip(["out", "dq", "dk", "dv"], dirty, clean,
                                [qrows, qrows, krows, krows]):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(torch.where(rows, a, 0), torch.where(rows, e, 0)), name
    for name, a in zip(["dk", "dv"], dirty[2:4]):
        assert not torch.where(krows, 0, a).any(), f"{name} of padding keys"
