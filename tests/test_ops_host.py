"""The torch.library custom ops: registered schemas and the fake (shape-only)
implementations torch.compile traces with (no GPU needed)."""

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from vsa_mi355x import ops  # noqa: F401  (registers the ops)


def _t(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="cuda", dtype=dtype)


def test_ops_are_registered():
    for name in ("vsa_fwd", "vsa_bwd", "sparse_fwd", "sparse_bwd"):
        assert hasattr(torch.ops.vsa_mi355x, name), name


def test_full_op_fake_shapes():
    b, h, s, d, be, tk = 2, 3, 1024, 128, 256, 2
    qb = s // be
    with FakeTensorMode():
        q, k, v, g = (_t(b, h, s, d) for _ in range(4))
        vbs = _t(qb, dtype=torch.int32)
        outs = torch.ops.vsa_mi355x.vsa_fwd(q, k, v, g, vbs, vbs, tk, be, 0.1, True)
        want = [((b, h, s, d), torch.bfloat16), ((b, h, qb, d), torch.bfloat16),
                ((b, h, qb, d), torch.bfloat16), ((b, h, qb, d), torch.bfloat16),
                ((b, h, qb, qb), torch.float32), ((b, h, qb, d), torch.bfloat16),
                ((b, h, qb, tk), torch.int32), ((b, h, s, d), torch.bfloat16),
                ((b, h, s), torch.float32)]
        for o, (shape, dtype) in zip(outs, want):
            assert tuple(o.shape) == shape and o.dtype == dtype
        no_save = torch.ops.vsa_mi355x.vsa_fwd(q, k, v, None, vbs, vbs, tk, be, 0.1, False)
        assert tuple(no_save[0].shape) == (b, h, s, d)
        assert all(o.numel() == 0 for o in no_save[1:])
        grads = torch.ops.vsa_mi355x.vsa_bwd(q, q, k, v, g, vbs, vbs, *outs[1:], be, 0.1)
        assert [tuple(x.shape) for x in grads] == [(b, h, s, d)] * 4
        grads = torch.ops.vsa_mi355x.vsa_bwd(q, q, k, v, None, vbs, vbs, *outs[1:], be, 0.1)
        assert grads[3].numel() == 0


def test_explicit_route_fake_shapes():
    b, h, s, d, be, tk = 1, 2, 512, 64, 64, 3
    with FakeTensorMode():
        q, k, v = (_t(b, h, s, d) for _ in range(3))
        sel = _t(b, h, s // be, tk, dtype=torch.int32)
        vbs = _t(s // be, dtype=torch.int32)
        out, lse = torch.ops.vsa_mi355x.sparse_fwd(q, k, v, sel, vbs, be, 0.125, True)
        assert tuple(out.shape) == (b, h, s, d) and tuple(lse.shape) == (b, h, s)
        assert lse.dtype == torch.float32
        grads = torch.ops.vsa_mi355x.sparse_bwd(q, q, k, v, out, lse, sel, vbs, be, 0.125)
        assert [tuple(x.shape) for x in grads] == [(b, h, s, d)] * 3
