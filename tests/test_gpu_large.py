"""GPU: tensors of more than 2^31 elements (every offset into q, k, v, the
gate, dO and the outputs is 64-bit).

The c4 shape (S = 92,160, 40 heads, head_dim 128, blocks of 256 with every
eighth block at 192 tokens, topk 45, full gate) at batch 5 holds 2.36e9
elements per tensor (4.7 GB each, about 60 GB for the step).  Heads and batch
entries are independent and the kernels are deterministic, so the first and
the last batch entry of that step (the last one sits wholly past element 2^31)
must equal the op run on that entry alone, output and every gradient, bit for
bit."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
B, H, S, D, BE, TOPK = 5, 40, 92160, 128, 256, 45


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _step(q, k, v, gate, do, vbs):
    from vsa_mi355x import mi355x as M
    leaves = [x.detach().requires_grad_() for x in (q, k, v, gate)]
    out = M.mi355x_vsa(*leaves[:3], vbs, vbs, TOPK, (1, 1, BE), leaves[3])
    grads = torch.autograd.grad(out, leaves, do)
    return [out.detach()] + list(grads)


def test_batch_entries_past_2_31_elements_equal_single_entry_runs():
    assert B * H * S * D > 2 ** 31
    free, _ = torch.cuda.mem_get_info()
    if free < 100 * 2 ** 30:
        pytest.skip(f"needs about 60 GB of free HBM ({free / 2 ** 30:.0f} GiB free)")
    g = torch.Generator(device=DEV).manual_seed(8)
    shape = (B, H, S, D)
    q, k, v, do = (torch.randn(shape, generator=g, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = torch.rand(shape, generator=g, device=DEV, dtype=torch.bfloat16)
    vbs = torch.full((S // BE,), BE, dtype=torch.int32, device=DEV)
    vbs[7::8] = 192
    print(f"batch {B} step, {B * H * S * D / 1e9:.2f}e9 elements per tensor", flush=True)
    full = _step(q, k, v, gate, do, vbs)
    torch.cuda.synchronize()
    for b in (0, B - 1):
        print(f"batch entry {b} alone", flush=True)
        one = _step(*(x[b:b + 1].clone() for x in (q, k, v, gate, do)), vbs)
        for name, a, e in zip(["out", "dq", "dk", "dv", "dgate"], full, one):
            assert torch.isfinite(e.float()).all(), name
            assert torch.equal(a[b:b + 1], e), (name, b)
        del one
