"""GPU: the fwd+bwd step captured in a HIP graph (torch.cuda.CUDAGraph) and
replayed.

The op launches only kernels on the current stream, allocates with
torch.empty and never synchronises or reads device memory on the host, so a
training or serving loop can capture it.  Each replay runs on new inputs copied
into the captured tensors, with eager work and synchronisations between the
replays, and must equal the eager op on the same inputs bit for bit (the
kernels are deterministic).  Block sizes are device int32 tensors (a host
tensor would need a copy inside the capture)."""

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


def _capture_and_replay(step, make_inputs, replays=3):
    """step(*inputs) -> list of tensors; inputs from make_inputs(seed)."""
    static = [x.clone() for x in make_inputs(0)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(*static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(*static)
    for seed in range(1, replays + 1):
        fresh = make_inputs(seed)
        with torch.no_grad():
            for s_, f in zip(static, fresh):
                s_.copy_(f)
        graph.replay()
        torch.cuda.synchronize()
        eager = step(*[f.clone() for f in fresh])
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (seed, i, (a.float() - b.float()).abs().max().item())


def _qkv(seed, shape, dtype=torch.bfloat16, n=4):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn(*shape, generator=g, device=DEV, dtype=dtype) for _ in range(n)]


def test_full_op_fwd_bwd_replays_equal_eager():
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be, topk = 1, 4, 8, 128, 256, 3
    shape = (b, h, nb * be, d)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = 200

    def make(seed):
        q, k, v, do = _qkv(seed, shape)
        gate = torch.rand(*shape, generator=torch.Generator(device=DEV).manual_seed(seed + 99),
                          device=DEV, dtype=torch.bfloat16)
        return [q, k, v, gate, do]

    def step(q, k, v, gate, do):
        leaves = [x.detach().requires_grad_() for x in (q, k, v, gate)]
        out = M.mi355x_vsa(*leaves[:3], vbs, vbs, topk, (4, 8, 8), leaves[3])
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do))

    _capture_and_replay(step, make)


def test_explicit_route_fwd_bwd_replays_equal_eager():
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be, topk = 1, 3, 10, 64, 64, 4
    shape = (b, h, nb * be, d)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    sel = torch.stack([torch.randperm(nb, generator=g, device=DEV)[:topk]
                       for _ in range(b * h * nb)]).view(b, h, nb, topk).to(torch.int32)

    def step(q, k, v, do):
        leaves = [x.detach().requires_grad_() for x in (q, k, v)]
        out = M.mi355x_sparse_attention(*leaves, sel, vbs, block_size=(1, 1, be))
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do))

    _capture_and_replay(step, lambda seed: _qkv(seed, shape))


def test_token_major_views_fwd_bwd_replays_equal_eager():
    from vsa_mi355x import mi355x as M
    b, h, nb, d, be, topk = 1, 4, 6, 128, 128, 2
    s = nb * be
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)

    def step(q, k, v, do):
        leaves = [x.detach().requires_grad_() for x in (q, k, v)]
        views = [x.transpose(1, 2) for x in leaves]
        out = M.mi355x_vsa(*views, vbs, vbs, topk, (1, 1, be))
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do.transpose(1, 2)))

    _capture_and_replay(step, lambda seed: _qkv(seed, (b, s, h, d)))
