"""GPU: the op on two HIP streams at once.

Every launch goes to torch's current stream.  The dK/dV tile order and its
counters live in a per-call workspace; the persistent forward and dQ kernels
take their query blocks from scheduling counters of their own stream's slot (a
device array with 256 slots per GPU; each launch leaves its slot zeroed), and
a stream that finds every slot taken runs them with a fixed stride instead.
So two fwd+bwd steps issued on two side streams, with their kernels free to
overlap, must give exactly the results of the same steps run one after the
other on the default stream, and so must a step on a stream without a slot."""

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


def _case(seed, b, h, nb, d, be):
    g = torch.Generator(device=DEV).manual_seed(seed)
    s = nb * be
    q, k, v, do = (torch.randn(b, h, s, d, generator=g, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = torch.rand(b, h, s, d, generator=g, device=DEV, dtype=torch.bfloat16)
    vbs = torch.full((nb,), be, dtype=torch.int32, device=DEV)
    vbs[-1] = be - 29
    return q, k, v, gate, do, vbs


def _step(q, k, v, gate, do, vbs, be, topk):
    from vsa_mi355x import mi355x as M
    leaves = [x.detach().clone().requires_grad_() for x in (q, k, v, gate)]
    out = M.mi355x_vsa(*leaves[:3], vbs, vbs, topk, (1, 1, be), leaves[3])
    return [out.detach()] + list(torch.autograd.grad(out, leaves, do))


@pytest.mark.parametrize("be,nb,d,h", [(256, 16, 128, 20), (64, 24, 64, 6)])
def test_two_streams_give_the_sequential_results(be, nb, d, h):
    topk = 4
    cases = [_case(11, 1, h, nb, d, be), _case(12, 2, h, nb, d, be)]
    ref = [_step(*c, be, topk) for c in cases]
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    main = torch.cuda.current_stream()
    got = [None, None]
    for i, st in enumerate(streams):
        st.wait_stream(main)
    for rep in range(3):  # several rounds, so that the two streams' kernels interleave
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                got[i] = _step(*cases[i], be, topk)
        for st in streams:
            main.wait_stream(st)
        torch.cuda.synchronize()
        for i in range(2):
            for name, a, e in zip(["out", "dq", "dk", "dv", "dgate"], got[i], ref[i]):
                assert torch.equal(a, e), (rep, i, name)


def test_stream_without_a_scheduling_slot_gives_the_same_results():
    """More streams than slots: the forward and dQ kernels of the 8-wave path
    (head dim 128, block 256, >= 256 query blocks) fall back to a fixed
    stride over their XCD's range and must give the results of the counters."""
    from vsa_mi355x import mi355x as M
    be, nb, d, h, topk = 256, 16, 128, 20, 4                 # 320 query blocks
    case = _case(13, 1, h, nb, d, be)
    ref = _step(*case, be, topk)
    torch.cuda.synchronize()
    # one small forward of the 8-wave kernel on each new stream takes a slot
    g = torch.Generator(device=DEV).manual_seed(5)
    sq = 16 * 256                                            # 16 heads x 16 blocks = 256
    q1, k1, v1 = (torch.randn(1, 16, sq, 128, generator=g, device=DEV, dtype=torch.bfloat16)
                  for _ in range(3))
    sel = torch.zeros(1, 16, 16, 1, dtype=torch.int32, device=DEV)
    vbs1 = torch.full((16,), 256, dtype=torch.int32, device=DEV)
    want = M.sparse_forward(q1, k1, v1, sel, vbs1, 256, 0.1)[0]
    streams = [torch.cuda.Stream() for _ in range(260)]      # default priority
    main = torch.cuda.current_stream()
    for st in streams:
        st.wait_stream(main)
        with torch.cuda.stream(st):
            got1 = M.sparse_forward(q1, k1, v1, sel, vbs1, 256, 0.1)[0]
        main.wait_stream(st)
        torch.cuda.synchronize()
        assert torch.equal(got1, want)
    last = torch.cuda.Stream()
    last.wait_stream(main)
    with torch.cuda.stream(last):
        got = _step(*case, be, topk)
    main.wait_stream(last)
    torch.cuda.synchronize()
    for name, a, e in zip(["out", "dq", "dk", "dv", "dgate"], got, ref):
        assert torch.equal(a, e), name
