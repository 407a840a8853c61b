"""GPU: the backward's delta comes from the fine output as stored in T.

The reference keeps the fine (sparse) output as its own tensor, rounded to the
input dtype, and forms ``delta = rowsum(float(O) * float(dO))`` from it
(triton_impl.py:408, 598-700).  Recovering the fine output from the rounded
combined output instead (``T(out) - out_c * gate``) carries the rounding error
of ``|out|``, not of ``|O|``: on video-like inputs, where neighbouring tokens
share a large per-block component and the coarse branch is as large as the fine
one, that doubles the delta error.  These tests use such inputs: every block
gets a per-block offset ~ N(0, 2^2) per channel, broadcast over its tokens, plus
0.2 * N(0, 1) per token, and the gate is U(0, 2).
"""

import pytest
import torch

from oracle import vsa_oracle as O

from test_gpu_parity import DEV

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _video(shape, be, gen, offset=2.0, noise=0.2):
    b, h, s, d = shape
    nb = s // be
    blocks = torch.randn(b, h, nb, 1, d, generator=gen) * offset
    return blocks.expand(b, h, nb, be, d).reshape(shape) + noise * torch.randn(shape, generator=gen)


def _case(seed, be=256, nb=8, h=2, d=128, tk=4, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    shape = (1, h, nb * be, d)
    q, k, v = (_video(shape, be, g).to(dtype) for _ in range(3))
    do = torch.randn(shape, generator=g).to(dtype)
    gate = (2.0 * torch.rand(shape, generator=g)).to(dtype)
    vbs = torch.full((nb,), be)
    vbs[-1] = be - 37
    return q, k, v, do, gate, vbs, tk, be


@pytest.mark.parametrize("seed", [61, 62])
def test_delta_from_stored_fine_output_on_video_like_inputs(seed):
    """delta against the exact fine output: relative L2 <= 2.4e-3.  With
    T(out) - out_c*gate the same inputs give about 3.4e-3 (a CPU simulation of
    both schemes gives 1.7e-3 vs 3.4e-3 at these settings)."""
    from vsa_mi355x import mi355x as M
    q, k, v, do, gate, vbs, tk, be = _case(seed)
    scale = q.shape[-1] ** -0.5
    qd, kd, vd, dod, gd = (t.to(DEV) for t in (q, k, v, do, gate))
    vbs_d = vbs.to(DEV, torch.int32)
    with torch.no_grad():
        qc, kc, vc = M.block_mean_qkv(qd, kd, vd, vbs_d, vbs_d, be)
        _, _, outc, sel = M.coarse_forward(qc, kc, vc, tk, scale)
        out, _, fine = M.sparse_forward(qd, kd, vd, sel, vbs_d, be, scale, out_c=outc, gate=gd)
        delta, _, _ = M.backward_prep(fine, dod, be, out_c=outc, gate=gd)
        # the stored fine output is bit for bit the explicit-route forward's output
        alone, _, _ = M.sparse_forward(qd, kd, vd, sel, vbs_d, be, scale)
    assert torch.equal(fine, alone)
    o_s, _ = O.sparse_attention_reference(q, k, v, sel.cpu().long(), vbs, be, scale)
    exact = (o_s * do.float()).sum(-1)
    err = (delta.cpu() - exact).norm() / exact.norm()
    assert err <= 2.4e-3, f"delta rel-L2 {err:.3e}"
    # the combine is as large as the fine branch here (otherwise the test pins nothing)
    c = (out.float().cpu() - fine.float().cpu()).norm() / fine.float().cpu().norm()
    assert c > 0.5, f"coarse/fine ratio {c:.2f}"


@pytest.mark.parametrize("seed", [63, 64])
def test_full_op_parity_on_video_like_inputs(seed):
    """Full fused op, forward and every gradient, on the GPU's route.

    Relative L2 against the oracle stays at the north-star 1e-2.  A plain
    max-abs 2e-2 does not fit these magnitudes (out and dq reach |x| ~ 20,
    where one bf16 ulp is 0.125): the oracle itself, run on the same bf16
    inputs, is 0.07-0.25 max-abs away from the same formula evaluated in fp64.
    So the elementwise bar is taken against the fp64 evaluation: the GPU's
    worst element is no further from it than the oracle's worst element plus
    2e-2."""
    from vsa_mi355x import mi355x as M
    q, k, v, do, gate, vbs, tk, be = _case(seed)
    qg, kg, vg, gg = (x.to(DEV).requires_grad_() for x in (q, k, v, gate))
    vbs_d = vbs.to(DEV)
    out = M.mi355x_vsa(qg, kg, vg, vbs_d, vbs_d, tk, (4, 8, 8), gg)
    out.backward(do.to(DEV))
    _, sel = M.mi355x_route(qg.detach(), kg.detach(), vg.detach(), vbs_d, vbs_d, tk, (4, 8, 8))

    def oracle(dtype):
        leaves = [x.clone().to(dtype).requires_grad_() for x in (q, k, v, gate)]
        ref = O.torch_vsa(*leaves[:3], vbs, vbs, tk, (4, 8, 8), leaves[3],
                          selected=sel.cpu().long())
        ref.backward(do.to(dtype))
        return [ref] + [x.grad for x in leaves]

    ref, exact = oracle(q.dtype), oracle(torch.float64)
    gpu = [out, qg.grad, kg.grad, vg.grad, gg.grad]
    for name, a, e, x in zip(("out", "dq", "dk", "dv", "dgate"), gpu, ref, exact):
        a, e, x = (t.detach().double().cpu() for t in (a, e, x))
        assert torch.isfinite(a).all(), f"{name}: non-finite values"
        rel = ((a - e).norm() / e.norm()).item()
        worst, worst_ref = (a - x).abs().max().item(), (e - x).abs().max().item()
        assert rel <= 1e-2 and worst <= worst_ref + 2e-2, (
            f"{name}: rel-L2 vs oracle {rel:.3e}; max-abs vs fp64 {worst:.3e} "
            f"(oracle's {worst_ref:.3e})")
