"""GPU parity of the coarse branch on the MFMA kernels and of the radix Top-K.

Bars: Top-K ids bit-exact against the oracle's rule on identical fp32 scores;
coarse scores and probabilities within 2 ulp of T of the oracle's (fp32 sums
taken in another order flip a rounding now and then); out_c and the coarse
gradients within max-abs 2e-2 and relative-L2 1e-2 (bf16 / fp16)."""

import numpy as np
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


def _parity(actual, expected, what, max_abs=2e-2, rel_l2=1e-2):
    a, e = actual.detach().float().cpu(), expected.detach().float().cpu()
    assert a.shape == e.shape, what
    assert torch.isfinite(a).all(), what
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    assert diff <= max_abs and rel <= rel_l2, f"{what}: max-abs {diff:.3e}, rel-L2 {rel:.3e}"


def _within_ulps(got, exp, dtype, n, what, slack=0.0):
    """|got - exp| <= n ulp of T at exp, plus `slack` (an absolute bound on the
    fp32 error of a sum taken in another order)."""
    g, e = got.float().cpu(), exp.float().cpu()
    fi = torch.finfo(dtype)
    ulp = fi.eps * e.abs() + fi.eps * fi.tiny      # the subnormal spacing below tiny
    bad = (g - e).abs() > n * ulp + slack
    assert not bad.any(), f"{what}: {int(bad.sum())} values beyond {n} ulp"


# (qb, kb): tile remainders on both sides, one block, the c3 / t444 grids
SIZES = [(1, 1), (45, 37), (33, 70), (7, 258), (320, 320), (640, 640)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("qb,kb", SIZES)
def test_coarse_forward_mfma_matches_oracle(dtype, D, qb, kb):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(qb * 1000 + kb + D)
    bh, tk = 3, min(8, kb)
    qc, kc, vc = (torch.randn(1, bh, n, D, generator=g).to(dtype) for n in (qb, kb, kb))
    scale = D ** -0.5
    scores, probs, outc, sel = M.coarse_forward(qc.to(DEV), kc.to(DEV), vc.to(DEV), tk, scale)
    # block_mean over one-token blocks is the identity, so the oracle's coarse
    # branch on (qc, kc, vc) with block_elements 1 is the pooled computation
    ones_q, ones_k = torch.ones(qb, dtype=torch.long), torch.ones(kb, dtype=torch.long)
    exp_scores, exp_out = O.coarse_branch_compact(qc, kc, vc, ones_k, ones_q, 1, scale)
    s_gpu = scores.cpu()
    if s_gpu.numel() >= 1000:
        assert (s_gpu != exp_scores.float()).float().mean() < 0.01
    # a dot product that cancels to near zero carries the fp32 summation error
    # (at most D eps32 sum|q_d k_d|, twice for the two orders) into the rounding
    absdot = torch.matmul(qc.float().abs(), kc.float().abs().transpose(-2, -1).contiguous())
    slack = scale * 2 * D * torch.finfo(torch.float32).eps * absdot
    _within_ulps(s_gpu, exp_scores, dtype, 2, "scores", slack)
    # probabilities: softmax of the kernel's own scores, rounded to T
    exp_p = torch.softmax(s_gpu, dim=-1).to(dtype)
    _within_ulps(probs.cpu(), exp_p, dtype, 1, "probs")
    _parity(outc, exp_out, "out_c")
    ref = np.sort(O.topk_reference(s_gpu, tk), axis=-1)
    assert np.array_equal(sel.cpu().numpy(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("qb,kb", [(1, 1), (45, 37), (33, 70), (320, 320), (640, 640)])
def test_coarse_backward_mfma_matches_oracle_autograd(dtype, D, qb, kb):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(qb * 7 + kb + D)
    bh = 2
    qc, kc, vc = (torch.randn(1, bh, n, D, generator=g).to(dtype) for n in (qb, kb, kb))
    dout = torch.randn(1, bh, qb, D, generator=g).to(dtype)
    scale = D ** -0.5
    _, probs, _, _ = M.coarse_forward(qc.to(DEV), kc.to(DEV), vc.to(DEV), None, scale)
    dqc, dkc, dvc = M.coarse_backward(qc.to(DEV), kc.to(DEV), vc.to(DEV), probs, dout.to(DEV),
                                      scale)
    leaves = [t.clone().requires_grad_() for t in (qc, kc, vc)]
    ones_q, ones_k = torch.ones(qb, dtype=torch.long), torch.ones(kb, dtype=torch.long)
    _, out = O.coarse_branch_compact(*leaves, ones_k, ones_q, 1, scale)
    rq, rk, rv = torch.autograd.grad(out, leaves, dout)
    for what, a, e in (("d_q_c", dqc, rq), ("d_k_c", dkc, rk), ("d_v_c", dvc, rv)):
        # relative to the gradient's own size: coarse gradients are small
        s = e.float().abs().max().clamp_min(1e-6)
        _parity(a.float() / s, e.float() / s, what)


def test_coarse_backward_is_deterministic():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(3)
    qc, kc, vc, do = (torch.randn(1, 4, 200, 128, generator=g).to(torch.bfloat16).to(DEV)
                      for _ in range(4))
    _, probs, _, _ = M.coarse_forward(qc, kc, vc, None, 0.1)
    a = M.coarse_backward(qc, kc, vc, probs, do, 0.1)
    b = M.coarse_backward(qc, kc, vc, probs, do, 0.1)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


# ---------------------------------------------------------------------------
# Radix Top-K edge cases
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kb,tk", [(1, 1), (5, 5), (300, 1), (300, 300), (4096, 64),
                                   (4096, 4095), (1000, 999)])
def test_topk_radix_sizes_with_ties(kb, tk):
    from vsa_mi355x import mi355x as M
    rng = np.random.default_rng(kb + tk)
    scores = torch.from_numpy(rng.integers(-3, 4, size=(5, kb)).astype(np.float32) / 4)
    got = M.topk(scores.to(DEV), tk).cpu().numpy()
    assert np.array_equal(got, np.sort(O.topk_reference(scores, tk), axis=-1))


def test_topk_radix_special_values():
    from vsa_mi355x import mi355x as M
    inf = float("inf")
    rows = torch.tensor([
        [0.0, -0.0, 0.0, -0.0, 1e-30, -1e-30],      # -0 == +0: ties go to smaller ids
        [-inf, inf, 3.0, inf, -inf, 2.0],
        [5.0] * 6,                                    # one value everywhere
        [-1.0, -2.0, -3.0, -4.0, -5.0, -6.0],
        [1.0, float("nan"), 3.0, float("nan"), -inf, 2.0],  # NaN ranks above +inf
    ], dtype=torch.float32)
    got = M.topk(rows.to(DEV), 3).cpu().tolist()
    assert got[0] == [0, 1, 4]
    assert got[1] == [1, 2, 3]
    assert got[2] == [0, 1, 2]
    assert got[3] == [0, 1, 2]
    assert got[4] == [1, 2, 3]
    # the oracle's rule agrees wherever no NaN is present
    ref = np.sort(O.topk_reference(rows[:4], 3), axis=-1)
    assert np.array_equal(np.array(got[:4]), ref)


def test_topk_radix_one_distinct_winner_many_ties_below():
    # the k-th value is shared by most of the row: the last digit pass resolves it
    from vsa_mi355x import mi355x as M
    kb = 2048
    row = torch.full((2, kb), 0.5)
    row[0, 1000] = 0.75
    row[1, 5] = 0.75
    row[1, 2000] = 0.625
    got = M.topk(row.to(DEV), 4).cpu().tolist()
    assert got[0] == [0, 1, 2, 1000]
    assert got[1] == [0, 1, 5, 2000]
