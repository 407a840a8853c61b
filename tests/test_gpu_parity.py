"""GPU parity: every MI355X kernel against the CPU oracle on seeded inputs.

Bars (north_star): Top-K ids and CSR metadata bit-exact given identical fp32
scores / routes; outputs and gradients within max-abs 2e-2 and relative-L2
1e-2 for bf16 / fp16.  Inputs are generated on the CPU and copied over, the
oracle runs on the CPU.  Cases mirror tests/test_triton_vsa.py and
tests/test_helion_vsa.py of the reference."""

import math

import numpy as np
import pytest
import torch

from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_ABS = 2e-2
REL_L2 = 1e-2


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")


@pytest.fixture(autouse=True)
def _gpu_only():
    _need_gpu()
    from vsa_mi355x import _lib
    _lib.load()          # fail loudly (not skip) when the kernels are not built
    yield


def assert_parity(actual, expected, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    diff = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    assert diff <= max_abs and rel <= rel_l2, f"{what}: max-abs {diff:.3e}, rel-L2 {rel:.3e}"


def _randn(shape, gen, dtype, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(dtype)


def _gpu(*ts):
    return [t.to(DEV) if t is not None else None for t in ts]


# ---------------------------------------------------------------------------
# Pooling (fused_common.py:20-59; tests/test_triton_vsa.py:25-61)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("be,vbs", [(64, [64, 37, 11]), (256, [256, 191, 73, 0])])
def test_block_mean_matches_oracle(dtype, be, vbs):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(11)
    nb = len(vbs)
    q = _randn((1, 2, nb * be, 128), g, dtype)
    k = _randn((1, 2, nb * be, 128), g, dtype)
    v = _randn((1, 2, nb * be, 128), g, dtype)
    vbs_t = torch.tensor(vbs)
    qc, kc, vc = M.block_mean_qkv(*_gpu(q, k, v), vbs_t.to(DEV), vbs_t.to(DEV), be)
    torch.cuda.synchronize()
    tol = 0 if dtype == torch.float32 else 1
    for got, x in ((qc, q), (kc, k), (vc, v)):
        exp = O.block_mean(x, vbs_t, be)
        if dtype == torch.float32:
            torch.testing.assert_close(got.cpu(), exp, atol=1e-6, rtol=1e-5)
        else:
            # fp32 sums in a different order: at most one ulp of T apart
            ulp = torch.finfo(dtype).eps * exp.float().abs().clamp_min(torch.finfo(dtype).tiny)
            assert ((got.cpu().float() - exp.float()).abs() <= ulp * 2 + 1e-30).all()


# ---------------------------------------------------------------------------
# Top-K: bit-exact on identical fp32 scores, ties to the smaller id
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kb,tk", [(13, 5), (160, 20), (360, 45), (640, 32)])
def test_topk_bit_exact_with_ties(kb, tk):
    from vsa_mi355x import mi355x as M
    rng = np.random.default_rng(kb)
    # coarse values produce many exact ties at the k-th boundary
    scores = torch.from_numpy(rng.integers(-6, 7, size=(3, 37, kb)).astype(np.float32) / 8)
    got = M.topk(scores.to(DEV), tk).cpu().numpy()
    ref = np.sort(O.topk_reference(scores, tk), axis=-1)      # ascending ids
    assert np.array_equal(got, ref)


def test_topk_agrees_with_torch_topk_on_untied_rows():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(5)
    scores = torch.randn(2, 4, 50, 160, generator=g)
    got = M.topk(scores.to(DEV), 20).cpu()
    ref = scores.topk(20, dim=-1).indices.sort(dim=-1).values.to(torch.int32)
    assert torch.equal(got, ref)


# ---------------------------------------------------------------------------
# Coarse branch + routing (common.py:137-167)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_coarse_forward_matches_oracle_and_routes_by_its_own_scores(dtype):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(7)
    b, h, be, nb, d = 1, 3, 64, 40, 128
    q, k, v = (_randn((b, h, nb * be, d), g, dtype) for _ in range(3))
    vbs = torch.full((nb,), be)
    vbs[-1] = 17
    scale = d ** -0.5
    qc, kc, vc = (O.block_mean(x, vbs, be) for x in (q, k, v))
    scores, probs, outc, sel = M.coarse_forward(*_gpu(qc, kc, vc), 8, scale)
    exp_scores, exp_out = O.coarse_branch_compact(q, k, v, vbs, vbs, be, scale)
    s_gpu = scores.cpu()
    if dtype == torch.float32:
        torch.testing.assert_close(s_gpu, exp_scores, atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(outc.cpu(), exp_out, atol=1e-5, rtol=1e-5)
    else:
        # dtype-faithful scores: identical bf16 values except rare accumulation-order flips
        e = exp_scores.float()
        mism = (s_gpu != e)
        assert mism.float().mean() < 0.01
        ulp = torch.finfo(dtype).eps * e.abs()
        assert ((s_gpu - e).abs() <= 2 * ulp + 1e-30).all()
        assert_parity(outc, exp_out, what="out_c")
    # the route is exactly the Top-K rule applied to the kernel's own scores
    ref = np.sort(O.topk_reference(s_gpu, 8), axis=-1)
    assert np.array_equal(sel.cpu().numpy(), ref)


# ---------------------------------------------------------------------------
# CSR inverse routing (tests/test_triton_vsa.py:163-196)
# ---------------------------------------------------------------------------

def _zipf_routes(h, qb, kb, tk, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, kb + 1) ** 1.2
    p /= p.sum()
    perm = rng.permutation(kb)
    sel = np.stack([np.stack([perm[rng.choice(kb, tk, replace=False, p=p)] for _ in range(qb)])
                    for _ in range(h)])
    return torch.from_numpy(sel[None].astype(np.int32))


@pytest.mark.parametrize("case", ["random", "zipf", "hot", "duplicates"])
def test_csr_bit_exact(case):
    from vsa_mi355x import mi355x as M
    if case == "random":
        kb = 13
        sel = torch.randn(2, 3, 7, kb, generator=torch.Generator().manual_seed(17)).topk(
            5, dim=-1, sorted=False).indices.to(torch.int32)
    elif case == "zipf":
        kb = 640
        sel = _zipf_routes(2, 640, kb, 32, 3)
    elif case == "hot":
        kb = 9
        sel = torch.zeros(1, 2, 300, 1, dtype=torch.int32)
    else:
        kb = 6
        sel = torch.randint(0, kb, (1, 2, 50, 4), generator=torch.Generator().manual_seed(2),
                            dtype=torch.int32)
    inv, off, cnt = M.invert_routes(sel.to(DEV), kb)
    ri, ro, rc = O.csr_reference(sel, kb)
    assert np.array_equal(cnt.cpu().numpy(), rc)
    assert np.array_equal(off.cpu().numpy(), ro)
    assert np.array_equal(inv.cpu().numpy(), ri)


def test_csr_ignores_out_of_range_ids():
    from vsa_mi355x import mi355x as M
    sel = torch.tensor([[[[0, 5], [-1, 1], [2, 9]]]], dtype=torch.int32)
    inv, off, cnt = M.invert_routes(sel.to(DEV), 3)
    assert cnt.cpu().tolist() == [[[1, 1, 1]]]
    assert off.cpu().tolist() == [[[0, 1, 2]]]
    assert inv.cpu()[0, 0, :3].tolist() == [0, 1, 2]


# ---------------------------------------------------------------------------
# Explicit-route fine forward / backward
# ---------------------------------------------------------------------------

def _route(h, qb, kb, tk, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, h, qb, kb, generator=g).topk(tk, dim=-1).indices.to(torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("be,d,vbs,tk", [
    (64, 128, [64, 41, 64, 19], 2),
    (64, 64, [64, 64, 33, 64, 1, 64], 3),
    (256, 128, [256, 191, 73], 2),
    (128, 64, [128, 100, 128], 2),
])
def test_sparse_attention_fwd_bwd_matches_oracle(dtype, be, d, vbs, tk):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(31)
    h, nb = 2, len(vbs)
    q, k, v, do = (_randn((1, h, nb * be, d), g, dtype) for _ in range(4))
    vbs_t = torch.tensor(vbs)
    sel = _route(h, nb, nb, tk, 3)
    scale = d ** -0.5
    qg, kg, vg = (x.to(DEV).requires_grad_() for x in (q, k, v))
    out = M.mi355x_sparse_attention(qg, kg, vg, sel.to(DEV), vbs_t.to(DEV), block_size=(1, 1, be))
    out.backward(do.to(DEV))
    qr, kr, vr = (x.clone().requires_grad_() for x in (q, k, v))
    ref = O.sparse_attention(qr, kr, vr, sel, vbs_t, block_size=(1, 1, be))
    ref.backward(do)
    assert_parity(out, ref, what="out")
    assert_parity(qg.grad, qr.grad, what="dq")
    assert_parity(kg.grad, kr.grad, what="dk")
    assert_parity(vg.grad, vr.grad, what="dv")


def test_sparse_forward_lse_matches_oracle():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(41)
    be, d, h = 256, 128, 2
    vbs = torch.tensor([256, 200, 256, 7])
    q, k, v = (_randn((1, h, 4 * be, d), g, torch.bfloat16) for _ in range(3))
    sel = _route(h, 4, 4, 3, 9)
    out, lse, _ = M.sparse_forward(*_gpu(q, k, v, sel, vbs.to(torch.int32)), be, d ** -0.5)
    ref_out, ref_lse = O.sparse_attention_reference(q, k, v, sel, vbs, be, d ** -0.5)
    assert_parity(out, ref_out, what="out")
    torch.testing.assert_close(lse.cpu(), ref_lse.float(), atol=2e-3, rtol=1e-4)


def test_hot_kv_every_query_block_routes_to_block_zero():
    # tests/test_helion_vsa.py:332-403: KV ownership under maximal in-degree
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(51)
    be, nb, h, d = 256, 3, 2, 128
    q, k, v, do = (_randn((1, h, be * nb, d), g, torch.bfloat16) for _ in range(4))
    sel = torch.zeros(1, h, nb, 1, dtype=torch.int32)
    vbs = torch.tensor([256, 173, 91])
    qg, kg, vg = (x.to(DEV).requires_grad_() for x in (q, k, v))
    out = M.mi355x_sparse_attention(qg, kg, vg, sel.to(DEV), vbs.to(DEV), block_size=(1, 1, be))
    out.backward(do.to(DEV))
    qr, kr, vr = (x.clone().requires_grad_() for x in (q, k, v))
    key, val = kr[:, :, :be].float(), vr[:, :, :be].float()
    blocks = [torch.softmax(qr[:, :, i * be:(i + 1) * be].float() @ key.transpose(-2, -1) * d ** -0.5,
                            dim=-1) @ val for i in range(nb)]
    ref = torch.cat(blocks, dim=-2)
    ref.backward(do.float())
    assert_parity(out, ref, what="out")
    for a, e, n in ((qg, qr, "dq"), (kg, kr, "dk"), (vg, vr, "dv")):
        assert_parity(a.grad, e.grad, what=n)


def test_negative_and_custom_scale():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(43)
    be, d, h = 64, 64, 1
    vbs = torch.tensor([64, 50, 64])
    q, k, v = (_randn((1, h, 3 * be, d), g, torch.bfloat16) for _ in range(3))
    sel = _route(h, 3, 3, 2, 4)
    for scale in (-0.2, 0.31):
        out = M.mi355x_sparse_attention(*_gpu(q, k, v, sel, vbs), block_size=(1, 1, be),
                                        sm_scale=scale)
        ref = O.sparse_attention(q, k, v, sel, vbs, block_size=(1, 1, be), sm_scale=scale)
        assert_parity(out, ref, what=f"scale {scale}")


def test_sparse_executor_protocol():
    """An orchestrator in the shape of _vsa_with_sparse_executor
    (triton_impl.py:1655-1731) driving the executor callable: coarse route,
    then execute(q, k, v, selected, vbs, sm_scale=scale) for the fine branch;
    the fine branch equals mi355x_sparse_attention on the same route, bitwise,
    in value and gradient, and matches the oracle."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(44)
    be, d, h, nb, tk = 256, 128, 2, 5, 2
    vbs = torch.tensor([256, 256, 200, 256, 256])
    q, k, v, do = (_randn((1, h, nb * be, d), g, torch.bfloat16) for _ in range(4))
    qg, kg, vg, vbs_g, dog = _gpu(q, k, v, vbs, do)
    _, sel = M.mi355x_route(qg, kg, vg, vbs_g, vbs_g, tk, (4, 8, 8))
    execute = M.mi355x_sparse_executor((4, 8, 8))
    scale = 1.0 / math.sqrt(d)
    outs = []
    for run in (lambda a, b, c: execute(a, b, c, sel, vbs_g, sm_scale=scale),
                lambda a, b, c: M.mi355x_sparse_attention(a, b, c, sel, vbs_g,
                                                          block_size=(4, 8, 8), sm_scale=scale)):
        leaves = [t.clone().requires_grad_() for t in (qg, kg, vg)]
        out = run(*leaves)
        outs.append((out.detach(), torch.autograd.grad(out, leaves, dog)))
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)
    ref = O.sparse_attention(q, k, v, sel.cpu(), vbs, block_size=(4, 8, 8), sm_scale=scale)
    assert_parity(outs[0][0], ref, what="executor out")


# ---------------------------------------------------------------------------
# Full VSA vs torch_vsa (tests/test_triton_vsa.py:199-398)
# ---------------------------------------------------------------------------

def _full_vsa_case(dtype, be, d, h, vbs, tk, gate_kind, seed):
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(seed)
    nb = len(vbs)
    shape = (1, h, nb * be, d)
    q, k, v, do = (_randn(shape, g, dtype) for _ in range(4))
    gate = None
    if gate_kind == "full":
        gate = torch.rand(shape, generator=g).to(dtype)
    elif gate_kind == "token":
        gate = torch.rand((1, h, nb * be, 1), generator=g).to(dtype)
    vbs_t = torch.tensor(vbs)
    qg, kg, vg = (x.to(DEV).requires_grad_() for x in (q, k, v))
    gg = gate.to(DEV).requires_grad_() if gate is not None else None
    out = M.mi355x_vsa(qg, kg, vg, vbs_t.to(DEV), vbs_t.to(DEV), tk, (1, 1, be), gg)
    out.backward(do.to(DEV))
    _, sel = M.mi355x_route(qg.detach(), kg.detach(), vg.detach(), vbs_t.to(DEV), vbs_t.to(DEV),
                            tk, (1, 1, be))
    # routing parity: the GPU route is the Top-K rule on the oracle's scores,
    # up to exact ties / one-ulp score differences (checked on the scores)
    qr, kr, vr = (x.clone().requires_grad_() for x in (q, k, v))
    gr = gate.clone().requires_grad_() if gate is not None else None
    ref = O.torch_vsa(qr, kr, vr, vbs_t, vbs_t, tk, (1, 1, be), gr, selected=sel.cpu().long())
    ref.backward(do)
    assert_parity(out, ref, what="out")
    for a, e, n in ((qg, qr, "dq"), (kg, kr, "dk"), (vg, vr, "dv")):
        assert_parity(a.grad, e.grad, what=n)
    if gate is not None:
        assert_parity(gg.grad, gr.grad, what="dgate")
    return sel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_full_vsa_padding_and_gate_be64(dtype):
    _full_vsa_case(dtype, 64, 128, 2, [64, 41, 64, 19], 2, "full", 31)


@pytest.mark.parametrize("be,d", [(256, 128), (64, 64)])
def test_full_vsa_unselected_key_blocks_get_compression_gradient(be, d):
    # tests/test_torch_vsa.py:89-109 on the GPU: with topk 1 most key blocks
    # have no CSR in-edge, so their dK/dV tiles run no item and carry only the
    # pooled (compression-branch) gradient, folded in the dK/dV epilogue
    vbs = [be] * 9
    vbs[4] = be - 29          # a ragged block: the pooled division is not by a power of two
    sel = _full_vsa_case(torch.bfloat16, be, d, 2, vbs, 1, None, 41)
    unselected = [len(vbs) - len(set(sel[0, h].flatten().tolist())) for h in range(sel.shape[1])]
    assert all(n > 0 for n in unselected), f"the case must leave key blocks unselected: {unselected}"


def test_full_vsa_be256_padded_no_gate():
    _full_vsa_case(torch.bfloat16, 256, 128, 1, [256, 173], 2, None, 35)


def test_full_vsa_be256_per_token_gate():
    _full_vsa_case(torch.bfloat16, 256, 128, 2, [256, 256, 256, 200], 2, "token", 37)


def test_full_vsa_be64_d64_many_blocks():
    _full_vsa_case(torch.bfloat16, 64, 64, 2, [64] * 15 + [30], 4, "full", 39)


def test_full_vsa_route_matches_oracle_topk_on_identical_scores():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(45)
    be, nb, d, h, tk = 64, 24, 128, 3, 5
    q, k, v = (_randn((1, h, nb * be, d), g, torch.bfloat16) for _ in range(3))
    vbs = torch.full((nb,), be)
    scores, sel = M.mi355x_route(*_gpu(q, k, v), vbs.to(DEV), vbs.to(DEV), tk, (1, 1, be))
    s = scores.cpu()
    assert np.array_equal(sel.cpu().numpy(), np.sort(O.topk_reference(s, tk), axis=-1))
    # and on rows with no tie at the boundary it equals torch.topk of those scores
    exp_scores, _ = O.coarse_branch_compact(q, k, v, vbs, vbs, be, d ** -0.5)
    ref = s.topk(tk, dim=-1)
    kth = ref.values[..., -1:]
    untied = ((s == kth).sum(-1) == 1)
    same = (ref.indices.sort(-1).values.to(torch.int32) == sel.cpu()).all(-1)
    assert same[untied].all()
    assert (s.to(exp_scores.dtype) == exp_scores).float().mean() > 0.99


def test_full_vsa_is_deterministic():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(47)
    be, nb, d, h = 256, 6, 128, 2
    q, k, v, do = (_randn((1, h, nb * be, d), g, torch.bfloat16) for _ in range(4))
    vbs = torch.full((nb,), be)
    res = []
    for _ in range(2):
        qg, kg, vg = (x.to(DEV).requires_grad_() for x in (q, k, v))
        out = M.mi355x_vsa(qg, kg, vg, vbs.to(DEV), vbs.to(DEV), 2, (4, 8, 8))
        out.backward(do.to(DEV))
        res.append([t.detach().cpu() for t in (out, qg.grad, kg.grad, vg.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_no_grad_forward_equals_grad_forward():
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(49)
    be, nb, d, h = 64, 5, 128, 2
    q, k, v = (_randn((1, h, nb * be, d), g, torch.bfloat16).to(DEV) for _ in range(3))
    vbs = torch.tensor([64, 64, 10, 64, 64]).to(DEV)
    gate = torch.rand(1, h, nb * be, d, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        a = M.mi355x_vsa(q, k, v, vbs, vbs, 2, (1, 1, be), gate)
    b = M.mi355x_vsa(q.requires_grad_(), k, v, vbs, vbs, 2, (1, 1, be), gate)
    assert torch.equal(a, b.detach())


def test_registry_loader_full_op_parity(tmp_path, monkeypatch):
    """The full op called the way the reference's users call a backend: through
    a lazy loader in a ``vsa`` package (vsa/__init__.py:28-33), here a stand-in
    written with the loaders the integration notes give."""
    import importlib
    import sys
    from test_registry import _stub_package
    monkeypatch.syspath_prepend(str(_stub_package(tmp_path)))
    for name in [m for m in sys.modules if m == "vsa" or m.startswith("vsa.")]:
        monkeypatch.delitem(sys.modules, name)
    vsa = importlib.import_module("vsa")
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(65)
    be, nb, h, d, tk = 256, 6, 2, 128, 3
    shape = (1, h, nb * be, d)
    q, k, v, do = (_randn(shape, g, torch.bfloat16) for _ in range(4))
    gate = torch.rand(shape, generator=g).to(torch.bfloat16)
    vbs = torch.tensor([256, 256, 190, 256, 256, 256])
    qg, kg, vg, gg = (x.to(DEV).requires_grad_() for x in (q, k, v, gate))
    out = vsa.mi355x_vsa(qg, kg, vg, vbs.to(DEV), vbs.to(DEV), tk, (4, 8, 8),
                         compress_attn_weight=gg)
    out.backward(do.to(DEV))
    _, sel = M.mi355x_route(qg.detach(), kg.detach(), vg.detach(), vbs.to(DEV), vbs.to(DEV), tk,
                            (4, 8, 8))
    qr, kr, vr, gr = (x.clone().requires_grad_() for x in (q, k, v, gate))
    ref = O.torch_vsa(qr, kr, vr, vbs, vbs, tk, (4, 8, 8), gr, selected=sel.cpu().long())
    ref.backward(do)
    assert_parity(out, ref, what="out")
    for a, e, n in ((qg, qr, "dq"), (kg, kr, "dk"), (vg, vr, "dv"), (gg, gr, "dgate")):
        assert_parity(a.grad, e.grad, what=n)
    # and the explicit-route loader against the oracle on the same route
    so = vsa.mi355x_sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), sel, vbs.to(DEV),
                                     block_size=(4, 8, 8))
    assert_parity(so, O.sparse_attention(q, k, v, sel.cpu(), vbs, block_size=(4, 8, 8)),
                  what="explicit-route out")


def test_route_agrees_with_the_oracles_own_topk_end_to_end():
    """End-to-end routing without the route override: the GPU's Top-K against
    torch.topk of the oracle's own bf16 scores (torch_impl.py:85), at the
    north-star block statistics (be 256, 160 key blocks, topk 20).  Rows whose
    scores match bit for bit and whose 20th and 21st scores are not tied must
    select the same set; tied rows may differ only in the tie order (the GPU
    takes the smaller block id, torch.topk's order is implementation-defined)."""
    from vsa_mi355x import mi355x as M
    g = torch.Generator().manual_seed(67)
    be, nb, h, d, tk = 256, 160, 2, 128, 20
    q, k, v = (_randn((1, h, nb * be, d), g, torch.bfloat16) for _ in range(3))
    vbs = torch.full((nb,), be)
    scores, sel = M.mi355x_route(*_gpu(q, k, v), vbs.to(DEV), vbs.to(DEV), tk, (4, 8, 8))
    o_scores, _ = O.coarse_branch_compact(q, k, v, vbs, vbs, be, d ** -0.5)
    o_sel = o_scores.topk(tk, dim=-1).indices.sort(-1).values
    srt = o_scores.sort(dim=-1, descending=True).values
    tied = srt[..., tk - 1] == srt[..., tk]
    same_scores = (scores.cpu() == o_scores.float()).all(-1)
    agree = (sel.cpu().long() == o_sel).all(-1)
    print(f"route agreement: all rows {agree.float().mean():.4f}, untied rows "
          f"{agree[~tied].float().mean():.4f}; tied rows {tied.float().mean():.4f}; rows with "
          f"bit-identical scores {same_scores.float().mean():.4f}", flush=True)
    assert agree[~tied & same_scores].all()
    assert same_scores.float().mean() > 0.95
    # on tied rows the selected sets share every block above the tied value
    for i in torch.nonzero(tied & same_scores & ~agree).tolist():
        row = o_scores[tuple(i)].float()
        kth = srt[tuple(i)][tk - 1].float()
        above = set(torch.nonzero(row > kth).flatten().tolist())
        assert above <= set(sel.cpu()[tuple(i)].tolist())
        assert all(row[j] >= kth for j in sel.cpu()[tuple(i)].tolist())
