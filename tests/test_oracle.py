"""Pins the CPU oracle against the reference's own known answers and against
independent mathematics (SDPA, brute force, finite differences), so a plausible
slip in the oracle (dropped mask, wrong divisor, transposed operand, wrong
tie rule) fails a test here.  Mirrors tests/test_common.py and
tests/test_torch_vsa.py of the reference."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import vsa_oracle as O


def _full(nb, be):
    return torch.full((nb,), be, dtype=torch.long)


# --- block bookkeeping / block mean (common.py:39-82) ----------------------

def test_block_elements_int_is_cube_and_tuple_is_product():
    assert O.as_block_elements(2) == 8
    assert O.as_block_elements((4, 8, 8)) == 256
    assert O.as_block_elements((1, 1, 64)) == 64


def test_block_mean_ignores_padding_values_kat():
    # tests/test_common.py:81-88: padding 999 must not leak -> [2.0, 2.0]
    x = torch.zeros(1, 1, 4, 2)
    x[0, 0, 0] = torch.tensor([1.0, 3.0])
    x[0, 0, 1] = torch.tensor([3.0, 1.0])
    x[0, 0, 2:] = 999.0
    out = O.block_mean(x, torch.tensor([2]), block_elements=4)
    torch.testing.assert_close(out, torch.tensor([[[[2.0, 2.0]]]]))


def test_block_mean_matches_explicit_masked_mean():
    # tests/test_common.py:63-78
    torch.manual_seed(0)
    x = torch.randn(2, 3, 12, 8)
    out = O.block_mean(x, torch.tensor([4, 2, 4]), block_elements=4)
    blocks = x.reshape(2, 3, 3, 4, 8)
    expected = torch.stack([blocks[:, :, 0].mean(2), blocks[:, :, 1, :2].mean(2),
                            blocks[:, :, 2].mean(2)], dim=2)
    torch.testing.assert_close(out, expected)


def test_block_mean_zero_valid_block_is_zero_not_nan():
    x = torch.randn(1, 1, 8, 4)
    out = O.block_mean(x, torch.tensor([4, 0]), block_elements=4)
    assert torch.equal(out[0, 0, 1], torch.zeros(4))


def test_valid_token_mask_brute_force():
    vbs = torch.tensor([3, 0, 5, 1])
    m = O.valid_token_mask(vbs, 5)
    for n in range(4):
        for t in range(5):
            assert bool(m[n, t]) == (t < int(vbs[n]))


# --- validation error texts (tests/test_torch_vsa.py:112-130) --------------

def test_rejects_non_divisible_sequence_length():
    q = torch.randn(1, 1, 10, 8)
    with pytest.raises(ValueError, match="divisible"):
        O.torch_vsa(q, q, q, _full(2, 4), _full(2, 4), topk=1, block_size=(1, 1, 4))


def test_rejects_wrong_block_sizes_length():
    q = torch.randn(1, 1, 12, 8)
    with pytest.raises(ValueError, match="variable_block_sizes"):
        O.torch_vsa(q, q, q, _full(2, 4), _full(2, 4), topk=1, block_size=(1, 1, 4))


def test_rejects_topk_out_of_range():
    q = torch.randn(1, 1, 12, 8)
    with pytest.raises(ValueError, match="topk"):
        O.torch_vsa(q, q, q, _full(3, 4), _full(3, 4), topk=4, block_size=(1, 1, 4))


# --- coarse branch (common.py:137-197) -------------------------------------

def test_coarse_branch_fp32_is_sdpa_on_pooled_tokens():
    torch.manual_seed(7)
    be, nb, d = 4, 5, 8
    q = torch.randn(1, 2, be * nb, d, dtype=torch.float64)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    vbs = torch.tensor([4, 3, 2, 4, 1])
    scale = d ** -0.5
    scores, out_c = O.coarse_branch_compact(q, k, v, vbs, vbs, be, scale)
    qc, kc, vc = (O.block_mean(t, vbs, be) for t in (q, k, v))
    torch.testing.assert_close(out_c, F.scaled_dot_product_attention(qc, kc, vc))
    # scores are the scaled dot products, row by row
    for i in range(nb):
        for j in range(nb):
            torch.testing.assert_close(scores[0, 1, i, j], (qc[0, 1, i] * kc[0, 1, j]).sum() * scale)


def test_compact_coarse_matches_expanded_branch():
    torch.manual_seed(7)
    be, nb, d = 4, 3, 8
    q = torch.randn(1, 2, be * nb, d)
    k, v = torch.randn_like(q), torch.randn_like(q)
    vbs = torch.tensor([4, 3, 2])
    s1, ex = O.coarse_branch(q, k, v, vbs, vbs, be, d ** -0.5)
    s2, cp = O.coarse_branch_compact(q, k, v, vbs, vbs, be, d ** -0.5)
    torch.testing.assert_close(s1, s2)
    torch.testing.assert_close(cp[:, :, :, None].expand(-1, -1, -1, be, -1).reshape_as(ex), ex)


# --- Top-K rule ------------------------------------------------------------

def test_topk_reference_brute_force_and_tie_rule():
    rng = np.random.default_rng(0)
    s = rng.integers(-3, 4, size=(50, 11)).astype(np.float32)   # many ties
    got = O.topk_reference(s, 4)
    for r in range(50):
        pairs = sorted(((-s[r, j], j) for j in range(11)))
        assert got[r].tolist() == [j for _, j in pairs[:4]]


def test_topk_reference_matches_torch_topk_without_ties():
    torch.manual_seed(3)
    s = torch.randn(2, 3, 17, 40)
    got = torch.from_numpy(O.topk_reference(s, 7)).long()
    ref = s.topk(7, dim=-1).indices            # sorted=True, no ties in randn
    assert torch.equal(got, ref)


def test_topk_mask_selects_exactly_topk_blocks():
    torch.manual_seed(4)
    q = torch.randn(1, 1, 20, 8)
    _, aux = O.video_sparse_attn(q, torch.randn_like(q), torch.randn_like(q), _full(5, 4),
                                 _full(5, 4), topk=3, block_size=(1, 1, 4), return_aux=True)
    assert aux["block_mask"].sum(-1).unique().tolist() == [3]


# --- dense masked-fill oracle (common.py:200-285) --------------------------

@pytest.mark.parametrize("be", [4, 8])
def test_selecting_all_blocks_sparse_branch_equals_sdpa(be):
    torch.manual_seed(1)
    nb = 3
    q = torch.randn(2, 2, nb * be, 16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    _, aux = O.video_sparse_attn(q, k, v, _full(nb, be), _full(nb, be), topk=nb,
                                 block_size=(1, 1, be), return_aux=True)
    torch.testing.assert_close(aux["out_sparse"], F.scaled_dot_product_attention(q, k, v),
                               atol=1e-5, rtol=1e-5)


def test_output_is_compress_plus_sparse_and_gate_scales():
    torch.manual_seed(3)
    q = torch.randn(1, 1, 12, 8)
    k, v = torch.randn_like(q), torch.randn_like(q)
    vbs = _full(3, 4)
    base, aux = O.video_sparse_attn(q, k, v, vbs, vbs, topk=2, block_size=(1, 1, 4), return_aux=True)
    torch.testing.assert_close(base, aux["out_compress"] + aux["out_sparse"])
    zero = O.video_sparse_attn(q, k, v, vbs, vbs, topk=2, block_size=(1, 1, 4),
                               compress_attn_weight=torch.zeros_like(q))
    torch.testing.assert_close(zero, aux["out_sparse"])
    two = O.video_sparse_attn(q, k, v, vbs, vbs, topk=2, block_size=(1, 1, 4),
                              compress_attn_weight=torch.full_like(q, 2.0))
    torch.testing.assert_close(two, 2.0 * aux["out_compress"] + aux["out_sparse"])


# --- gather oracle == masked-fill oracle (tests/test_torch_vsa.py:12-72) ----

@pytest.mark.parametrize("case", ["full", "padded", "gate", "int_block"])
def test_torch_vsa_matches_masked_fill_reference(case):
    torch.manual_seed({"full": 1, "padded": 2, "gate": 3, "int_block": 4}[case])
    if case == "int_block":
        be, nb, d, bs = 8, 3, 8, 2
    else:
        be, nb, d, bs = 4, 4 if case != "padded" else 3, 16, (1, 1, 4)
    q = torch.randn(2 if case == "full" else 1, 2, be * nb, d)
    k, v = torch.randn_like(q), torch.randn_like(q)
    vbs = torch.tensor([4, 2, 3]) if case == "padded" else _full(nb, be)
    gate = torch.randn_like(q) if case == "gate" else None
    a = O.torch_vsa(q, k, v, vbs, vbs, topk=2, block_size=bs, compress_attn_weight=gate)
    e = O.video_sparse_attn(q, k, v, vbs, vbs, topk=2, block_size=bs, compress_attn_weight=gate)
    torch.testing.assert_close(a, e, atol=1e-5, rtol=1e-5)


def test_unselected_blocks_get_gradient_through_compression():
    # tests/test_torch_vsa.py:89-109
    torch.manual_seed(6)
    be, nb = 4, 4
    q = torch.randn(1, 1, be * nb, 8)
    k = torch.randn(1, 1, be * nb, 8, requires_grad=True)
    v = torch.randn(1, 1, be * nb, 8, requires_grad=True)
    vbs = _full(nb, be)
    scores, _ = O.coarse_branch(q, k.detach(), v.detach(), vbs, vbs, be, 8 ** -0.5)
    sel = scores.topk(1, dim=-1).indices
    unselected = sorted(set(range(nb)) - set(sel.flatten().tolist()))
    assert unselected
    O.torch_vsa(q, k, v, vbs, vbs, topk=1, block_size=(1, 1, be)).square().mean().backward()
    for blk in unselected:
        assert k.grad[0, 0, blk * be:(blk + 1) * be].abs().sum() > 0


def test_torch_vsa_gradcheck_fp64():
    torch.manual_seed(8)
    be, nb, d = 4, 3, 4
    mk = lambda: torch.randn(1, 1, be * nb, d, dtype=torch.float64, requires_grad=True)
    q, k, v, g = mk(), mk(), mk(), mk()
    vbs = torch.tensor([4, 3, 2])
    sel = torch.tensor([[[[0, 2], [1, 2], [0, 1]]]])
    f = lambda q, k, v, g: O.torch_vsa(q, k, v, vbs, vbs, 2, (1, 1, be), g, selected=sel)
    assert torch.autograd.gradcheck(f, (q, k, v, g), eps=1e-6, atol=1e-6)


def test_route_override_equals_own_topk_and_head_chunking():
    torch.manual_seed(9)
    be, nb = 4, 5
    q = torch.randn(1, 3, be * nb, 8)
    k, v = torch.randn_like(q), torch.randn_like(q)
    vbs = torch.tensor([4, 4, 3, 4, 2])
    scores, _ = O.coarse_branch(q, k, v, vbs, vbs, be, 8 ** -0.5)
    sel = scores.topk(2, dim=-1).indices
    a = O.torch_vsa(q, k, v, vbs, vbs, 2, (1, 1, be))
    b = O.torch_vsa(q, k, v, vbs, vbs, 2, (1, 1, be), selected=sel, head_chunk=2)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


# --- explicit-route executor contract --------------------------------------

def test_hot_kv_all_routes_to_block_zero_matches_dense_per_block_softmax():
    # tests/test_helion_vsa.py:332-403 (explicit dense reference per query block)
    torch.manual_seed(51)
    be, nb, heads, d = 16, 3, 2, 8
    q = torch.randn(1, heads, be * nb, d)
    k, v = torch.randn_like(q), torch.randn_like(q)
    sel = torch.zeros(1, heads, nb, 1, dtype=torch.int32)
    vbs = torch.tensor([16, 9, 5])
    out, lse = O.sparse_attention_reference(q, k, v, sel, vbs, be, d ** -0.5)
    key, val = k[:, :, :be], v[:, :, :be]
    for qb in range(nb):
        qq = q[:, :, qb * be:(qb + 1) * be]
        p = torch.softmax(qq @ key.transpose(-2, -1) * d ** -0.5, dim=-1)
        torch.testing.assert_close(out[:, :, qb * be:(qb + 1) * be], p @ val)


def test_lse2_is_log2_sum_exp2_brute_force():
    torch.manual_seed(12)
    be, nb, d = 4, 3, 4
    q = torch.randn(1, 1, be * nb, d, dtype=torch.float64)
    k, v = torch.randn_like(q), torch.randn_like(q)
    vbs = torch.tensor([4, 2, 3])
    sel = torch.tensor([[[[2, 1], [0, 2], [1, 0]]]])
    scale = 0.37
    _, lse = O.sparse_attention_reference(q, k, v, sel, vbs, be, scale)
    for i in range(be * nb):
        acc = 0.0
        for kvb in sel[0, 0, i // be].tolist():
            for t in range(int(vbs[kvb])):
                s = float((q[0, 0, i] * k[0, 0, kvb * be + t]).sum()) * scale
                acc += 2.0 ** (s * math.log2(math.e))
        assert abs(float(lse[0, 0, i]) - math.log2(acc)) < 1e-9


def test_sparse_attention_all_selected_full_blocks_is_sdpa():
    torch.manual_seed(13)
    be, nb = 8, 4
    q = torch.randn(1, 2, be * nb, 16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    sel = torch.arange(nb).view(1, 1, 1, nb).expand(1, 2, nb, nb)
    out = O.sparse_attention(q, k, v, sel, _full(nb, be), block_size=(1, 1, be))
    torch.testing.assert_close(out, F.scaled_dot_product_attention(q, k, v), atol=1e-5, rtol=1e-5)


def test_sparse_attention_gradcheck_fp64():
    torch.manual_seed(14)
    be, nb, d = 4, 3, 4
    mk = lambda: torch.randn(1, 2, be * nb, d, dtype=torch.float64, requires_grad=True)
    q, k, v = mk(), mk(), mk()
    sel = torch.tensor([[[0, 2], [1, 2], [0, 1]], [[1, 0], [2, 2], [0, 2]]]).unsqueeze(0)
    vbs = torch.tensor([4, 1, 3])
    f = lambda q, k, v: O.sparse_attention(q, k, v, sel, vbs, block_size=(1, 1, be), sm_scale=0.7)
    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-6)


# --- CSR inverse routing (tests/test_triton_vsa.py:163-196) ----------------

def test_csr_reference_matches_brute_force():
    torch.manual_seed(17)
    kb = 13
    sel = torch.randn(2, 3, 7, kb).topk(5, dim=-1, sorted=False).indices.to(torch.int32)
    inv, off, cnt = O.csr_reference(sel, kb)
    assert inv.shape == (2, 3, 7 * 5)
    assert (cnt.sum(-1) == 7 * 5).all()
    for b in range(2):
        for h in range(3):
            for kv in range(kb):
                seg = inv[b, h, off[b, h, kv]:off[b, h, kv] + cnt[b, h, kv]].tolist()
                assert seg == sel[b, h].eq(kv).nonzero()[:, 0].tolist()   # ascending


# --- planted mistakes: each must be caught by a pin above ------------------

def test_planted_mistake_wrong_divisor_is_caught(monkeypatch):
    def bad_block_mean(x, vbs, block_elements):     # divides by the padded volume
        be = block_elements
        b, h, s, d = x.shape
        blocks = x.reshape(b, h, s // be, be, d).float()
        valid = O.valid_token_mask(vbs, be).view(1, 1, s // be, be, 1)
        return ((blocks * valid).sum(3) / be).to(x.dtype)
    monkeypatch.setattr(O, "block_mean", bad_block_mean)
    with pytest.raises(AssertionError):
        test_block_mean_ignores_padding_values_kat()


def test_planted_mistake_unmasked_padding_keys_is_caught(monkeypatch):
    real = O.valid_token_mask
    monkeypatch.setattr(O, "valid_token_mask", lambda vbs, be: torch.ones_like(real(vbs, be)))
    with pytest.raises(AssertionError):
        test_lse2_is_log2_sum_exp2_brute_force()
