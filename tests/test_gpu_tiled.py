"""GPU: VSA on raster-order tokens with tile / untile fused into the op.

``mi355x_vsa_tiled`` must equal the unfused composition
``untile(mi355x_vsa(tile(q), tile(k), tile(v), vbs, vbs, topk, tile_size, tile(gate)))``
(tile / untile of fastvideo_tiling.py:130-145 along the sequence dim) bit for
bit: the output and every gradient.  The slot -> raster table it is built on
is checked against the tiling oracle's index tensors."""

import math

import pytest
import torch

from oracle import tiling_oracle as TO

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


@pytest.mark.parametrize("shape,ts", [((5, 12, 20), (4, 4, 4)), ((6, 16, 24), (4, 8, 8)),
                                      ((3, 9, 10), (2, 8, 8)), ((4, 8, 8), (4, 8, 8)),
                                      ((1, 1, 1), (4, 4, 4)), ((21, 30, 52), (4, 4, 4))])
def test_slot_rows_invert_the_tiling_indices(shape, ts):
    from vsa_mi355x import tiled
    rows = tiled.slot_rows(shape, ts, DEV).cpu().long()
    ref = TO.build_vsa_metadata(shape, ts)
    tpi, npi = ref["tile_partition_indices"], ref["non_pad_index"]
    nb, be = math.prod(ref["num_tiles"]), ref["max_block_size"]
    assert rows.numel() == nb * be
    expect = torch.full((nb * be,), -1, dtype=torch.long)
    expect[npi] = tpi
    assert torch.equal(rows, expect)


def _inputs(shape, heads, d, dtype, gate, seed):
    g = torch.Generator().manual_seed(seed)
    s = math.prod(shape)
    q, k, v, do = (torch.randn(1, heads, s, d, generator=g).to(dtype) for _ in range(4))
    gt = None
    if gate == "full":
        gt = (2.0 * torch.rand(1, heads, s, d, generator=g)).to(dtype)
    elif gate == "token":
        gt = (2.0 * torch.rand(1, heads, s, 1, generator=g)).to(dtype)
    return q, k, v, do, gt


def _run(fn, q, k, v, do, gate):
    leaves = [x.to(DEV).requires_grad_() for x in (q, k, v)]
    gl = gate.to(DEV).requires_grad_() if gate is not None else None
    out = fn(*leaves, gl)
    out.backward(do.to(DEV))
    grads = [x.grad for x in leaves] + ([gl.grad] if gl is not None else [])
    return [out.detach()] + grads


CASES = [
    # shape, tile, heads, head_dim, dtype, gate, topk
    ((5, 12, 20), (4, 4, 4), 2, 64, torch.bfloat16, "full", 4),     # block 64, partial tiles
    ((6, 16, 24), (4, 8, 8), 22, 128, torch.float16, "token", 3),   # block 256, ping-pong kernels
    ((3, 9, 10), (2, 8, 8), 3, 128, torch.bfloat16, None, 2),       # block 128, no gate
    ((6, 16, 24), (4, 8, 8), 2, 64, torch.bfloat16, "full", 5),     # block 256, 4-wave kernels
    # 81 920 tokens: batch * seq_len of a token-major [B, S, H, D] tensor exceeds
    # the 65 535 batch * heads bound, which must not be mistaken for it
    ((4, 128, 160), (4, 8, 8), 2, 64, torch.bfloat16, None, 4),
]


@pytest.mark.parametrize("shape,ts,heads,d,dtype,gate,topk", CASES)
def test_fused_tiled_op_equals_the_composition_bit_for_bit(shape, ts, heads, d, dtype, gate,
                                                           topk):
    from vsa_mi355x import tiled
    q, k, v, do, gt = _inputs(shape, heads, d, dtype, gate, seed=sum(shape) + heads)
    print(f"case shape={shape} tile={ts} heads={heads} d={d} {dtype} gate={gate}", flush=True)
    fused = _run(lambda q_, k_, v_, g_: tiled.mi355x_vsa_tiled(q_, k_, v_, shape, topk, ts, g_),
                 q, k, v, do, gt)
    ref = _run(lambda q_, k_, v_, g_: tiled._composition(
        q_, k_, v_, __import__("vsa_mi355x").tiling.build_vsa_metadata(shape, ts, device=DEV),
        math.prod([math.ceil(a / b) for a, b in zip(shape, ts)]), math.prod(ts), ts, topk, g_),
        q, k, v, do, gt)
    names = ["out", "dq", "dk", "dv", "dgate"]
    for name, a, b in zip(names, fused, ref):
        assert a.shape == b.shape and a.dtype == b.dtype, name
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), (name, (a.float() - b.float()).abs().max().item())


def test_fused_tiled_no_grad_equals_grad_forward():
    from vsa_mi355x import tiled
    shape, ts = (5, 12, 20), (4, 4, 4)
    q, k, v, _, gt = _inputs(shape, 2, 128, torch.bfloat16, "full", seed=3)
    qd, kd, vd, gd = (x.to(DEV) for x in (q, k, v, gt))
    with torch.no_grad():
        a = tiled.mi355x_vsa_tiled(qd, kd, vd, shape, 4, ts, gd)
    b = tiled.mi355x_vsa_tiled(qd.requires_grad_(), kd, vd, shape, 4, ts, gd)
    assert torch.equal(a, b.detach())


def test_unfused_shapes_run_the_composition():
    """fp32 and a broadcast gate take the composition; the result is the same op."""
    from vsa_mi355x import tiled, tiling
    shape, ts = (4, 8, 8), (4, 4, 4)
    q, k, v, _, _ = _inputs(shape, 2, 64, torch.float32, None, seed=5)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    gate = torch.rand(1, 1, math.prod(shape), 1, device=DEV)
    out = tiled.mi355x_vsa_tiled(qd, kd, vd, shape, 2, ts, gate)
    meta = tiling.build_vsa_metadata(shape, ts, device=DEV)
    ref = tiled._composition(qd, kd, vd, meta, 4, 64, ts, 2, gate)
    assert torch.equal(out, ref)


def test_fused_tiled_op_at_c3_size_equals_the_composition():
    """The c3 workload as a video DiT holds it: a 20x32x64 latent in (4,8,8)
    tiles, 40 heads, head_dim 128, topk 20, full gate; output and every
    gradient bit for bit (the ping-pong forward / dQ and the persistent dK/dV
    at their real grid sizes)."""
    from vsa_mi355x import tiled, tiling
    shape, ts, H, d, tk = (20, 32, 64), (4, 8, 8), 40, 128, 20
    g = torch.Generator(device=DEV).manual_seed(91)
    s = math.prod(shape)
    q, k, v, do = (torch.randn(1, H, s, d, generator=g, device=DEV, dtype=torch.bfloat16)
                   for _ in range(4))
    gate = torch.rand(1, H, s, d, generator=g, device=DEV, dtype=torch.bfloat16)
    meta = tiling.build_vsa_metadata(shape, ts, device=DEV)
    outs = []
    for fn in (lambda *a: tiled.mi355x_vsa_tiled(*a[:3], shape, tk, ts, a[3]),
               lambda *a: tiled._composition(*a[:3], meta, 160, 256, ts, tk, a[3])):
        leaves = [x.clone().requires_grad_() for x in (q, k, v, gate)]
        out = fn(*leaves)
        grads = torch.autograd.grad(out, leaves, do)
        outs.append([out.detach()] + list(grads))
        del out, grads, leaves
    for name, a, b in zip(["out", "dq", "dk", "dv", "dgate"], *outs):
        assert torch.equal(a, b), (name, (a.float() - b.float()).abs().max().item())


@pytest.mark.parametrize("case", [0, 1, 4])
def test_token_major_tiled_op_equals_head_major_and_composition(case):
    """q, k, v, gate, dout as [B, S, H, D] (the projection's layout, tile()'s
    [batch, seq, ...]): the same values as the head-major op, transposed, and
    as tile -> op -> untile along dim 1."""
    from vsa_mi355x import tiled, tiling
    shape, ts, heads, d, dtype, gate, topk = CASES[case]
    q, k, v, do, gt = _inputs(shape, heads, d, dtype, gate, seed=77 + case)
    tm = (lambda x: None if x is None else x.transpose(1, 2).contiguous())
    head_major = _run(lambda q_, k_, v_, g_: tiled.mi355x_vsa_tiled(q_, k_, v_, shape, topk, ts, g_),
                      q, k, v, do, gt)
    token_major = _run(lambda q_, k_, v_, g_: tiled.mi355x_vsa_tiled(
        q_, k_, v_, shape, topk, ts, g_, token_major=True), tm(q), tm(k), tm(v), tm(do), tm(gt))
    meta = tiling.build_vsa_metadata(shape, ts, device=DEV)
    nb = math.prod([math.ceil(a / b) for a, b in zip(shape, ts)])
    ref = _run(lambda q_, k_, v_, g_: tiled._composition(q_, k_, v_, meta, nb, math.prod(ts), ts,
                                                         topk, g_, token_major=True),
               tm(q), tm(k), tm(v), tm(do), tm(gt))
    for name, a, b, c in zip(["out", "dq", "dk", "dv", "dgate"], head_major, token_major, ref):
        assert b.shape == c.shape, name
        assert torch.equal(b, c), (name, "token-major vs composition")
        assert torch.equal(a.transpose(1, 2), b), (name, "token-major vs head-major")
