"""GPU parity of the tiling row: vsa.tiling against oracle/tiling_oracle.py.

Everything here is integer / byte movement, so the bar is bit-exact."""

import math

import pytest
import torch

from oracle import tiling_oracle as TO
from oracle import vsa_oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [((2, 6, 6), (2, 3, 3)), ((3, 5, 5), (2, 4, 4)), ((5, 7, 9), (4, 4, 4)),
          ((1, 1, 1), (4, 4, 4)), ((4, 8, 8), (4, 8, 8)), ((6, 3, 10), (4, 2, 3)),
          ((21, 30, 52), (4, 4, 4))]


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from vsa_mi355x import _lib
    _lib.load()
    yield


def _meta(shape, ts, device="cuda"):
    from vsa_mi355x import tiling
    return tiling.build_vsa_metadata(shape, ts, device=device)


@pytest.mark.parametrize("shape,ts", SHAPES)
@pytest.mark.parametrize("device", ["cuda", "cpu"])
def test_metadata_bit_exact(shape, ts, device):
    got = _meta(shape, ts, device)
    ref = TO.build_vsa_metadata(shape, ts)
    assert got["num_tiles"] == ref["num_tiles"]
    assert got["max_block_size"] == ref["max_block_size"]
    for key in ("tile_partition_indices", "reverse_tile_partition_indices",
                "variable_block_sizes", "non_pad_index"):
        assert got[key].device.type == device
        assert got[key].dtype == torch.int64
        assert torch.equal(got[key].cpu(), ref[key]), key


@pytest.mark.parametrize("shape,ts", SHAPES[:4] + SHAPES[5:])
@pytest.mark.parametrize("trail,dtype", [((), torch.float32), ((3,), torch.bfloat16),
                                         ((2, 5), torch.float16), ((4, 64), torch.bfloat16),
                                         ((7,), torch.int32)])
def test_tile_untile_bit_exact(shape, ts, trail, dtype):
    from vsa_mi355x import tiling
    meta = _meta(shape, ts)
    ref = TO.build_vsa_metadata(shape, ts)
    S = math.prod(shape)
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    g = torch.Generator(device="cuda").manual_seed(7)
    if dtype == torch.int32:
        x = torch.randint(-1000, 1000, (3, S, *trail), generator=g, device="cuda", dtype=dtype)
    else:
        x = torch.randn(3, S, *trail, generator=g, device="cuda").to(dtype)
    t = tiling.tile(x, meta["tile_partition_indices"], meta["non_pad_index"], nb, be)
    tr = TO.tile(x.cpu(), ref["tile_partition_indices"], ref["non_pad_index"], nb, be)
    assert t.shape == tr.shape and t.dtype == x.dtype
    assert torch.equal(t.cpu(), tr)
    u = tiling.untile(t, meta["non_pad_index"], meta["reverse_tile_partition_indices"])
    assert torch.equal(u, x)
    # untile of an arbitrary padded tensor (padding rows non-zero) ignores the padding
    y = torch.randn(2, nb * be, *trail, generator=g, device="cuda").to(dtype) if dtype != torch.int32 \
        else torch.randint(-9, 9, (2, nb * be, *trail), generator=g, device="cuda", dtype=dtype)
    uy = tiling.untile(y, meta["non_pad_index"], meta["reverse_tile_partition_indices"])
    assert torch.equal(uy.cpu(), TO.untile(y.cpu(), ref["non_pad_index"],
                                           ref["reverse_tile_partition_indices"]))


def test_reference_kats_on_gpu():
    from vsa_mi355x import tiling
    # tests/test_common.py:194-209
    meta = _meta((2, 6, 6), (2, 3, 3))
    seq = 2 * 6 * 6
    x = torch.arange(seq, dtype=torch.float32, device="cuda").reshape(1, seq, 1)
    tiled = tiling.tile(x, meta["tile_partition_indices"], meta["non_pad_index"],
                        num_blocks=math.prod(meta["num_tiles"]),
                        max_block_size=meta["max_block_size"])
    assert torch.equal(tiling.untile(tiled, meta["non_pad_index"],
                                     meta["reverse_tile_partition_indices"]), x)
    # tests/test_common.py:212-218
    meta = _meta((3, 5, 5), (2, 4, 4))
    assert int(meta["variable_block_sizes"].sum()) == 75
    assert meta["non_pad_index"].numel() == 75


@pytest.mark.parametrize("shape,ts", [((3, 5, 5), (2, 4, 4)), ((5, 7, 9), (4, 4, 4))])
def test_gradients_match_oracle_autograd(shape, ts):
    from vsa_mi355x import tiling
    meta = _meta(shape, ts)
    ref = TO.build_vsa_metadata(shape, ts)
    S = math.prod(shape)
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    x = torch.randn(2, S, 3, device="cuda", dtype=torch.float64, requires_grad=True)
    gt = torch.randn(2, nb * be, 3, device="cuda", dtype=torch.float64)
    (dx,) = torch.autograd.grad(
        tiling.tile(x, meta["tile_partition_indices"], meta["non_pad_index"], nb, be), x, gt)
    xr = x.detach().cpu().requires_grad_()
    (dxr,) = torch.autograd.grad(
        TO.tile(xr, ref["tile_partition_indices"], ref["non_pad_index"], nb, be), xr, gt.cpu())
    assert torch.equal(dx.cpu(), dxr)
    y = torch.randn(2, nb * be, 3, device="cuda", dtype=torch.float64, requires_grad=True)
    gu = torch.randn(2, S, 3, device="cuda", dtype=torch.float64)
    (dy,) = torch.autograd.grad(
        tiling.untile(y, meta["non_pad_index"], meta["reverse_tile_partition_indices"]), y, gu)
    yr = y.detach().cpu().requires_grad_()
    (dyr,) = torch.autograd.grad(
        TO.untile(yr, ref["non_pad_index"], ref["reverse_tile_partition_indices"]), yr, gu.cpu())
    assert torch.equal(dy.cpu(), dyr)


def test_full_size_c3_latent():
    # a 20 x 32 x 64 latent (40,960 tokens) in (4, 8, 8) tiles: the c3 sequence
    from vsa_mi355x import tiling
    shape, ts = (20, 32, 64), (4, 8, 8)
    meta = _meta(shape, ts)
    ref = TO.build_vsa_metadata(shape, ts)
    for key in ("tile_partition_indices", "reverse_tile_partition_indices",
                "variable_block_sizes", "non_pad_index"):
        assert torch.equal(meta[key].cpu(), ref[key]), key
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(1, 40960, 40, 128, generator=g, device="cuda", dtype=torch.bfloat16)
    t = tiling.tile(x, meta["tile_partition_indices"], meta["non_pad_index"], nb, be)
    assert torch.equal(t.cpu(), TO.tile(x.cpu(), ref["tile_partition_indices"],
                                        ref["non_pad_index"], nb, be))
    assert torch.equal(tiling.untile(t, meta["non_pad_index"],
                                     meta["reverse_tile_partition_indices"]), x)


def test_tile_vsa_untile_chain_matches_oracle():
    # DiT usage: raster [B, S, H, D] -> tile -> [B, H, S_pad, D] -> mi355x_vsa -> untile
    from vsa_mi355x import tiling
    from vsa_mi355x import mi355x as M
    shape, ts = (3, 10, 12), (2, 4, 8)       # partial tiles in every direction, be = 64
    meta = _meta(shape, ts)
    ref = TO.build_vsa_metadata(shape, ts)
    nb, be = math.prod(meta["num_tiles"]), meta["max_block_size"]
    S, H, D, topk = math.prod(shape), 2, 64, 3
    g = torch.Generator(device="cuda").manual_seed(11)
    q, k, v = (torch.randn(1, S, H, D, generator=g, device="cuda", dtype=torch.bfloat16)
               for _ in range(3))

    def to_bhsd(x):
        return tiling.tile(x, meta["tile_partition_indices"], meta["non_pad_index"], nb,
                           be).transpose(1, 2).contiguous()

    vbs = meta["variable_block_sizes"].to(torch.int32)
    out = M.mi355x_vsa(to_bhsd(q), to_bhsd(k), to_bhsd(v), vbs, vbs, topk, ts)
    res = tiling.untile(out.transpose(1, 2).contiguous(), meta["non_pad_index"],
                        meta["reverse_tile_partition_indices"])
    scores, sel = M.mi355x_route(to_bhsd(q), to_bhsd(k), to_bhsd(v), vbs, vbs, topk, ts)

    def to_bhsd_ref(x):
        return TO.tile(x.cpu(), ref["tile_partition_indices"], ref["non_pad_index"], nb,
                       be).transpose(1, 2).contiguous()

    vr = ref["variable_block_sizes"]
    oref = O.torch_vsa(to_bhsd_ref(q), to_bhsd_ref(k), to_bhsd_ref(v), vr, vr, topk, ts,
                       selected=sel.cpu().long())
    rref = TO.untile(oref.transpose(1, 2).contiguous(), ref["non_pad_index"],
                     ref["reverse_tile_partition_indices"])
    diff = (res.float().cpu() - rref.float()).abs().max().item()
    assert diff <= 2e-2, diff
