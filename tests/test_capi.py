"""CPU-side checks of the drop-in boundary: the C-ABI library loads, exports
every entry point ``include/vsa_capi.h`` declares, reports status text, and
the Python layer raises the reference's ValueError texts before any launch
(tests/test_torch_vsa.py:112-130)."""

import ctypes
import os
import re

import pytest
import torch

from vsa_mi355x import _lib
from vsa_mi355x import mi355x as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vsa_capi.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int)\s+(vsa_\w+)\s*\(", text, re.M)))


def test_header_declares_the_expected_entry_points():
    names = _declared_symbols()
    for must in ("vsa_pool_qkv", "vsa_coarse_fwd", "vsa_topk", "vsa_csr_build", "vsa_sparse_fwd",
                 "vsa_bwd_prep", "vsa_coarse_bwd", "vsa_sparse_bwd_dq", "vsa_sparse_bwd_dkdv",
                 "vsa_dkdv_tile_order", "vsa_sparse_bwd_dkdv_noalloc",
                 "vsa_status_string", "vsa_version"):
        assert must in names


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings_and_version():
    assert _lib.status_string(0) == "ok"
    assert "NULL" in _lib.status_string(-1)
    assert "unknown" in _lib.status_string(-99)
    assert b"gfx950" in _lib.load().vsa_version()


def test_entry_points_reject_bad_arguments_without_a_gpu():
    lib = _lib.load()
    # NULL pointers and impossible sizes are rejected before any launch.
    assert lib.vsa_pool_qkv(None, None, None, None, None, None, None, None,
                            1, 64, 64, 128, 64, 0, None) == -1
    assert lib.vsa_topk(None, None, 1, 4, 2, None) == -1
    p = _lib.ptr(torch.zeros(1))
    assert lib.vsa_topk(p, p, 1, 4, 5, None) == -2          # topk > Kb
    assert lib.vsa_csr_build(p, p, p, p, 1, 4, 0, 2, None) == -2
    # tile order: the buffer must hold 8 * ceil(tiles / 8) + 16 entries
    assert lib.vsa_dkdv_tile_order(None, p, 24, 1, 1024, 128, 256, None) == -1
    assert lib.vsa_dkdv_tile_order(p, p, 23, 1, 1024, 128, 256, None) == -2   # 8 tiles
    assert lib.vsa_dkdv_tile_order(p, p, 64, 1, 1024, 128, 96, None) == -2   # 1024 % 96
    assert lib.vsa_dkdv_tile_order(p, p, 64, 1, 960, 128, 96, None) == -4    # no kernel
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, None, None, 0, 0,
                              1, 100, 128, 128, 64, 1, 0.1, 0, None) == -2   # 100 % 64
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, None, None, 0, 0,
                              1, 96, 96, 128, 96, 1, 0.1, 0, None) == -4     # be 96: no kernel
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, None, None, 0, 0,
                              1, 64, 64, 128, 64, 1, 0.1, 7, None) == -3     # no dtype 7
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, None, None, 0, 0,
                              1, 96, 96, 128, 96, 1, 0.1, 2, None) == -4     # fp32, be 96
    # token-major gate: the heads count must divide batch*heads
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, p, p, 3, 3,
                              4, 64, 64, 128, 64, 1, 0.1, 0, None) == -2
    assert lib.vsa_bwd_prep(p, p, p, p, 3, 0, p, p, p, 4, 64, 128, 64, 0, None) == -2
    # an fp32 gate beside bf16 inputs runs the fine pass, then a combine pass;
    # the combine's limit (batch * heads <= 65535) is checked before the fine
    # pass writes anything (with no GPU here a launch would fail with -5)
    f32_full = _lib.GATE_FULL | _lib.GATE_F32
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, p, None, p, p, f32_full, 0,
                              65536, 64, 64, 128, 64, 1, 0.1, 0, None) == -2
    # no-allocation dK/dV: sizes whose tile order exceeds the 1 MiB static scratch
    # (8 * ceil(tiles / 8) + 16 > 262144 int32) are rejected before any launch
    noalloc = [p] * 14
    assert lib.vsa_sparse_bwd_dkdv_noalloc(*noalloc, 64, 1024, 128 * 4096, 128, 256, 8, 0.1,
                                           0, None) == -6
    assert "static scratch" in _lib.status_string(-6)
    assert lib.vsa_sparse_bwd_dkdv_noalloc(*noalloc, 1, 1024, 1024, 128, 96, 8, 0.1,
                                           0, None) == -2              # 1024 % 96
    assert lib.vsa_sparse_bwd_dkdv_noalloc(*noalloc, 1, 1024, 1024, 128, 256, 8, 0.1,
                                           7, None) == -3              # no dtype 7
    assert lib.vsa_sparse_bwd_dkdv_noalloc(*([None] + noalloc[1:]), 1, 1024, 1024, 128, 256, 8,
                                           0.1, 0, None) == -1
    # alignment (checked before any launch, nothing is dereferenced): rows of the
    # element type 16 bytes, int32 arrays and lse / delta 4, int64 indices 8
    buf = torch.zeros(256)
    a16 = (buf.data_ptr() + 15) // 16 * 16

    def at(off):
        return ctypes.c_void_p(a16 + off)

    assert "misaligned" in _lib.status_string(-7)
    assert lib.vsa_pool_qkv(at(2), p, p, p, p, p, p, p, 1, 64, 64, 128, 64, 0, None) == -7
    assert lib.vsa_pool_qkv(p, p, p, at(2), p, p, p, p, 1, 64, 64, 128, 64, 0, None) == -7
    assert lib.vsa_sparse_fwd(p, at(8), p, p, p, p, None, None, None, None, 0, 0,
                              1, 64, 64, 128, 64, 1, 0.1, 0, None) == -7   # k at 8 bytes
    assert lib.vsa_sparse_fwd(p, p, p, p, p, p, None, None, p, at(4), 1, 0,
                              1, 64, 64, 128, 64, 1, 0.1, 0, None) == -7   # gate at 4 bytes
    # an int32 route 4 bytes past a 16-byte boundary passes; the shape check fails next
    assert lib.vsa_sparse_fwd(p, p, p, at(4), p, p, None, None, None, None, 0, 0,
                              1, 100, 128, 128, 64, 1, 0.1, 0, None) == -2
    assert lib.vsa_bwd_prep(p, p, None, None, 0, 0, at(2), None, None, 1, 64, 128, 64, 0,
                            None) == -7                                    # delta at 2 bytes
    assert lib.vsa_sparse_bwd_dkdv_noalloc(*noalloc[:10], at(16), at(24), None, None, 1, 1024,
                                           1024, 128, 256, 8, 0.1, 0, None) == -7  # dv at 8
    assert lib.vsa_csr_build(p, p, at(2), p, 1, 4, 4, 2, None) == -7
    assert lib.vsa_rows_move(p, 4, 16, p, 4, 16, 16, 1, at(4), 4, None, None, 0, None, 4,
                             None) == -7                                   # int64 at 4 bytes
    # blocks per sequence: 16000 for the route, the CSR and the MFMA coarse
    # kernels (bf16 / fp16 at head dims 64, 128), 4096 for the generic ones
    assert lib.vsa_topk(p, p, 1, 16001, 2, None) == -2
    assert lib.vsa_csr_build(p, p, p, p, 1, 4, 16001, 2, None) == -2
    assert lib.vsa_csr_build(p, p, p, p, 1, 16001, 4, 2, None) == -2
    assert lib.vsa_coarse_fwd(p, p, p, p, p, p, None, 1, 4, 16001, 128, 2, 0.1, 0, None) == -2
    assert lib.vsa_coarse_fwd(p, p, p, p, p, p, None, 1, 4, 4097, 128, 2, 0.1, 2, None) == -2
    assert lib.vsa_coarse_fwd(p, p, p, p, p, p, None, 1, 4, 4097, 256, 2, 0.1, 0, None) == -2
    assert lib.vsa_coarse_bwd(*([p] * 9), 1, 4, 4097, 96, 0.1, 1, None) == -2
    # tiling entry points validate before launching
    assert lib.vsa_tile_metadata(0, 4, 4, 2, 2, 2, p, p, p, p, None) == -2
    assert lib.vsa_tile_metadata(4, 4, 4, 2, 2, 2, None, p, p, p, None) == -1
    assert lib.vsa_rows_move(None, 4, 16, p, 4, 16, 16, 1, None, 0, None, None, 0, None, 4,
                             None) == -1
    assert lib.vsa_rows_move(p, 4, 16, p, 4, 16, 0, 1, None, 0, None, None, 0, None, 4,
                             None) == -2
    assert lib.vsa_rows_move(p, 4, 16, p, 4, 8, 16, 1, None, 0, None, None, 0, None, 4,
                             None) == -2     # copy longer than the destination row
    assert lib.vsa_rows_zero_unmarked(p, 4, 1, 16, None, 2, p, None) == -1
    # tiled-sequence entry points validate before launching
    assert lib.vsa_tile_slot_rows(0, 4, 4, 2, 2, 2, p, None) == -2
    assert lib.vsa_tile_slot_rows(4, 4, 4, 2, 2, 2, None, None) == -1
    assert lib.vsa_tile_pool_qkv(*([p] * 11 + [None]), 1, 64, 0, 1, 128, 64, 0, None) == -1
    assert lib.vsa_tile_pool_qkv(*([p] * 12), 1, 65, 0, 1, 128, 64, 0, None) == -2  # s_out > nb*be
    assert lib.vsa_tile_pool_qkv(*([p] * 12), 3, 64, 2, 1, 128, 64, 0, None) == -2  # 3 % 2 heads
    fwd = [p] * 10
    assert lib.vsa_sparse_fwd_tiled(*fwd, 1, None, 64, 0, 1, 64, 64, 128, 64, 1, 0.1, 0,
                                    None) == -1                   # no slot_rows
    assert lib.vsa_sparse_fwd_tiled(*fwd, 3, p, 64, 0, 1, 64, 64, 128, 64, 1, 0.1, 0,
                                    None) == -2                   # gate mode 3
    assert lib.vsa_sparse_fwd_tiled(*fwd, 1, p, 65, 0, 1, 64, 64, 128, 64, 1, 0.1, 0,
                                    None) == -2                   # s_out > tiled length
    assert lib.vsa_sparse_fwd_tiled(*fwd, 1, p, 64, 2, 3, 64, 64, 128, 64, 1, 0.1, 0,
                                    None) == -2                   # heads must divide bh
    assert lib.vsa_sparse_fwd_tiled(*fwd, 1, p, 64, 0, 1, 64, 64, 256, 64, 1, 0.1, 0,
                                    None) == -4                   # head_dim 256: composition
    assert lib.vsa_sparse_fwd_tiled(*fwd, 1, p, 64, 0, 1, 64, 64, 128, 64, 1, 0.1, 2,
                                    None) == -4                   # fp32: composition
    assert lib.vsa_bwd_prep_tiled(p, p, p, p, 1, p, 64, 0, p, p, p, None, 1, 64, 128, 64, 0,
                                  None) == -1                     # no dout_t
    assert lib.vsa_bwd_prep_tiled(p, p, p, p, 3, p, 64, 0, p, p, p, p, 1, 64, 128, 64, 0,
                                  None) == -2
    assert lib.vsa_sparse_bwd_dq_tiled(*([p] * 11), None, 64, 0, 1, 64, 64, 128, 64, 1, 0.1, 0,
                                       None) == -1
    assert lib.vsa_sparse_bwd_dq_tiled(*([p] * 12), 64, 0, 1, 64, 64, 128, 96, 1, 0.1, 0,
                                       None) == -2               # 64 % 96
    assert lib.vsa_sparse_bwd_dkdv_tiled(*([p] * 14), None, 64, 0, 1, 64, 64, 128, 64, 1, 0.1,
                                         None, 0, None) == -1
    assert lib.vsa_sparse_bwd_dkdv_tiled(*([p] * 15), 64, 0, 1, 64, 64, 128, 64, 1, 0.1, None,
                                         7, None) == -3          # no dtype 7


def _full(nb, be):
    return torch.full((nb,), be, dtype=torch.long)


def test_validation_texts_match_reference():
    q = torch.randn(1, 1, 10, 8)
    with pytest.raises(ValueError, match="divisible"):
        M.mi355x_vsa(q, q, q, _full(2, 4), _full(2, 4), topk=1, block_size=(1, 1, 4))
    q = torch.randn(1, 1, 12, 8)
    with pytest.raises(ValueError, match="variable_block_sizes"):
        M.mi355x_vsa(q, q, q, _full(2, 4), _full(2, 4), topk=1, block_size=(1, 1, 4))
    with pytest.raises(ValueError, match="topk"):
        M.mi355x_vsa(q, q, q, _full(3, 4), _full(3, 4), topk=4, block_size=(1, 1, 4))


def test_cpu_tensors_are_rejected_not_computed_elsewhere():
    q = torch.randn(1, 1, 128, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        M.mi355x_vsa(q, q, q, _full(2, 64), _full(2, 64), topk=1, block_size=(1, 1, 64))
    sel = torch.zeros(1, 1, 2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        M.mi355x_sparse_attention(q, q, q, sel, _full(2, 64), block_size=(1, 1, 64))
    # the executor protocol (sparse_executor(q, k, v, selected, vbs, *, sm_scale)) goes
    # through the same checks
    execute = M.mi355x_sparse_executor((1, 1, 64))
    with pytest.raises(ValueError, match="GPU"):
        execute(q, q, q, sel, _full(2, 64), sm_scale=0.125)


def test_block_volume_and_gate_shape_helpers():
    assert M.as_block_elements((4, 8, 8)) == 256
    assert M.as_block_elements(4) == 64
    q = torch.randn(1, 2, 16, 8)
    assert M._prepare_gate(torch.ones(1, 2, 16, 1), q).shape == (1, 2, 16, 1)
    with pytest.raises(ValueError, match="compress_attn_weight"):
        M._prepare_gate(torch.ones(1, 2, 16, 4), q)


def test_kernel_shape_mapping_and_limits():
    # shapes the reference's GPU path accepts map onto kernel shapes; others raise
    assert M._kernel_block(256) == 256 and M._kernel_block(64) == 64
    assert M._kernel_block(27) == 64 and M._kernel_block(100) == 128 and M._kernel_block(1) == 64
    assert M._kernel_dim(80) == 128 and M._kernel_dim(32) == 64 and M._kernel_dim(128) == 128
    assert M._kernel_dim(129) == 256 and M._kernel_dim(192) == 256 and M._kernel_dim(256) == 256
    with pytest.raises(ValueError, match=r"\[1, 128\] or 256"):
        M._kernel_block(200)
    with pytest.raises(ValueError, match="head_dim"):
        M._kernel_dim(257)
    rows = M._block_rows(12, 3, 64, torch.device("cpu"))
    assert rows.tolist() == [0, 1, 2, 64, 65, 66, 128, 129, 130, 192, 193, 194]
    # blocks per sequence (the route / CSR rows in LDS; the generic coarse kernels)
    bf, f32 = torch.zeros(1, 1, 1, 96, dtype=torch.bfloat16), torch.zeros(1, 1, 1, 64)
    M._check_block_count(16000, bf)
    with pytest.raises(ValueError, match="at most 16000 blocks"):
        M._check_block_count(16001, bf)
    M._check_block_count(4096, f32)
    with pytest.raises(ValueError, match="at most 4096 blocks"):
        M._check_block_count(4097, f32)
    with pytest.raises(ValueError, match="at most 4096 blocks"):   # head dim 256: generic coarse
        M._check_block_count(4097, torch.zeros(1, 1, 1, 200, dtype=torch.float16))
    M._check_block_count(16000, f32, coarse=False)                 # explicit route: no coarse
