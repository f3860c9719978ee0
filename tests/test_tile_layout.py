"""Host-side helpers of the MFMA tile layouts (pure torch, no GPU): the fp32 tile layout of the
decode residual stream against its element-offset definition, its inverse, and the gate / up
interleave of the fused SwiGLU projection."""

import torch

from mdlarc_scale_amd import kernels as K


def _tile_off32(m: int, j: int, cols: int) -> int:
    # the definition in include/mdlarc_hip.h / csrc/common.h tile_off32: 16 x 32 blocks of 512
    # floats, lane 16 q + m % 16 owns columns 8 q .. 8 q + 7 (q = (j / 8) % 4), elements 0..3 at
    # 4 lane and 4..7 at 256 + 4 lane of the block
    return (512 * ((m // 16) * (cols // 32) + j // 32) + 256 * ((j // 4) % 2)
            + 4 * (16 * ((j // 8) % 4) + m % 16) + j % 4)


def test_tile_f32_follows_the_layout_definition():
    rows, cols = 37, 96
    x = torch.arange(rows * cols, dtype=torch.float32).view(rows, cols)
    t = K.tile_f32(x)
    assert t.numel() == K.tile_rows(rows) * cols == 48 * cols
    for m in range(rows):
        for j in range(cols):
            assert t[_tile_off32(m, j, cols)] == x[m, j]
    # padding rows are zero
    covered = torch.zeros_like(t, dtype=torch.bool)
    for m in range(rows):
        for j in range(cols):
            covered[_tile_off32(m, j, cols)] = True
    assert bool((t[~covered] == 0).all())


def test_tile_f32_round_trip_and_contiguous_quads():
    g = torch.Generator().manual_seed(3)
    for rows, cols in ((1, 32), (16, 64), (50, 1280)):
        x = torch.randn(rows, cols, generator=g)
        assert torch.equal(K.untile_f32(K.tile_f32(x), rows, cols), x)
    # four consecutive columns starting at a multiple of 4 are contiguous (float4 stores)
    for m, j in ((0, 0), (17, 36), (5, 92)):
        base = _tile_off32(m, j, 96)
        assert [_tile_off32(m, j + e, 96) for e in range(4)] == [base + e for e in range(4)]


def test_tile_rows_and_split_numel():
    assert [K.tile_rows(r) for r in (0, 1, 16, 17, 256)] == [0, 16, 16, 32, 256]
    assert K.split_numel(3, 64, False) == 3 * 128
    assert K.split_numel(3, 64, True) == 16 * 128


def test_interleave_gate_up():
    f, k = 48, 8
    wg = torch.arange(f * k, dtype=torch.float32).view(f, k)
    wu = -wg - 1
    w = K.interleave_gate_up(wg, wu)
    assert w.shape == (2 * f, k)
    for b in range(f // 16):
        assert torch.equal(w[32 * b:32 * b + 16], wg[16 * b:16 * b + 16])
        assert torch.equal(w[32 * b + 16:32 * b + 32], wu[16 * b:16 * b + 16])
