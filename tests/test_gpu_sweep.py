"""A seeded sweep of op-level shapes against the CPU oracle: grids whose rank
spaces take every form of the sort (LSD passes below 11 bits, one or two
blocks per group at 11..19 bits, 8192-key slices at 20 bits), channel counts
around the channel-block and summing-lane limits, fp32 and bf16 features, and
point sets that are uniform, concentrated in a few cells, or packed into one
group of the global pass.  Forward and backward bit-exact (bf16: the fp32 sum
rounded once; its gradient a copy)."""
from __future__ import annotations

import pytest
import torch

from test_gpu_op import assert_bit_equal, oracle_op, run_op

pytestmark = pytest.mark.gpu

# (B, D, H, W): 6, 11, 15, 16, 17, 19 and 20-bit rank spaces
GRIDS = [(1, 1, 5, 10), (2, 3, 17, 19), (1, 2, 128, 100), (1, 1, 256, 256), (1, 1, 360, 360),
         (4, 1, 360, 360), (1, 2, 720, 720)]
CHANNELS = [1, 3, 4, 16, 80, 96, 130]


def sweep_case(seed):
    """Case `seed`: grid, channels, dtype, point count and layout, all drawn
    from a generator seeded with `seed`."""
    g = torch.Generator().manual_seed(1000 + seed)
    pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=g))]
    B, D, H, W = GRIDS[seed % len(GRIDS)]
    # at most 20 M output elements (the oracle's CPU tensors)
    C = pick([c for c in CHANNELS if B * D * H * W * c <= 20_000_000])
    dtype = torch.bfloat16 if seed % 4 == 3 else torch.float32
    N = int(torch.randint(1, 160_000, (1,), generator=g))
    layout = ('uniform', 'dense cells', 'one group')[seed % 3]
    x = torch.randint(0, H, (N,), generator=g)
    y = torch.randint(0, W, (N,), generator=g)
    z = torch.randint(0, D, (N,), generator=g)
    b = torch.randint(0, B, (N,), generator=g)
    if layout == 'dense cells':
        # 70% of the points in 5 cells, in random places of the point order
        hot = torch.rand(N, generator=g) < 0.7
        k = torch.randint(0, 5, (N,), generator=g)
        x = torch.where(hot, (k * 7 + 3) % H, x)
        y = torch.where(hot, (k * 13 + 1) % W, y)
        z = torch.where(hot, torch.zeros_like(z), z)
        b = torch.where(hot, torch.zeros_like(b), b)
    elif layout == 'one group':
        # 60% of the points in the 256 consecutive ranks from one random
        # rank: one group of the global pass, or a few at small grids
        cells = B * D * H * W
        hot = torch.rand(N, generator=g) < 0.6
        r0 = int(torch.randint(0, max(cells - 256, 1), (1,), generator=g))
        r = r0 + torch.randint(0, min(256, cells), (N,), generator=g)
        rb, rem = r // (D * H * W), r % (D * H * W)
        rz, rem = rem // (H * W), rem % (H * W)
        rx, ry = rem // W, rem % W
        x, y, z, b = (torch.where(hot, a, c) for a, c in ((rx, x), (ry, y), (rz, z), (rb, b)))
    coords = torch.stack([x, y, z, b], 1).to(torch.int32)
    feats = torch.randn((N, C), generator=g).to(dtype)
    return (B, D, H, W), C, dtype, N, layout, feats, coords


@pytest.mark.parametrize('seed', range(21))
def test_sweep(pkg, cuda, seed):
    sizes, C, dtype, N, layout, feats, coords = sweep_case(seed)
    what = f'seed {seed}: {sizes} C={C} {dtype} N={N} {layout}'
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, _ = oracle_op(feats.float(), coords, sizes, up)
    assert_bit_equal(out, out32.to(dtype), f'{what} fwd')
    _, gref = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(grad, gref, f'{what} bwd')
