"""The allocation-free op-level forward (``bevpool_op_forward_noalloc``, whose
workspace is a static device array inside the library) through the C ABI,
against ``bevpool_op_forward`` with a caller-owned workspace on the same
inputs: bit-exact on two calls in a row, the second with a smaller input (the
array keeps the first call's contents), the documented refusal of a
workspace larger than the array, and, after a warm-up call, no change in free
device memory and no timing records."""
from __future__ import annotations

import pytest
import torch

from oracle import torch_fallback as ref
from test_gpu_op import assert_bit_equal, rand_case

pytestmark = pytest.mark.gpu

BEVPOOL_NOALLOC_MAX_BYTES = 96 << 20  # include/bevpool.h


def _noalloc(pkg, feats, coords, sizes, out):
    from bevfusion_triton_amd import _lib as L

    B, D, H, W = sizes
    n, C = feats.shape
    return L.library().bevpool_op_forward_noalloc(
        L.ptr(feats), L.DTYPE_CODES[feats.dtype], C, C, L.ptr(coords), coords.element_size(), 4,
        n, B, D, H, W, L.ptr(out), L.stream_handle(feats.device))


def _with_workspace(feats, coords, sizes):
    from bevfusion_triton_amd import _pipeline as P

    B, D, H, W = sizes
    n, C = feats.shape
    index = P.op_index(n, B * D * H * W, feats.device)
    scratch = P.op_scratch(n, B * D * H * W, C, feats.device)
    out = torch.empty((B, C, D, H, W), dtype=feats.dtype, device=feats.device)
    P.op_forward(feats, coords, B, D, H, W, out, index, scratch)
    return out


@pytest.mark.parametrize('cases', [
    # det-sized op call (1.77 M kept points, 360 x 360, C = 80: 78 MiB of workspace), then a
    # smaller one; and a bf16 pair
    [(1774050, 80, (1, 1, 360, 360), 1, torch.float32), (30000, 24, (1, 2, 40, 50), 2,
                                                          torch.float32)],
    [(200000, 64, (2, 1, 100, 100), 3, torch.bfloat16), (5000, 16, (1, 1, 30, 30), 4,
                                                          torch.bfloat16)],
])
def test_noalloc_matches_workspace_entry(pkg, cuda, cases):
    for N, C, sizes, seed, dtype in cases:
        feats, coords = rand_case(N, C, *sizes, dtype=dtype, seed=seed)
        f, c = feats.to(cuda), coords.to(cuda)
        out = torch.full((sizes[0], C, *sizes[1:]), 7.0, dtype=dtype, device=cuda)
        st = _noalloc(pkg, f, c, sizes, out)
        assert st == 0, pkg.library().bevpool_last_error()
        torch.cuda.synchronize()
        assert_bit_equal(out, _with_workspace(f, c, sizes), f'noalloc N={N}')
        if N <= 30000:  # and against the oracle where it is quick
            assert_bit_equal(out, ref.bev_pool(feats.float(), coords, *sizes).to(dtype),
                             f'noalloc N={N} vs oracle')


def test_noalloc_refuses_oversized(pkg, cuda):
    lib = pkg.library()
    n, sizes, C = 4_000_000, (2, 1, 360, 360), 80
    assert lib.bevpool_op_workspace_bytes(n, 2 * 360 * 360, C) > BEVPOOL_NOALLOC_MAX_BYTES
    feats = torch.empty((1, C), device=cuda)  # never read: the size check comes first
    coords = torch.zeros((1, 4), dtype=torch.int32, device=cuda)
    from bevfusion_triton_amd import _lib as L

    st = lib.bevpool_op_forward_noalloc(L.ptr(feats), 0, C, C, L.ptr(coords), 4, 4, n, *sizes,
                                        L.ptr(feats), L.stream_handle(cuda))
    assert st == -3
    assert b'static scratch' in lib.bevpool_last_error()
    # a valid call right after still works
    f, c = rand_case(1000, 8, 1, 1, 10, 10, seed=5)
    out = torch.empty((1, 8, 1, 10, 10), device=cuda)
    assert _noalloc(pkg, f.to(cuda), c.to(cuda), (1, 1, 10, 10), out) == 0
    assert_bit_equal(out, ref.bev_pool(f, c, 1, 1, 10, 10), 'after refusal')


def test_noalloc_allocates_nothing(pkg, cuda):
    """The property the entry point exists for: after one warm-up call on the
    device, a call leaves the device's free memory unchanged (no hipMalloc)
    and records no timing events even with the library's timing on."""
    from bevfusion_triton_amd import _lib as L

    sizes = (1, 2, 40, 50)
    f, c = rand_case(30000, 24, *sizes, seed=6)
    f, c = f.to(cuda), c.to(cuda)
    out = torch.empty((1, 24, 2, 40, 50), device=cuda)
    assert _noalloc(pkg, f, c, sizes, out) == 0  # warm-up: resolves the array's address
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info(cuda)
    L.timing_reset()
    L.timing_enable(True)
    try:
        for _ in range(3):
            assert _noalloc(pkg, f, c, sizes, out) == 0, pkg.library().bevpool_last_error()
        torch.cuda.synchronize()
    finally:
        L.timing_enable(False)
    free1, _ = torch.cuda.mem_get_info(cuda)
    assert free1 == free0, f'free device memory changed by {free0 - free1} bytes'
    assert L.timing_read() == {}, 'the allocation-free call recorded timing events'
    assert_bit_equal(out, ref.bev_pool(f.cpu(), c.cpu(), *sizes), 'noalloc after warm-up')
