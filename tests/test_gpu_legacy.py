"""GPU parity of the legacy-module drop-in (``legacy.bev_pool``,
``legacy.QuickCumsumCuda``: ``ops/bev_pool/bev_pool_legacy.py:53-108``)
against the CPU oracle.  The legacy path sums each cell in the order of a
non-stable argsort; the drop-in sums in point order (a permitted order, and
the CPU fallback's), so the bar is bit-exact against the oracle, forward and
backward, including the reference's own legacy-vs-Triton case
(``tests/test_ops/test_bev_pool.py:87-119``: B, D, H, W = 2, 3, 4, 5, N = 64,
C = 8)."""
from __future__ import annotations

import pytest
import torch

from oracle import torch_fallback as ref
from test_gpu_op import assert_bit_equal, rand_case as make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('N,C,sizes,seed', [(64, 8, (2, 3, 4, 5), 0),
                                            (20000, 32, (2, 4, 30, 40), 1),
                                            (5000, 80, (1, 1, 64, 64), 2)])
def test_legacy_bev_pool(pkg, cuda, N, C, sizes, seed):
    feats, coords = make_case(N, C, *sizes, seed=seed)
    f = feats.to(cuda).requires_grad_(True)
    out = pkg.legacy.bev_pool(f, coords.to(cuda), *sizes)
    fr = feats.clone().requires_grad_(True)
    out_ref = ref.bev_pool(fr, coords, *sizes)
    assert out.is_contiguous()
    assert_bit_equal(out, out_ref, 'legacy forward')
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 9))
    (out * g.to(cuda)).sum().backward()
    (out_ref * g).sum().backward()
    assert_bit_equal(f.grad, fr.grad, 'legacy backward')
    # and the same bits as the op-level function
    assert_bit_equal(out, pkg.bev_pool(feats.to(cuda), coords.to(cuda), *sizes), 'legacy = op')


def test_quick_cumsum_cuda_presorted(pkg, cuda):
    """QuickCumsumCuda on inputs pre-sorted by the legacy (x, y, z, b) rank,
    as bev_pool_legacy.py:102-106 calls it: (B, D, H, W, C) output."""
    B, D, H, W = 2, 3, 16, 12
    feats, coords = make_case(3000, 16, B, D, H, W, seed=4)
    c = coords.long()
    ranks = c[:, 0] * (W * D * B) + c[:, 1] * (D * B) + c[:, 2] * B + c[:, 3]
    order = torch.argsort(ranks, stable=True)
    fs, cs, rs = feats[order], coords[order], ranks[order]
    f = fs.to(cuda).requires_grad_(True)
    out = pkg.legacy.QuickCumsumCuda.apply(f, cs.to(cuda), rs.to(cuda), B, D, H, W)
    assert out.shape == (B, D, H, W, 16) and out.is_contiguous()
    fr = fs.clone().requires_grad_(True)
    out_ref = ref.bev_pool_cpu(fr, cs, B, D, H, W)
    assert_bit_equal(out, out_ref, 'QuickCumsumCuda forward')
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5))
    (out * g.to(cuda)).sum().backward()
    (out_ref * g).sum().backward()
    assert_bit_equal(f.grad, fr.grad, 'QuickCumsumCuda backward')


def test_legacy_requires_fp32(pkg, cuda):
    feats, coords = make_case(64, 8, 2, 3, 4, 5, seed=0)
    with pytest.raises(RuntimeError, match='expected scalar type Float'):
        pkg.legacy.bev_pool(feats.to(cuda).half(), coords.to(cuda), 2, 3, 4, 5)
    with pytest.raises(AssertionError):
        pkg.legacy.bev_pool(feats.to(cuda), coords[:10].to(cuda), 2, 3, 4, 5)
