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


def _legacy_sorted_case(N, C, sizes, seed):
    """bev_pool_legacy.py:102-104: rows sorted by the legacy (x, y, z, b)
    rank (stably here), geom_feats as int32, the runs of equal ranks."""
    feats, coords = make_case(N, C, *sizes, seed=seed)
    ranks = ref.legacy_ranks(coords, *sizes)
    order = torch.sort(ranks, stable=True).indices
    fs, cs, rs = feats[order].contiguous(), coords[order].int().contiguous(), ranks[order]
    starts, lengths = ref.runs(rs)
    return fs, cs, rs, starts, lengths


@pytest.mark.parametrize('N,C,sizes,seed', [(64, 8, (2, 3, 4, 5), 0),
                                            (20000, 80, (1, 1, 90, 90), 1),
                                            (3000, 130, (2, 2, 8, 9), 2),
                                            (5000, 300, (1, 1, 16, 16), 3)])
def test_ext_module_vs_oracle(pkg, cuda, N, C, sizes, seed):
    """ext_module.bev_pool_forward / bev_pool_backward (the reference's pybind
    functions, csrc/bev_pool_cpu.cpp:22-94) on the intervals the legacy
    module builds: bit-exact against the oracle's restatement of the legacy
    kernels, forward (row-order sums into the first row's cell, zeros
    elsewhere) and backward (the cell's gradient row into every row)."""
    fs, cs, _, starts, lengths = _legacy_sorted_case(N, C, sizes, seed)
    ext = pkg.legacy.ext_module
    out = ext.bev_pool_forward(fs.to(cuda), cs.to(cuda), lengths.to(cuda), starts.to(cuda), *sizes)
    exp, bad = ref.legacy_forward(fs, cs, lengths, starts, *sizes)
    assert bad == 0 and out.shape == exp.shape
    assert_bit_equal(out, exp, 'ext forward')
    g = torch.randn(exp.shape, generator=torch.Generator().manual_seed(seed + 40))
    xg = ext.bev_pool_backward(g.to(cuda), cs.to(cuda), lengths.to(cuda), starts.to(cuda), *sizes)
    exp_g, _ = ref.legacy_backward(g, cs, lengths, starts, *sizes)
    assert_bit_equal(xg, exp_g, 'ext backward')
    pkg.check_errors()


def test_ext_module_arbitrary_intervals(pkg, cuda):
    """Intervals that are not the runs of a rank: gaps (rows in no interval
    get a zero gradient), empty intervals, rows of several cells summed into
    the first row's cell; and the reference's type checks."""
    sizes = (1, 2, 6, 7)
    feats, coords = make_case(400, 12, *sizes, seed=6)
    starts = torch.tensor([0, 10, 40, 41, 100, 250], dtype=torch.int32)
    lengths = torch.tensor([7, 25, 0, 30, 90, 150], dtype=torch.int32)
    # distinct first-row cells (two intervals of one cell race in the reference)
    cells = ref.flatten_ranks(coords[starts.long()], *sizes)
    assert len(set(cells.tolist())) == len(cells)
    ext = pkg.legacy.ext_module
    c = coords.int()
    out = ext.bev_pool_forward(feats.to(cuda), c.to(cuda), lengths.to(cuda), starts.to(cuda),
                               *sizes)
    exp, _ = ref.legacy_forward(feats, c, lengths, starts, *sizes)
    assert_bit_equal(out, exp, 'arbitrary intervals forward')
    g = torch.randn(exp.shape, generator=torch.Generator().manual_seed(8))
    xg = ext.bev_pool_backward(g.to(cuda), c.to(cuda), lengths.to(cuda), starts.to(cuda), *sizes)
    assert_bit_equal(xg, ref.legacy_backward(g, c, lengths, starts, *sizes)[0], 'gaps backward')
    with pytest.raises(RuntimeError, match='expected scalar type Float but found Half'):
        ext.bev_pool_forward(feats.half().to(cuda), c.to(cuda), lengths.to(cuda),
                             starts.to(cuda), *sizes)
    with pytest.raises(RuntimeError, match='expected scalar type Int but found Long'):
        ext.bev_pool_forward(feats.to(cuda), coords.long().to(cuda), lengths.to(cuda),
                             starts.to(cuda), *sizes)
    pkg.check_errors()


def test_ext_module_invalid_intervals_skipped(pkg, cuda):
    """An interval past the rows or whose first row's cell lies outside the
    grid is skipped (the reference reads/writes out of bounds) and reported
    by check_errors(); the other intervals are unaffected."""
    sizes = (1, 1, 5, 5)
    feats, coords = make_case(50, 4, *sizes, seed=9)
    c = coords.int()
    c[20] = torch.tensor([7, 0, 0, 0], dtype=torch.int32)  # x >= H
    starts = torch.tensor([0, 20, 30, 45], dtype=torch.int32)
    lengths = torch.tensor([5, 3, 4, 9], dtype=torch.int32)  # the last one runs past n = 50
    out = pkg.legacy.ext_module.bev_pool_forward(feats.to(cuda), c.to(cuda), lengths.to(cuda),
                                                 starts.to(cuda), *sizes)
    exp, bad = ref.legacy_forward(feats, c, lengths, starts, *sizes)
    assert bad == 2
    assert_bit_equal(out, exp, 'valid intervals')
    with pytest.raises(RuntimeError, match='2 intervals'):
        pkg.check_errors()


def test_quick_cumsum_honours_runs(pkg, cuda):
    """QuickCumsumCuda (bev_pool_legacy.py:53-96) defines the intervals from
    the caller's ranks: with ranks coarser than the coords (two cells share a
    rank), each run is summed into the cell of its first row, as the legacy
    kernel does -- not pooled by coords."""
    B, D, H, W = 1, 2, 10, 12
    fs, cs, rs, _, _ = _legacy_sorted_case(4000, 24, (B, D, H, W), seed=12)
    coarse = rs // 3
    starts, lengths = ref.runs(coarse)
    f = fs.to(cuda).requires_grad_(True)
    out = pkg.legacy.QuickCumsumCuda.apply(f, cs.to(cuda), coarse.to(cuda), B, D, H, W)
    exp, _ = ref.legacy_forward(fs, cs, lengths, starts, B, D, H, W)
    assert_bit_equal(out, exp, 'coarse runs forward')
    assert not torch.equal(exp, ref.bev_pool_cpu(fs, cs, B, D, H, W))  # the runs matter
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(13))
    out.backward(g.to(cuda))
    assert_bit_equal(f.grad, ref.legacy_backward(g, cs, lengths, starts, B, D, H, W)[0],
                     'coarse runs backward')
    # int32 ranks (the legacy module's int32 coords give int32 ranks)
    out32 = pkg.legacy.QuickCumsumCuda.apply(fs.to(cuda), cs.to(cuda), coarse.int().to(cuda),
                                              B, D, H, W)
    assert_bit_equal(out32, exp, 'int32 ranks')
    pkg.check_errors()


def test_runs_entry(pkg, cuda):
    """bevpool_runs through the C ABI: the runs of an unsorted int64 / int32
    array (bev_pool_legacy.py:56-61), count in meta."""
    from bevfusion_triton_amd import legacy as lg

    g = torch.Generator().manual_seed(14)
    for n in (1, 255, 256, 257, 70000):
        r = torch.randint(0, 5, (n,), generator=g).cumsum(0) // 7
        for dt in (torch.int64, torch.int32):
            starts, lengths, meta = lg._runs(r.to(dt).to(cuda))
            m = int(meta[1].item())
            es, el = ref.runs(r)
            assert m == es.numel()
            assert torch.equal(starts[:m].cpu(), es) and torch.equal(lengths[:m].cpu(), el)
