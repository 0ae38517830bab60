"""GPU parity of the op-level ``bev_pool(feats, coords, B, D, H, W)`` (through
the C ABI) against the CPU oracle (oracle/torch_fallback.py).

Bar: indices (ranks, stable permutation, interval starts/lengths) and fp32
forward/backward bit-exact; fp16/bf16 forward bit-exact against the fp32
sequential sum rounded once (fp32 accumulation) and within 1e-2 relative of
the fp32 reference; fp16/bf16 backward bit-exact (a copy).
"""
from __future__ import annotations

import json
import time

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import torch_fallback as ref

pytestmark = pytest.mark.gpu


def rand_case(N, C, B, D, H, W, dtype=torch.float32, seed=0, idx_dtype=torch.int32):
    """The reference's _build_case_tensors (tests/test_ops/test_bev_pool.py:24-47),
    generated on the CPU with a seeded generator."""
    g = torch.Generator().manual_seed(seed)
    feats = torch.randn((N, C), generator=g).to(dtype)
    coords = torch.stack([
        torch.randint(0, H, (N,), generator=g), torch.randint(0, W, (N,), generator=g),
        torch.randint(0, D, (N,), generator=g), torch.randint(0, B, (N,), generator=g),
    ], 1).to(idx_dtype)
    return feats, coords


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def assert_bit_equal(a, b, what=''):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert a.dtype == b.dtype, (what, a.dtype, b.dtype)
    if not torch.equal(bits(a), bits(b)):
        d = (a.detach().cpu().double() - b.detach().cpu().double()).abs()
        raise AssertionError(f'{what}: not bit-identical (max |diff| {d.max().item():.3e}, '
                             f'{int((bits(a) != bits(b)).sum())} elements)')


def run_op(pkg, feats, coords, sizes, cuda, upstream=None):
    f = feats.to(cuda).requires_grad_(True)
    out = pkg.bev_pool(f, coords.to(cuda), *sizes)
    if upstream is None:
        upstream = torch.randn(out.shape, generator=torch.Generator().manual_seed(11))
    (out * upstream.to(cuda, out.dtype)).sum().backward()
    torch.cuda.synchronize()
    return out, f.grad, upstream


def oracle_op(feats, coords, sizes, upstream):
    f = feats.clone().requires_grad_(True)
    out = ref.bev_pool(f, coords, *sizes)
    (out * upstream.to(out.dtype)).sum().backward()
    return out, f.grad


def test_known_case(pkg, cuda):
    k = json.loads((GOLDEN / 'known_case.json').read_text())
    feats = torch.tensor(k['feats'], device=cuda)
    coords = torch.tensor(k['coords'], dtype=torch.int32, device=cuda)
    out = pkg.bev_pool(feats, coords, k['B'], k['D'], k['H'], k['W'])
    assert out.is_contiguous() and list(out.shape) == k['expected_shape']
    assert torch.equal(out.cpu(), torch.tensor(k['expected']))


def test_known_case_rejects(pkg, cuda):
    k = json.loads((GOLDEN / 'known_case.json').read_text())
    for case in k['reject']:
        feats = torch.zeros((4, 3), dtype=getattr(torch, case['feats_dtype']), device=cuda)
        coords = torch.zeros((4, 4), dtype=getattr(torch, case['coords_dtype']), device=cuda)
        with pytest.raises(TypeError):
            pkg.bev_pool(feats, coords, 1, 1, 1, 1)


def test_order_case(pkg, cuda):
    o = json.loads((GOLDEN / 'order_case.json').read_text())
    feats = torch.from_numpy(np.array(o['feats_f32_bits'], np.uint32).view(np.float32).copy())
    coords = torch.tensor(o['coords'], dtype=torch.int64)
    out = pkg.bev_pool(feats.to(cuda), coords.to(cuda), o['B'], o['D'], o['H'], o['W'])
    got = out.cpu().reshape(-1).view(torch.int32).numpy().astype(np.uint32).tolist()
    assert got == o['expected_f32_bits']


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_reference_parity_case(pkg, cuda, dtype):
    """The reference's legacy-vs-Triton case (test_bev_pool.py:87-119):
    B,D,H,W = 2,3,4,5, N=64, C=8, seed 0, random upstream gradient."""
    sizes = (2, 3, 4, 5)
    feats, coords = rand_case(64, 8, *sizes, dtype=dtype)
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, grad32 = oracle_op(feats.float(), coords, sizes, up)
    assert out.dtype == dtype and out.is_contiguous()
    if dtype == torch.float32:
        assert_bit_equal(out, out32, 'fwd')
        assert_bit_equal(grad, grad32, 'bwd')
    else:
        assert_bit_equal(out, out32.to(dtype), 'fwd (fp32 accumulation, one rounding)')
        rel = (out.cpu().float() - out32).norm() / out32.norm()
        assert rel <= 1e-2, rel
        # backward: a copy of the (dtype-rounded) upstream gradient
        _, gref = oracle_op(feats, coords, sizes, up)
        assert_bit_equal(grad, gref, 'bwd')


@pytest.mark.parametrize('idx_dtype', [torch.int32, torch.int64])
def test_index_stage_bit_exact(pkg, cuda, idx_dtype):
    sizes = (2, 3, 17, 19)
    _, coords = rand_case(20000, 1, *sizes, seed=3, idx_dtype=idx_dtype)
    exp = pkg.BevPoolIndexExport(coords.to(cuda), *sizes)
    ranks = ref.flatten_ranks(coords, *sizes)
    assert torch.equal(exp.rank.cpu(), ranks)
    perm = ref.sort_perm(ranks)
    assert torch.equal(exp.perm.cpu(), perm)
    assert torch.equal(exp.sorted_ranks.cpu(), ranks[perm])
    starts, lengths = ref.intervals(ranks[perm])
    assert torch.equal(exp.starts.cpu(), starts)
    assert torch.equal(exp.lengths.cpu(), lengths)
    assert torch.equal(exp.cells.cpu().long(), ranks[perm][starts.long()])
    assert exp.n_bad == 0


@pytest.mark.parametrize('N,sizes,C', [
    (0, (1, 1, 2, 3), 4),           # empty input -> zeros
    (1, (1, 1, 1, 1), 1),           # single point, single cell
    (30000, (1, 1, 1, 1), 5),       # every point in one cell: one 30000-long interval
    (5000, (3, 2, 7, 300), 3),      # C not a multiple of 4, >10-bit ranks (2 radix passes)
    (4000, (1, 1, 40, 50), 300),    # C > 256 (channel blocking)
    (70000, (2, 4, 64, 64), 16),    # 15-bit ranks
])
def test_shapes_and_edges(pkg, cuda, N, sizes, C):
    feats, coords = rand_case(N, C, *sizes, seed=N + C)
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, grad32 = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(out, out32, 'fwd')
    assert_bit_equal(grad, grad32, 'bwd')


@pytest.mark.parametrize('idx_dtype', [torch.int32, torch.int64])
@pytest.mark.parametrize('N', [5000, 9001])
def test_strided_coords(pkg, cuda, idx_dtype, N):
    """coords as the first four columns of a wider integer tensor (row stride
    6, passed to the library without a copy), int32 and int64, with a
    partial last index tile: ranks read through the row stride, forward and
    backward bit-exact."""
    sizes = (2, 3, 17, 19)
    feats, coords = rand_case(N, 8, *sizes, seed=N, idx_dtype=idx_dtype)
    wide = torch.full((N, 6), 7777, dtype=idx_dtype)
    wide[:, :4] = coords
    cw = wide.to(cuda)[:, :4]
    assert cw.stride() == (6, 1)
    out, grad, up = run_op(pkg, feats, cw, sizes, cuda)
    out32, grad32 = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(out, out32, 'fwd')
    assert_bit_equal(grad, grad32, 'bwd')


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
@pytest.mark.parametrize('C', [90, 136, 200, 264])
def test_half_channel_blocks(pkg, cuda, dtype, C):
    """16-bit rows with fp32 sums: one channel block (136), a second partial
    block beyond the 192 channels one block of 16-bit rows holds (200, 264),
    and a row size that is not a multiple of 16 bytes (90: the element-wise
    accumulation).  Forward = the fp32 sum of the same values rounded once;
    backward = the upstream gradient gathered (a copy)."""
    sizes = (1, 2, 20, 25)
    feats, coords = rand_case(6000, C, *sizes, dtype=dtype, seed=C)
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, _ = oracle_op(feats.float(), coords, sizes, up)
    assert out.dtype == dtype
    assert_bit_equal(out, out32.to(dtype), f'fwd C={C}')
    _, gref = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(grad, gref, f'bwd C={C}')


@pytest.mark.parametrize('name,sizes', [
    ('11-bit ranks, 2-cell groups', (1, 1, 5, 205)),
    ('16-bit ranks, 9 + 7 bits', (1, 1, 256, 256)),
    ('16-bit ranks, 9 + 7 bits, one group holding most points', (1, 1, 256, 256)),
    ('17-bit ranks, groups at the part threshold', (1, 1, 360, 360)),
    ('20-bit ranks, 1024-cell groups', (1, 1, 1024, 1024)),
    ('17-bit ranks, one group holding most points', (1, 1, 360, 360)),
    ('20-bit ranks, one group holding most points', (1, 1, 1024, 1024)),
    ('20-bit ranks, groups at slice boundaries', (1, 1, 1024, 1024)),
])
def test_bucket_sort_edges(pkg, cuda, name, sizes):
    """Ranks of 11..20 bits: one global pass by the high digit (half the
    bits rounded up; 9 of 16), then the low bits are sorted per group (groups
    of up to 512 cells by one block, or by two blocks each taking half the
    keys above 8192 keys; groups of 1024 cells are cut into slices of 8192
    keys) and the group's cell ranges written.  Cases: the smallest groups,
    the largest rank space, one group far larger than the rest (90% of the
    points in 3 cells, sizes not multiples of 64) with empty groups around
    it, groups of 8192, 8193 and 20,000 keys spread over the point order (one
    block; two parts; two parts too large for registers), and groups of
    exactly 1, 2 and 4 slices and one key more."""
    N = 120000
    feats, coords = rand_case(N, 8, *sizes, seed=11)
    if 'part threshold' in name:
        # rank x * 360 + y: group g (rank >> 8) holds ranks [256 g, 256 g + 256);
        # groups 10, 20, 30 get 8192, 8193 and 20,000 points at random places
        # of the point order, on random cells of the group
        g = torch.Generator().manual_seed(14)
        order = torch.randperm(N, generator=g)
        at = 0
        for grp, n in ((10, 8192), (20, 8193), (30, 20000)):
            idx = order[at:at + n]
            r = grp * 256 + torch.randint(0, 256, (n,), generator=g)
            coords[idx, 0] = (r // 360).to(coords.dtype)
            coords[idx, 1] = (r % 360).to(coords.dtype)
            at += n
        rest = order[at:]
        r = torch.randint(0, 360 * 360, (len(rest),), generator=g)
        r = torch.where((r >> 8 == 10) | (r >> 8 == 20) | (r >> 8 == 30), r + 256, r)
        coords[rest, 0] = (r // 360).to(coords.dtype)
        coords[rest, 1] = (r % 360).to(coords.dtype)
    if 'one group' in name:
        g = torch.Generator().manual_seed(12)
        hot = torch.rand(N, generator=g) < 0.9
        cell = torch.randint(0, 3, (N,), generator=g)
        coords[hot, 0] = 200  # x: cells 200*W + 100..102 share one group
        coords[hot, 1] = 100 + cell[hot].to(coords.dtype)
    if 'slice boundaries' in name:
        # with W = 1024 the group of a point is its x: groups 5, 9, 11, 13,
        # 17, 19 get 8192, 8193, 16384, 16385, 32768, 32769 points, spread
        # over the point order; the other points fall in other groups
        g = torch.Generator().manual_seed(13)
        xs = torch.randint(0, 1024, (N,), generator=g)
        xs[(xs == 5) | (xs == 9) | (xs == 11) | (xs == 13) | (xs == 17) | (xs == 19)] = 0
        order = torch.randperm(N, generator=g)
        at = 0
        for x, n in ((5, 8192), (9, 8193), (11, 16384), (13, 16385), (17, 32768), (19, 32769)):
            xs[order[at:at + n]] = x
            at += n
        coords[:, 0] = xs.to(coords.dtype)
    B, D, H, W = sizes
    exp = pkg.BevPoolIndexExport(coords.to(cuda), *sizes)
    ranks = ref.flatten_ranks(coords, *sizes)
    perm = ref.sort_perm(ranks)
    assert torch.equal(exp.perm.cpu(), perm), name
    starts, lengths = ref.intervals(ranks[perm])
    assert torch.equal(exp.starts.cpu(), starts), name
    assert torch.equal(exp.lengths.cpu(), lengths), name
    # dense cell ranges: [start, end) of every occupied cell, (0, 0) elsewhere
    n_cells = B * D * H * W
    cs = torch.zeros(n_cells, dtype=torch.int32)
    ce = torch.zeros(n_cells, dtype=torch.int32)
    cells = ranks[perm][starts.long()]
    cs[cells] = starts
    ce[cells] = starts + lengths
    assert torch.equal(exp.index.cell_start.cpu(), cs), name
    assert torch.equal(exp.index.cell_end.cpu(), ce), name
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, grad32 = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(out, out32, f'{name} fwd')
    assert_bit_equal(grad, grad32, f'{name} bwd')


@pytest.mark.parametrize('N', [50000, 4_500_000])
def test_large_rank_space(pkg, cuda, N):
    """2^21 cells: three radix passes; with more than 4 Mi points the tile
    kernels take 4096-key tiles (16 keys per thread)."""
    sizes = (2, 1, 1024, 1024)
    feats, coords = rand_case(N, 4, *sizes, seed=9)
    exp = pkg.BevPoolIndexExport(coords.to(cuda), *sizes)
    perm = ref.sort_perm(ref.flatten_ranks(coords, *sizes))
    assert torch.equal(exp.perm.cpu(), perm)
    del exp
    out, grad, up = run_op(pkg, feats, coords, sizes, cuda)
    out32, grad32 = oracle_op(feats, coords, sizes, up)
    assert_bit_equal(out, out32, 'fwd')
    assert_bit_equal(grad, grad32, 'bwd')


def test_noncontiguous_feats(pkg, cuda):
    sizes = (1, 2, 9, 11)
    feats, coords = rand_case(3000, 12, *sizes, seed=4)
    wide = torch.randn(3000, 30)
    wide[:, 5:17] = feats
    f = wide.to(cuda)[:, 5:17]  # row stride 30, channel stride 1
    assert not f.is_contiguous()
    out = pkg.bev_pool(f, coords.to(cuda), *sizes)
    assert_bit_equal(out, ref.bev_pool(feats, coords, *sizes), 'fwd strided rows')
    ft = feats.t().contiguous().to(cuda).t()  # channel stride != 1
    out = pkg.bev_pool(ft, coords.to(cuda), *sizes)
    assert_bit_equal(out, ref.bev_pool(feats, coords, *sizes), 'fwd transposed view')


def test_signed_zero_and_specials(pkg, cuda):
    sizes = (1, 1, 2, 2)
    feats = torch.tensor([[-0.0, 1.0], [float('inf'), -0.0], [1.0, float('nan')],
                          [-0.0, -0.0]])
    coords = torch.tensor([[0, 0, 0, 0], [0, 1, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0]])
    out = pkg.bev_pool(feats.to(cuda), coords.to(cuda), *sizes)
    exp = ref.bev_pool(feats, coords, *sizes)
    assert_bit_equal(out, exp, 'fwd specials')


def test_out_of_range_coords_raise(pkg, cuda):
    feats, coords = rand_case(100, 3, 1, 2, 3, 4, seed=1)
    # x == H at z == D-1: rank ((0*2 + 1)*3 + 3)*4 + 0 = 24 == B*D*H*W
    coords[17] = torch.tensor([3, 0, 1, 0], dtype=torch.int32)
    # default: no host synchronisation in the call; the point is excluded and
    # the error is raised once the device has passed the call
    out = pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4)
    keep = torch.arange(100) != 17
    assert_bit_equal(out, ref.bev_pool(feats[keep], coords[keep], 1, 2, 3, 4), 'bad point excluded')
    with pytest.raises(RuntimeError, match='index 24 is out of bounds'):
        pkg.check_errors()
    pkg.check_errors()  # reported once
    # ... or by the next call of the library once the device has finished
    pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match='index 24 is out of bounds'):
        pkg.bev_pool(feats[keep].to(cuda), coords[keep].to(cuda), 1, 2, 3, 4)
    # check_bounds='sync' raises in the call itself
    with pytest.raises(RuntimeError, match='index 24 is out of bounds'):
        pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4, check_bounds='sync')
    coords[17] = torch.tensor([0, 0, 0, -1], dtype=torch.int32)  # negative batch
    with pytest.raises(RuntimeError, match='out of bounds'):
        pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4, check_bounds='sync')
    # check_bounds=False: excluded, never reported
    pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4, check_bounds=False)
    pkg.check_errors()
    # a rank inside [0, B*D*H*W) is accepted even if one coordinate is out of
    # range: the reference flattens first (x = -1, y = 5 -> (-1)*4 + 5 = 1)
    coords[17] = torch.tensor([-1, 5, 0, 0], dtype=torch.int32)
    out = pkg.bev_pool(feats.to(cuda), coords.to(cuda), 1, 2, 3, 4)
    assert_bit_equal(out, ref.bev_pool(feats, coords, 1, 2, 3, 4), 'flattened-rank semantics')


def test_deferred_report_on_side_stream(pkg, cuda):
    """An op-level call queued on a non-default stream: the kernels and the
    report's done flag go to that stream, so once that stream (and only it)
    has finished, the out-of-grid coordinate is raised."""
    feats, coords = rand_case(500, 6, 1, 2, 3, 4, seed=5)
    coords[123] = torch.tensor([0, 0, 0, 1], dtype=torch.int32)  # b == B
    keep = torch.arange(500) != 123
    f, c = feats.to(cuda), coords.to(cuda)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = pkg.bev_pool(f, c, 1, 2, 3, 4)
    side.synchronize()
    assert_bit_equal(out, ref.bev_pool(feats[keep], coords[keep], 1, 2, 3, 4), 'side stream')
    with pytest.raises(RuntimeError, match='index 24 is out of bounds'):
        pkg.check_errors()


def test_deferred_reports_from_threads(pkg, cuda):
    """Op-level calls with deferred bounds reports from several threads at
    once (the autograd engine polls from its own threads): more calls than
    pinned report slots, every result exact, every slot returned and no
    report lost; a bad call afterwards is still reported."""
    import threading

    from bevfusion_triton_amd import _pipeline as P

    sizes = (1, 2, 9, 11)
    feats, coords = rand_case(4000, 8, *sizes, seed=31)
    exp = ref.bev_pool(feats, coords, *sizes)
    f, c = feats.to(cuda), coords.to(cuda)
    g = torch.randn(exp.shape, generator=torch.Generator().manual_seed(32)).to(cuda)
    errors, outs = [], []

    def work():
        try:
            for _ in range(40):
                x = f.clone().requires_grad_(True)
                out = pkg.bev_pool(x, c, *sizes)
                (xg,) = torch.autograd.grad(out, x, g)
            outs.append(out.detach())
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=work) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    pkg.check_errors()
    for out in outs:
        assert_bit_equal(out, exp, 'threaded forward')
    assert not P._pending
    assert sorted(P._readback[cuda].free) == list(range(P._ReadBack._SLOTS))
    bad = coords.clone()
    bad[5] = torch.tensor([9, 0, 1, 0], dtype=torch.int32)  # x == H at z == D-1
    pkg.bev_pool(f, bad.to(cuda), *sizes)
    with pytest.raises(RuntimeError, match='out of bounds'):
        pkg.check_errors()


def test_deterministic(pkg, cuda):
    sizes = (1, 1, 40, 40)
    feats, coords = rand_case(100000, 20, *sizes, seed=8)
    f, c = feats.to(cuda), coords.to(cuda)
    a = pkg.bev_pool(f, c, *sizes)
    b = pkg.bev_pool(f, c, *sizes)
    assert torch.equal(bits(a), bits(b))


def test_zero_channels(pkg, cuda):
    out = pkg.bev_pool(torch.zeros(5, 0, device=cuda), torch.zeros(5, 4, dtype=torch.int32,
                                                                    device=cuda), 1, 1, 1, 1)
    assert out.shape == (1, 0, 1, 1, 1)


def test_op_entry_zero_dropped_flag(pkg, cuda):
    """bevpool_op_forward / bevpool_op_backward through the C ABI (the
    one-call op level): the forward equals the oracle; the backward with
    zero_dropped = 1 writes zero rows for invalid coords, with
    zero_dropped = 0 leaves them as the caller had them."""
    from bevfusion_triton_amd import _lib as L
    from bevfusion_triton_amd import _pipeline as P

    sizes = (2, 1, 12, 13)
    feats, coords = rand_case(5000, 20, *sizes, seed=21)
    # flattened ranks 312 (= B*D*H*W), 312 and -1: outside [0, 312)
    coords[[3, 77, 4999]] = torch.tensor([[12, 0, 0, 1], [0, 0, 0, 2], [0, -1, 0, 0]],
                                         dtype=torch.int32)
    keep = torch.ones(5000, dtype=torch.bool)
    keep[[3, 77, 4999]] = False
    f, c = feats.to(cuda), coords.to(cuda)
    index = P.op_index(5000, 2 * 12 * 13, cuda)
    scratch = P.op_scratch(5000, 2 * 12 * 13, 20, cuda)
    out = torch.empty((2, 20, 1, 12, 13), device=cuda)
    P.op_forward(f, c, *sizes, out, index, scratch)
    scratch.fill_(0x5a)  # the backward needs only the index the forward left
    assert_bit_equal(out, ref.bev_pool(feats[keep], coords[keep], *sizes), 'op entry forward')
    meta = P.op_meta(index).cpu()
    assert int(meta[L.META_N_BAD]) == 3 and int(meta[L.META_FIRST_BAD]) == 3
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(22)).to(cuda)
    exp = torch.zeros(5000, 20)
    exp[keep] = ref.backward_gather(g.cpu(), coords[keep], *sizes)
    xg = torch.full((5000, 20), 7.0, device=cuda)
    P.op_backward(g, 20, 5000, *sizes, xg, index, scratch, zero_dropped=True)
    assert_bit_equal(xg, exp, 'zero_dropped = 1')
    xg = torch.full((5000, 20), 7.0, device=cuda)
    P.op_backward(g, 20, 5000, *sizes, xg, index, scratch, zero_dropped=False)
    exp[~keep] = 7.0
    assert_bit_equal(xg, exp, 'zero_dropped = 0')


def test_meta_report_entry(pkg, cuda):
    """bevpool_meta_report through the C ABI: the counters land in pinned
    host memory, followed by the done flag (polled by the host, no event),
    and in device memory; pageable host memory, which the GPU cannot reach,
    is refused before anything is launched."""
    import ctypes

    from bevfusion_triton_amd import _lib as L

    lib = L.library()
    meta = torch.arange(100, 100 + L.META_LEN, dtype=torch.int32, device=cuda)
    s = L.stream_handle(cuda)
    host = torch.full((3, L.REPORT_LEN), -1, dtype=torch.int32, pin_memory=True)
    host[1, L.META_LEN] = 0
    assert lib.bevpool_meta_report(L.ptr(meta), host[1].data_ptr(), s) == 0
    deadline = time.monotonic() + 10.0
    while int(host[1, L.META_LEN]) != 1:  # the flag, then the counters
        assert time.monotonic() < deadline, 'done flag never set'
        time.sleep(1e-4)
    assert host[1, :L.META_LEN].tolist() == list(range(100, 100 + L.META_LEN))
    assert host[0].tolist() == [-1] * L.REPORT_LEN and host[2].tolist() == [-1] * L.REPORT_LEN
    dev = torch.zeros(L.REPORT_LEN, dtype=torch.int32, device=cuda)
    assert lib.bevpool_meta_report(L.ptr(meta), L.ptr(dev), s) == 0
    assert dev.cpu().tolist() == list(range(100, 100 + L.META_LEN)) + [1]
    pageable = (ctypes.c_int32 * L.REPORT_LEN)()
    assert lib.bevpool_meta_report(L.ptr(meta), ctypes.addressof(pageable), s) == -1
    assert list(pageable) == [0] * L.REPORT_LEN
    assert lib.bevpool_meta_report(L.ptr(meta), 0, s) == -1
    torch.cuda.synchronize()
