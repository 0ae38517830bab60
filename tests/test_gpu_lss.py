"""GPU parity of the LSS vtransform-level pooling (quantise -> kept mask ->
compaction -> sort -> pool -> Z-collapse, and its backward) against the CPU
oracle, on the synthetic camera rig of every benchmark configuration.

Bar: rank, kept mask, stable permutation, interval starts/lengths, fp32
forward and backward bit-exact; bf16 (config 3, op level) bit-exact against
the fp32 sums rounded once and within 1e-2 relative of the fp32 reference.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import torch_fallback as ref
from conftest import GOLDEN
from test_gpu_op import assert_bit_equal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def synthetic(pkg):
    from bevfusion_triton_amd import synthetic

    return synthetic


def grid_of(case):
    return ref.gen_dx_bx(case.xbound, case.ybound, case.zbound)


def check_index(pkg, case, cuda):
    dx, bx, nx = grid_of(case)
    exp = pkg.LSSIndexExport(case.geom.to(cuda), dx, bx, nx)
    oi = ref.lss_index(case.geom, dx, bx, nx)
    assert torch.equal(exp.rank.cpu(), oi.rank), 'rank'
    assert torch.equal(exp.kept.cpu(), oi.kept), 'kept mask'
    assert torch.equal(exp.perm.cpu(), oi.perm), 'stable sort permutation'
    assert torch.equal(exp.sorted_ranks.cpu(), oi.sorted_ranks), 'sorted ranks'
    assert torch.equal(exp.starts.cpu(), oi.starts), 'interval starts'
    assert torch.equal(exp.lengths.cpu(), oi.lengths), 'interval lengths'
    return oi


def check_fwd_bwd(pkg, case, cuda, seed=21):
    dx, bx, nx = grid_of(case)
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    x = case.x.to(cuda).requires_grad_(True)
    out = module.bev_pool(case.geom.to(cuda), x)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed))
    (out * g.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    xr = case.x.clone().requires_grad_(True)
    out_ref = ref.lss_bev_pool(case.geom, xr, dx, bx, nx)
    (out_ref * g).sum().backward()
    assert out.shape == out_ref.shape and out.is_contiguous()
    assert_bit_equal(out, out_ref, f'{case.name} forward')
    assert_bit_equal(x.grad, xr.grad, f'{case.name} backward')


@pytest.mark.parametrize('name', ['tiny', 'det', 'seg'])
def test_lss_single_sample_configs(pkg, cuda, synthetic, name):
    case = synthetic.make_case(name)
    oi = check_index(pkg, case, cuda)
    assert 0 < int(oi.kept.sum()) < case.n_points
    check_fwd_bwd(pkg, case, cuda)


def test_lss_train_batch4(pkg, cuda, synthetic):
    """Config 2: B=4 with per-sample rig perturbations."""
    case = synthetic.make_case('train')
    check_index(pkg, case, cuda)
    check_fwd_bwd(pkg, case, cuda)


def test_lss_hires_out_of_bounds(pkg, cuda, synthetic):
    """Config 4: 720x720 grid, B=2, 10% of points pushed out of bounds and a
    few at q in (-1, 0) (kept in cell 0)."""
    case = synthetic.make_case('hires')
    oi = check_index(pkg, case, cuda)
    assert int((~oi.kept).sum()) >= case.n_points // 10
    check_fwd_bwd(pkg, case, cuda)


def test_bf16_batch8_op_level(pkg, cuda, synthetic):
    """Config 3: bf16 features with fp32 accumulation, B=8, through the op
    level (the vtransform forces fp32, models/helper/amp.py:35-67)."""
    case = synthetic.make_case('bf16')
    dx, bx, nx = grid_of(case)
    q = ref.quantize(case.geom, dx, bx, nx)
    C = case.x.shape[-1]
    feats = case.x.reshape(-1, C)[q.kept]
    coords = q.coords[q.kept]
    B, sizes = case.geom.shape[0], (case.geom.shape[0], int(nx[2]), int(nx[0]), int(nx[1]))
    assert feats.dtype == torch.bfloat16 and B == 8
    out = pkg.bev_pool(feats.to(cuda), coords.to(cuda), *sizes)
    out32 = ref.bev_pool(feats.float(), coords, *sizes)
    assert_bit_equal(out, out32.to(torch.bfloat16), 'bf16 fwd = round(fp32 sequential sum)')
    rel = ((out.cpu().float() - out32).norm() / out32.norm()).item()
    assert rel <= 1e-2, rel
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    f = feats.to(cuda).requires_grad_(True)
    pkg.bev_pool(f, coords.to(cuda), *sizes).backward(g.to(cuda))
    assert_bit_equal(f.grad, ref.backward_gather(g, coords, *sizes), 'bf16 bwd (copy)')


@pytest.mark.parametrize('name', ['tiny_z4', 'det_z4'])
def test_lss_height_bins_z_collapse(pkg, cuda, synthetic, name):
    """Dz = 4 height bins: the (B, C*Dz, H, W) output of base.py:163
    (cat(unbind(2), 1): channel z*C + c) written directly, forward and
    backward bit-exact; points above or below the bins are dropped."""
    case = synthetic.make_case(name)
    dx, bx, nx = grid_of(case)
    assert int(nx[2]) == 4
    oi = check_index(pkg, case, cuda)
    assert 0 < int(oi.kept.sum()) < case.n_points
    check_fwd_bwd(pkg, case, cuda)


def test_lss_deterministic_and_stream(pkg, cuda, synthetic):
    case = synthetic.make_case('tiny')
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    geom, x = case.geom.to(cuda), case.x.to(cuda)
    a = module.bev_pool(geom, x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        b = module.bev_pool(geom, x)
    s.synchronize()
    assert torch.equal(a.cpu().view(torch.int32), b.cpu().view(torch.int32))


def check_planar(pkg, cuda, case, storage, view_of, seed=8):
    """Forward and backward through a channel-first (planar) view of
    ``storage``, bit-exact against the oracle on the same values; the
    gradient comes back in the planar layout."""
    leaf = storage.to(cuda).requires_grad_(True)
    view = view_of(leaf)
    assert not view.is_contiguous()
    from bevfusion_triton_amd.vtransform import planar_layout

    assert planar_layout(view) is not None
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    out = module.bev_pool(case.geom.to(cuda), view)
    dx, bx, nx = grid_of(case)
    xr = view_of(storage).detach().clone().requires_grad_(True)
    out_ref = ref.lss_bev_pool(case.geom, xr, dx, bx, nx)
    assert_bit_equal(out, out_ref, f'{case.name} planar forward')
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed))
    (out * g.to(cuda)).sum().backward()
    (out_ref * g).sum().backward()
    assert_bit_equal(view_of(leaf.grad), xr.grad, f'{case.name} planar backward')


def test_lss_channel_first_producer_view(pkg, cuda, synthetic):
    """x given as the reference's view of channel-first storage
    (depth_lss.py:94 rearrange) is transposed by one kernel and its gradient
    written back channel-first; both bit-exact."""
    case = synthetic.make_case('tiny')
    cf = case.x.permute(0, 1, 5, 2, 3, 4).contiguous()  # (B, N, C, D, fH, fW) storage
    check_planar(pkg, cuda, case, cf, lambda t: t.permute(0, 1, 3, 4, 5, 2))


def test_lss_channel_first_det(pkg, cuda, synthetic):
    """The planar path at the det shape (vector kernels)."""
    case = synthetic.make_case('det')
    cf = case.x.permute(0, 1, 5, 2, 3, 4).contiguous()
    check_planar(pkg, cuda, case, cf, lambda t: t.permute(0, 1, 3, 4, 5, 2))


def test_lss_channel_first_channel_slice(pkg, cuda, synthetic):
    """A planar view whose batch stride exceeds C*S (a channel slice of a
    wider tensor, as depth_lss.py:92 slices the depth-net output)."""
    case = synthetic.make_case('tiny')
    B, N, D, fH, fW, C = case.x.shape
    wide = torch.randn(B, N, C + 5, D, fH, fW, generator=torch.Generator().manual_seed(2))
    wide[:, :, 2:2 + C] = case.x.permute(0, 1, 5, 2, 3, 4)
    check_planar(pkg, cuda, case, wide, lambda t: t[:, :, 2:2 + C].permute(0, 1, 3, 4, 5, 2))


def test_lss_channel_first_odd_channels(pkg, cuda, synthetic):
    """C = 6 takes the element-wise planar kernels (no 16-byte form)."""
    case = synthetic.make_case('tiny', features=False)
    B, N, D, fH, fW = case.geom.shape[:5]
    cf = torch.randn(B, N, 6, D, fH, fW, generator=torch.Generator().manual_seed(4))
    check_planar(pkg, cuda, case, cf, lambda t: t.permute(0, 1, 3, 4, 5, 2))


def test_lss_all_points_dropped(pkg, cuda, synthetic):
    """Every point outside the grid: a zero map, zero gradients (the
    reference's empty x[kept] pooled by index_add_ into zeros)."""
    case = synthetic.make_case('tiny')
    geom = case.geom.clone()
    geom[..., 0] += 1000.0
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    x = case.x.to(cuda).requires_grad_(True)
    out = module.bev_pool(geom.to(cuda), x)
    dx, bx, nx = grid_of(case)
    assert_bit_equal(out, ref.lss_bev_pool(geom, case.x, dx, bx, nx), 'all dropped forward')
    out.sum().backward()
    assert int(torch.count_nonzero(x.grad)) == 0
    B, N, D, fH, fW = geom.shape[:5]
    depth = torch.rand(B * N, D, fH, fW, device=cuda).requires_grad_(True)
    context = torch.rand(B * N, 16, fH, fW, device=cuda).requires_grad_(True)
    out_d = module.bev_pool_depth(geom.to(cuda), depth, context)
    assert int(torch.count_nonzero(out_d)) == 0
    out_d.sum().backward()
    assert int(torch.count_nonzero(depth.grad)) == 0 and int(torch.count_nonzero(context.grad)) == 0


@pytest.mark.parametrize('BN,C,S,extra', [
    (3, 80, 332, 0),       # tiled, last tile of 12 points
    (2, 4, 68, 0),         # tiled, one 16-byte piece per row
    (2, 128, 196, 0),      # tiled, widest row
    (1, 20, 64, 3),        # tiled, channel slice of a wider tensor (channel stride > S)
    (2, 132, 100, 0),      # wider than the tile: register transpose
    (2, 6, 50, 0),         # C % 4 != 0: element-wise form
])
def test_planar_rows_transpose(pkg, cuda, BN, C, S, extra):
    """planar (BN, C, S) -> (BN*S, C) rows is an exact copy: compared with
    torch's permute at partial tiles, every tile width and both fallbacks."""
    from bevfusion_triton_amd import _pipeline as P

    g = torch.Generator().manual_seed(C + S)
    wide = torch.randn(BN, C + extra, S, generator=g).to(cuda)
    src = wide[:, extra:]
    rows = P.planar_rows(src)
    torch.cuda.synchronize()
    exp = src.permute(0, 2, 1).reshape(BN * S, C)
    assert_bit_equal(rows, exp, f'planar rows BN={BN} C={C} S={S}')


@pytest.mark.parametrize('seed', [11, 12, 13])
def test_lss_random_rigs(pkg, cuda, synthetic, seed):
    """Seeded jittered rigs (+-20 deg yaw, +-1 m translation per camera), an
    off-centre grid with unequal x/y cells and two height bins, 5% of the
    points pushed out of the grid and points just below its low x edge, on a
    16 x 44 frustum: indices and fp32 forward/backward bit-exact."""
    import dataclasses

    spec = dataclasses.replace(
        synthetic.CASES['det'], image=(128, 352), feature=(16, 44), focal=280.0,
        yaw_jitter_deg=20.0, trans_jitter_m=1.0, xbound=(-40.0, 56.0, 0.4),
        ybound=(-60.0, 36.0, 0.32), zbound=(-4.0, 4.0, 4.0), channels=20, oob_fraction=0.05,
        edge_points=16)
    geom = synthetic.make_geometry(spec, seed=seed)
    x = synthetic.make_features(spec, seed=seed)
    case = synthetic.Case(f'rig{seed}', spec, geom, x, spec.xbound, spec.ybound, spec.zbound)
    oi = check_index(pkg, case, cuda)
    assert 0 < int(oi.kept.sum()) < case.n_points
    check_fwd_bwd(pkg, case, cuda, seed=seed)


@pytest.mark.parametrize('dtype,autocast', [(torch.bfloat16, False), (torch.float16, False),
                                            (torch.bfloat16, True)])
def test_force_fp32_half_inputs(pkg, cuda, synthetic, dtype, autocast):
    """``@force_fp32`` on ``BaseTransform.bev_pool`` (models/helper/amp.py:35-67,
    models/vtransforms/base.py:131): half-precision x and geometry are cast
    to fp32 and pooled with autocast disabled, at the det shape.  The output
    is fp32 and bit-exact against the oracle on the upcast values; x's
    gradient comes back in x's dtype (autograd of the cast), equal to the
    oracle's fp32 gradient rounded to that dtype.  Running under
    torch.autocast changes nothing."""
    case = synthetic.make_case('det')
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    xh = case.x.to(dtype)
    gh = case.geom.to(dtype)
    x = xh.to(cuda).requires_grad_(True)
    with torch.autocast('cuda', dtype=dtype, enabled=autocast):
        out = module.bev_pool(gh.to(cuda), x)
    assert out.dtype == torch.float32
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(31))
    out.backward(g.to(cuda))
    torch.cuda.synchronize()
    assert x.grad.dtype == dtype
    dx, bx, nx = grid_of(case)
    xr = xh.float().requires_grad_(True)
    out_ref = ref.lss_bev_pool(gh.float(), xr, dx, bx, nx)
    out_ref.backward(g)
    assert_bit_equal(out, out_ref, f'{dtype} x: fp32 forward')
    assert_bit_equal(x.grad, xr.grad.to(dtype), f'{dtype} x: gradient in x dtype')


@pytest.mark.parametrize('layout', ['aligned', 'offset', 'batch2'])
def test_quantize_edges_golden(pkg, cuda, layout):
    """The quantisation's edge cases (tests/golden/quantize_edges.json, the
    same vectors the CPU oracles are held to) through the HIP quantise kernel:
    q in (-1, 0) kept as cell 0, q rounding up to the upper face dropped,
    height bounds, NaN / +inf / -inf coordinates dropped.  Ranks and kept mask
    as the vectors state.  Layouts: 16-byte aligned geometry (vector loads), a
    view starting 12 bytes into its storage (scalar loads), and the points
    repeated over a batch of 2 (ranks of batch 1 offset by one grid)."""
    q = json.loads((GOLDEN / 'quantize_edges.json').read_text())
    g = torch.from_numpy(
        np.array([p['geom_f32_bits'] for p in q['points']], dtype=np.uint32).view(np.float32))
    grid = q['grid']
    dx, bx, nx = ref.gen_dx_bx(grid['xbound'], grid['ybound'], grid['zbound'])
    want = [p['rank'] for p in q['points']]
    n_cells = int(nx[0] * nx[1] * nx[2])
    if layout == 'batch2':
        geom = torch.stack([g, g]).view(2, 1, 1, 1, -1, 3)
        want = want + [r + n_cells if r >= 0 else -1 for r in want]
    else:
        geom = g.view(1, 1, 1, 1, -1, 3)
    geom = geom.to(cuda)
    if layout == 'offset':
        buf = torch.zeros(geom.numel() + 3, dtype=torch.float32, device=cuda)
        buf[3:] = geom.reshape(-1)
        geom = buf[3:].view(geom.shape)
        assert geom.data_ptr() % 16 == 12
    exp = pkg.LSSIndexExport(geom, dx, bx, nx)
    assert exp.rank.cpu().tolist() == want
    assert exp.kept.cpu().tolist() == [r >= 0 for r in want]
    kept = [r for r in want if r >= 0]
    assert exp.sorted_ranks.cpu().tolist() == sorted(kept)
    assert exp.index.n_points == len(want)
