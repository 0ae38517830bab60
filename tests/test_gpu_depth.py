"""GPU parity of the depth-weighted pooling (``lss_bev_pool_depth``: the LSS
feature ``depth (x) context`` of ``depth_lss.py:91-94`` pooled without being
materialised) against the CPU oracle.

Bar: the forward map bit-exact against the oracle in fp32 (the product is one
fp32 multiplication per element and the sums keep point order, exactly as the
reference computes them).  Gradients: the reference's own fp32 gradients are
reductions whose order torch does not fix, so the GPU's are held to the
rounding-error bound of an n-term fp32 sum, |err| <= (n + 2) * 2^-24 * sum|terms|
per element (n = C for depth, n = D for context), against the float64 oracle,
and to a relative norm error of at most 1e-5.
"""
from __future__ import annotations

import pytest
import torch

from oracle import torch_fallback as ref
from test_gpu_op import assert_bit_equal

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


@pytest.fixture(scope='module')
def synthetic(pkg):
    from bevfusion_triton_amd import synthetic

    return synthetic


def depth_context(spec, seed=0, extra_channels=0):
    """Softmaxed depth (BN, D, fH, fW) and context (BN, C, fH, fW) as the
    depth net produces them; with ``extra_channels`` the context is a slice
    of a wider (BN, D + C + extra, fH, fW) tensor, as ``x[:, D:D+C]``."""
    from bevfusion_triton_amd.synthetic import YAWS_DEG

    BN = spec.batch * len(YAWS_DEG)
    fH, fW = spec.feature
    D = torch.arange(*spec.dbound, dtype=torch.float).shape[0]
    C = spec.channels
    gen = torch.Generator().manual_seed(seed)
    net = torch.randn(BN, D + C + extra_channels, fH, fW, generator=gen)
    depth = net[:, :D].softmax(dim=1)
    context = net[:, D:D + C]
    return depth, context, net


def check_depth_pool(pkg, name, synthetic, cuda, *, grads=True, seed=0, extra_channels=0):
    case = synthetic.make_case(name, features=False)
    spec = case.spec
    depth, context, net = depth_context(spec, seed, extra_channels)
    dx, bx, nx = ref.gen_dx_bx(case.xbound, case.ybound, case.zbound)
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    dg = depth.to(cuda).requires_grad_(grads)
    if extra_channels:
        # the slice of the device-resident net output, strided batch axis
        D = depth.shape[1]
        cg = net.to(cuda)[:, D:D + context.shape[1]]
        assert not cg.is_contiguous()
        assert not grads
    else:
        cg = context.to(cuda).requires_grad_(grads)
    out = module.bev_pool_depth(case.geom.to(cuda), dg, cg)
    out_ref = ref.lss_bev_pool_depth(case.geom, depth, context, dx, bx, nx)
    assert out.shape == out_ref.shape and out.is_contiguous()
    assert_bit_equal(out, out_ref, f'{name} depth-weighted forward')
    if not grads:
        return out
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 31))
    (out * g.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    d64 = depth.double().requires_grad_(True)
    c64 = context.double().requires_grad_(True)
    ref.lss_bev_pool_depth(case.geom, d64, c64, dx, bx, nx, dtype=torch.float64).mul(
        g.double()).sum().backward()
    # sum of |terms| per gradient element: the same sums over absolute values
    a64 = depth.double().abs().requires_grad_(True)
    b64 = context.double().abs().requires_grad_(True)
    ref.lss_bev_pool_depth(case.geom, a64, b64, dx, bx, nx, dtype=torch.float64).mul(
        g.double().abs()).sum().backward()
    D, C = depth.shape[1], context.shape[1]
    for got, exact, mag, n, what in ((dg.grad, d64.grad, a64.grad, C, 'grad depth'),
                                     (cg.grad, c64.grad, b64.grad, D, 'grad context')):
        got = got.cpu().double()
        err = (got - exact).abs()
        bound = (n + 2) * U * mag + 1e-30
        worst = (err / bound).max().item()
        assert worst <= 1.0, f'{name} {what}: error {worst:.3f} x the fp32 summation bound'
        rel = ((got - exact).norm() / exact.norm()).item()
        assert rel <= 1e-5, f'{name} {what}: relative error {rel:.2e}'
    return out


@pytest.mark.parametrize('name', ['tiny', 'det'])
def test_depth_pool_single_sample(pkg, cuda, synthetic, name):
    check_depth_pool(pkg, name, synthetic, cuda)


def test_depth_pool_train_batch4(pkg, cuda, synthetic):
    check_depth_pool(pkg, 'train', synthetic, cuda, seed=3)


def test_depth_pool_height_bins(pkg, cuda, synthetic):
    """Dz = 4: the fused path writes the (B, C*Dz, H, W) collapse directly."""
    check_depth_pool(pkg, 'tiny_z4', synthetic, cuda)


def test_depth_pool_hires_out_of_bounds_forward(pkg, cuda, synthetic):
    """720x720 grid, B=2, 10% of the points out of bounds (forward only: the
    float64 gradient oracle at 4.3 M points x 80 channels is left to the
    smaller cases)."""
    check_depth_pool(pkg, 'hires', synthetic, cuda, grads=False)


def test_depth_pool_context_slice(pkg, cuda, synthetic):
    """context given as the slice x[:, D:D+C] of a wider depth-net output
    (strided batch axis) pools without a copy and identically."""
    check_depth_pool(pkg, 'tiny', synthetic, cuda, grads=False, extra_channels=7)


def test_depth_pool_matches_materialised_feature(pkg, cuda, synthetic):
    """The fused path equals pooling the materialised feature on the GPU."""
    case = synthetic.make_case('det', features=False)
    depth, context, _ = depth_context(case.spec, 5)
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    geom, d, c = case.geom.to(cuda), depth.to(cuda), context.to(cuda)
    fused = module.bev_pool_depth(geom, d, c)
    B, N = case.geom.shape[:2]
    x = ref.lss_feature(d, c, B, N).contiguous()
    assert_bit_equal(fused, module.bev_pool(geom, x), 'fused vs materialised')


def test_depth_pool_odd_channels(pkg, cuda, synthetic):
    """C = 6 (not a multiple of 4) takes the materialised route, same result."""
    case = synthetic.make_case('tiny', features=False)
    depth, context, _ = depth_context(case.spec, 2)
    context = context[:, :6]
    dx, bx, nx = ref.gen_dx_bx(case.xbound, case.ybound, case.zbound)
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    out = module.bev_pool_depth(case.geom.to(cuda), depth.to(cuda), context.to(cuda))
    assert_bit_equal(out, ref.lss_bev_pool_depth(case.geom, depth, context, dx, bx, nx),
                     'C=6 forward')


def test_depth_pool_deterministic(pkg, cuda, synthetic):
    case = synthetic.make_case('tiny', features=False)
    depth, context, _ = depth_context(case.spec, 1)
    module = pkg.BevPoolTransform(case.xbound, case.ybound, case.zbound).to(cuda)
    geom, d, c = case.geom.to(cuda), depth.to(cuda), context.to(cuda)
    runs = []
    for _ in range(2):
        dd = d.clone().requires_grad_(True)
        cc = c.clone().requires_grad_(True)
        out = module.bev_pool_depth(geom, dd, cc)
        out.sum().backward()
        runs.append((out.detach(), dd.grad, cc.grad))
    for a, b in zip(*runs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
