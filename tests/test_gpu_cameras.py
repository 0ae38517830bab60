"""GPU parity of the geometry fused into the quantisation
(``lss_index_cameras`` / ``BevPoolTransform.index_cameras``: base.py:82-126
computed per point inside the quantise kernel) and of its index cache.

Bar (boundary policy): the GPU computes the geometry in fp32 with every
operation rounded once, torch's batched matmul rounds its own way, so a
point within rounding distance of a voxel face may fall on either side.
Every point whose float64 position is more than 1e-3 cell from every face
must get exactly the reference's rank (torch fp32 get_geometry, then the
reference quantisation); the others may differ, and at most 1e-4 of all
points (or 8) do.  Pooling on the camera index is then bit-exact against the
oracle pooling with the same ranks, forward and backward, for channel-last
features and for the fused depth (x) context path.
"""
from __future__ import annotations

import pytest
import torch

from oracle import torch_fallback as ref
from test_gpu_op import assert_bit_equal

pytestmark = pytest.mark.gpu

FACE_EPS = 1e-3


@pytest.fixture(scope='module')
def synthetic(pkg):
    from bevfusion_triton_amd import synthetic

    return synthetic


def to_dev(inp, cuda):
    return {k: (v.to(cuda) if v is not None else None) for k, v in inp.items()}


def check_ranks(pkg, cuda, spec, inp, module):
    dx, bx, nx = ref.gen_dx_bx(spec.xbound, spec.ybound, spec.zbound)
    ci = module.index_cameras(**to_dev(inp, cuda))
    rank = ci.index.rank.cpu().long()
    oi = ref.lss_index(ref.get_geometry(**inp), dx, bx, nx)
    q64 = ((ref.get_geometry(**inp, dtype=torch.float64) - (bx.double() - dx.double() / 2))
           / dx.double()).reshape(-1, 3)
    near = ((q64 - q64.round()).abs() < FACE_EPS).any(-1)
    mism = rank != oi.rank
    n = rank.numel()
    assert not bool((mism & ~near).any()), f'{int((mism & ~near).sum())} ranks differ off-face'
    assert int(mism.sum()) <= max(8, int(1e-4 * n)), int(mism.sum())
    assert 0 < int((rank >= 0).sum()) < n
    return ci, rank


@pytest.mark.parametrize('name,augment', [('tiny', False), ('tiny', True), ('det', True),
                                          ('train', True), ('tiny_z4', True)])
def test_camera_index_ranks(pkg, cuda, synthetic, name, augment):
    spec = synthetic.CASES[name]
    inp = synthetic.camera_inputs(spec, seed=7, augment=augment)
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    check_ranks(pkg, cuda, spec, inp, module)


@pytest.mark.parametrize('name', ['tiny_z4', 'det'])
def test_camera_index_pooling(pkg, cuda, synthetic, name):
    spec = synthetic.CASES[name]
    inp = synthetic.camera_inputs(spec, seed=11, augment=True)
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    ci, rank = check_ranks(pkg, cuda, spec, inp, module)
    dx, bx, nx = ref.gen_dx_bx(spec.xbound, spec.ybound, spec.zbound)
    x = synthetic.make_features(spec)
    C = x.shape[-1]
    xg = x.to(cuda).requires_grad_(True)
    out = module.bev_pool(ci, xg)
    xr = x.clone().requires_grad_(True)
    out_ref = ref.pool_ranks(xr.reshape(-1, C), rank, spec.batch, nx)
    assert_bit_equal(out, out_ref, f'{name} forward on the camera index')
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    (out * g.to(cuda)).sum().backward()
    (out_ref * g).sum().backward()
    assert_bit_equal(xg.grad, xr.grad, f'{name} backward on the camera index')


def test_camera_index_depth_path(pkg, cuda, synthetic):
    spec = synthetic.CASES['tiny_z4']
    inp = synthetic.camera_inputs(spec, seed=13, augment=True)
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    ci, rank = check_ranks(pkg, cuda, spec, inp, module)
    dx, bx, nx = ref.gen_dx_bx(spec.xbound, spec.ybound, spec.zbound)
    B, N, D, fH, fW = ci.shape
    gen = torch.Generator().manual_seed(3)
    depth = torch.randn(B * N, D, fH, fW, generator=gen).softmax(1)
    context = torch.randn(B * N, spec.channels, fH, fW, generator=gen)
    out = module.bev_pool_depth(ci, depth.to(cuda), context.to(cuda))
    x = ref.lss_feature(depth, context, B, N)
    out_ref = ref.pool_ranks(x.reshape(-1, spec.channels), rank, B, nx)
    assert_bit_equal(out, out_ref, 'depth path on the camera index')


def test_camera_index_cache(pkg, cuda, synthetic):
    """cache_index: the same tensors at the same version reuse the index;
    an in-place change or a new tensor recomputes it; off by default."""
    spec = synthetic.CASES['tiny']
    inp = to_dev(synthetic.camera_inputs(spec, seed=7, augment=True), cuda)
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound,
                                  cache_index=True).to(cuda)
    a = module.index_cameras(**inp)
    assert module.index_cameras(**inp) is a
    inp['post_trans'].add_(0.0)  # version bump
    b = module.index_cameras(**inp)
    assert b is not a
    assert module.index_cameras(**inp) is b
    inp2 = dict(inp, camera2lidar_trans=inp['camera2lidar_trans'].clone())
    c = module.index_cameras(**inp2)
    assert c is not b
    assert torch.equal(c.index.rank, b.index.rank)
    plain = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    assert plain.index_cameras(**inp) is not plain.index_cameras(**inp)


def _small_rig(B, N, D, fH, fW, seed):
    """Cameras of a tiny frustum (D*fH*fW points per camera), random poses
    and augmentations, on a small grid."""
    g = torch.Generator().manual_seed(seed)
    ds = torch.linspace(2.0, 12.0, D)
    us = torch.linspace(0, 63, fW)
    vs = torch.linspace(0, 31, fH)
    fr = torch.stack(torch.broadcast_tensors(us.view(1, 1, fW), vs.view(1, fH, 1),
                                             ds.view(D, 1, 1)), -1).contiguous()
    yaw = torch.rand(B, N, generator=g) * 6.283
    c, s = torch.cos(yaw), torch.sin(yaw)
    z, o = torch.zeros_like(c), torch.ones_like(c)
    rots = torch.stack((torch.stack((s, z, c), -1), torch.stack((-c, z, s), -1),
                        torch.stack((z, -o, z), -1)), -2)
    trans = torch.rand(B, N, 3, generator=g) - 0.5
    K = torch.tensor([[40.0, 0.0, 32.0], [0.0, 40.0, 16.0], [0.0, 0.0, 1.0]]).repeat(B, N, 1, 1)
    pr = torch.eye(3).repeat(B, N, 1, 1) * (0.95 + 0.1 * torch.rand(B, N, 1, 1, generator=g))
    pr[..., 2, 2] = 1.0
    pt = torch.rand(B, N, 3, generator=g) * 4.0
    pt[..., 2] = 0.0
    return dict(frustum=fr, camera2lidar_rots=rots, camera2lidar_trans=trans, intrins=K,
                post_rots=pr, post_trans=pt)


@pytest.mark.parametrize('extra', ['none', 'rots', 'trans', 'both'])
def test_camera_index_many_cameras_per_block(pkg, cuda, extra):
    """8 points per camera: one 2048-point block spans up to 256 cameras, more
    than the 16 it stages in LDS, so the per-point table path runs; extra_rots /
    extra_trans given alone take identity / zero for the other."""
    from bevfusion_triton_amd.synthetic import RigSpec

    B, N = 4, 40
    inp = _small_rig(B, N, 2, 2, 2, seed=21)
    g = torch.Generator().manual_seed(22)
    yaw = (torch.rand(B, generator=g) - 0.5) * 0.3
    er = torch.zeros(B, 3, 3)
    er[:, 0, 0], er[:, 0, 1], er[:, 1, 0], er[:, 1, 1] = (torch.cos(yaw), -torch.sin(yaw),
                                                          torch.sin(yaw), torch.cos(yaw))
    er[:, 2, 2] = 1.0
    et = torch.rand(B, 3, generator=g) - 0.5
    inp['extra_rots'] = er if extra in ('rots', 'both') else None
    inp['extra_trans'] = et if extra in ('trans', 'both') else None
    spec = RigSpec(xbound=(-14.0, 14.0, 0.7), ybound=(-14.0, 14.0, 0.7),
                   zbound=(-10.0, 10.0, 20.0))
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    check_ranks(pkg, cuda, spec, inp, module)


def test_camera_index_on_side_stream(pkg, cuda, synthetic):
    """The index built on a side stream while the main stream runs other work
    (the depth net, in a model), handed over with an event: same bits as the
    index built in line."""
    spec = synthetic.CASES['det']
    inp = to_dev(synthetic.camera_inputs(spec, seed=9, augment=True), cuda)
    module = pkg.BevPoolTransform(spec.xbound, spec.ybound, spec.zbound).to(cuda)
    module.grid()
    x = synthetic.make_features(spec, device=cuda)
    ref_out = module.bev_pool(module.index_cameras(**inp), x)
    side = torch.cuda.Stream()
    main = torch.cuda.current_stream()
    side.wait_stream(main)
    with torch.cuda.stream(side):
        ci = module.index_cameras(**inp)
        ready = torch.cuda.Event()
        ready.record(side)
    busy = torch.randn(4096, 4096, device=cuda)
    for _ in range(4):
        busy = busy @ busy.t() * 1e-4  # stand-in for the producer on the main stream
    main.wait_event(ready)
    for t in (ci.index.rank, ci.index.keys, ci.index.cell_start, ci.index.cell_end, ci.index.meta):
        t.record_stream(main)
    out = module.bev_pool(ci, x)
    assert_bit_equal(out, ref_out, 'index built on a side stream')
