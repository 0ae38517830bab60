"""Pins the oracle's ``get_geometry`` (``oracle/torch_fallback.py``, restating
``models/vtransforms/base.py:82-126``) against a per-point float64 formula
written out independently (explicit inverse of the intrinsics, scalar
arithmetic), against the closed-form projection back onto the image for
identity augmentation, and shows a planted inverse-for-transpose mistake
is caught.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torch_fallback as ref


@pytest.fixture(scope='module')
def synthetic(pkg):
    from bevfusion_triton_amd import synthetic

    return synthetic


def brute_geometry(inp, stride=97):
    """float64 per point, every `stride`-th point: returns (flat index, xyz)."""
    fr = inp['frustum'].double().numpy()
    R = inp['camera2lidar_rots'].double().numpy()
    t = inp['camera2lidar_trans'].double().numpy()
    K = inp['intrins'].double().numpy()
    PR = inp['post_rots'].double().numpy()
    PT = inp['post_trans'].double().numpy()
    ER = None if inp['extra_rots'] is None else inp['extra_rots'].double().numpy()
    ET = None if inp['extra_trans'] is None else inp['extra_trans'].double().numpy()
    B, N = t.shape[:2]
    D, fH, fW = fr.shape[:3]
    out = []
    n_all = B * N * D * fH * fW
    for p in range(0, n_all, stride):
        cam, f = divmod(p, D * fH * fW)
        b, n = divmod(cam, N)
        d, hw = divmod(f, fH * fW)
        h, w = divmod(hw, fW)
        a = [fr[d, h, w, k] - PT[b, n, k] for k in range(3)]
        q = [sum(PR[b, n, k, i] * a[k] for k in range(3)) for i in range(3)]  # PR^T a
        c = [q[0] * q[2], q[1] * q[2], q[2]]
        M = R[b, n] @ np.linalg.inv(K[b, n])
        g = [sum(M[i, k] * c[k] for k in range(3)) + t[b, n, i] for i in range(3)]
        if ER is not None:
            g = [sum(ER[b, i, k] * g[k] for k in range(3)) for i in range(3)]
        if ET is not None:
            g = [g[i] + ET[b, i] for i in range(3)]
        out.append((p, g))
    return out


@pytest.mark.parametrize('augment', [False, True])
def test_get_geometry_brute_force(synthetic, augment):
    spec = synthetic.CASES['tiny']
    inp = synthetic.camera_inputs(spec, seed=3, augment=augment)
    geo = ref.get_geometry(**inp, dtype=torch.float64).reshape(-1, 3).numpy()
    for p, g in brute_geometry(inp):
        np.testing.assert_allclose(geo[p], g, rtol=1e-12, atol=1e-9)
    # the fp32 restatement stays within fp32 rounding of the float64 one
    geo32 = ref.get_geometry(**inp).reshape(-1, 3).double().numpy()
    np.testing.assert_allclose(geo32, geo, rtol=0, atol=1e-4)


def test_get_geometry_projects_back(synthetic):
    """Identity augmentation: K R^-1 (g - t) = d (u, v, 1) for every point."""
    spec = synthetic.CASES['tiny']
    inp = synthetic.camera_inputs(spec, seed=5, augment=False)
    geo = ref.get_geometry(**inp, dtype=torch.float64)
    R = inp['camera2lidar_rots'].double()
    t = inp['camera2lidar_trans'].double()
    K = inp['intrins'].double()
    B, N = t.shape[:2]
    rel = geo - t.view(B, N, 1, 1, 1, 3)
    cam = (K @ torch.linalg.inv(R)).view(B, N, 1, 1, 1, 3, 3).matmul(rel.unsqueeze(-1))
    cam = cam.squeeze(-1)
    fr = inp['frustum'].double()
    expect = torch.stack((fr[..., 0] * fr[..., 2], fr[..., 1] * fr[..., 2], fr[..., 2]), -1)
    torch.testing.assert_close(cam, expect.expand_as(cam), rtol=1e-10, atol=1e-9)


def test_planted_inverse_for_transpose_is_caught(synthetic):
    """The reference multiplies by post_rots^T (not its inverse); with a
    scaling augmentation the two differ and the brute force tells them apart."""
    spec = synthetic.CASES['tiny']
    inp = synthetic.camera_inputs(spec, seed=3, augment=True)
    bad = dict(inp)
    bad['post_rots'] = torch.linalg.inv(inp['post_rots']).transpose(-1, -2)  # inv used instead
    geo_bad = ref.get_geometry(**bad, dtype=torch.float64).reshape(-1, 3).numpy()
    mism = [not np.allclose(geo_bad[p], g, rtol=1e-9, atol=1e-7) for p, g in brute_geometry(inp)]
    assert any(mism)


def test_pool_ranks_equals_lss_bev_pool(synthetic):
    case = synthetic.make_case('tiny_z4')
    dx, bx, nx = ref.gen_dx_bx(case.xbound, case.ybound, case.zbound)
    idx = ref.lss_index(case.geom, dx, bx, nx)
    C = case.x.shape[-1]
    out = ref.pool_ranks(case.x.reshape(-1, C), idx.rank, case.geom.shape[0], nx)
    expect = ref.lss_bev_pool(case.geom, case.x, dx, bx, nx)
    assert torch.equal(out.view(torch.int32), expect.view(torch.int32))
