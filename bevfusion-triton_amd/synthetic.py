"""Synthetic LSS workloads for tests and benchmarks (not on the pooling path).

Restates, in torch fp32 on the CPU, how the reference builds the pooling
inputs, so that the geometry has the real frustum structure (rays from six
cameras, dense near the car, sparse far away):
  * frustum         ``models/vtransforms/base.py:67-80`` (create_frustum)
  * geometry        ``models/vtransforms/base.py:82-126`` (get_geometry with
                    identity image/lidar augmentation)
  * feature values  ``models/vtransforms/depth_lss.py:91-94``: softmax over
                    depth logits ~N(0,1) times context ~N(0,1)

The camera rig: six cameras at yaw 0, +-55, +-110, 180 degrees, 1.5 m high,
pinhole intrinsics with the principal point at the image centre.  Named
cases follow the five benchmark configurations (det, seg, train, bf16,
hires) plus a small ``tiny`` case for smoke tests and two cases with four
height bins (``tiny_z4``, ``det_z4``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

YAWS_DEG = (0.0, 55.0, -55.0, 110.0, -110.0, 180.0)


@dataclass
class RigSpec:
    batch: int = 1
    image: tuple = (256, 704)  # (iH, iW)
    feature: tuple = (32, 88)  # (fH, fW)
    focal: float = 560.0
    dbound: tuple = (1.0, 60.0, 0.5)
    xbound: tuple = (-54.0, 54.0, 0.3)
    ybound: tuple = (-54.0, 54.0, 0.3)
    zbound: tuple = (-10.0, 10.0, 20.0)
    channels: int = 80
    yaw_jitter_deg: float = 0.0  # per sample and camera, uniform +-
    trans_jitter_m: float = 0.0  # per sample, camera and axis, uniform +-
    oob_fraction: float = 0.0  # fraction of points pushed out of the grid
    edge_points: int = 0  # points placed at q in (-1, 0) on the x axis
    dtype: torch.dtype = torch.float32


CASES = {
    'tiny': RigSpec(image=(64, 176), feature=(8, 22), focal=140.0, dbound=(1.0, 60.0, 2.0),
                    xbound=(-54.0, 54.0, 1.2), ybound=(-54.0, 54.0, 1.2), channels=16,
                    edge_points=8),
    'det': RigSpec(),
    'seg': RigSpec(xbound=(-51.2, 51.2, 0.4), ybound=(-51.2, 51.2, 0.4)),
    'train': RigSpec(batch=4, yaw_jitter_deg=5.0, trans_jitter_m=0.2),
    'bf16': RigSpec(batch=8, dtype=torch.bfloat16),
    'hires': RigSpec(batch=2, image=(512, 1408), feature=(64, 176), focal=1120.0,
                     xbound=(-54.0, 54.0, 0.15), ybound=(-54.0, 54.0, 0.15),
                     oob_fraction=0.10, edge_points=64),
    # several height bins (Z-collapse to C*Dz channels); points above/below drop
    'tiny_z4': RigSpec(image=(64, 176), feature=(8, 22), focal=140.0, dbound=(1.0, 60.0, 2.0),
                       xbound=(-54.0, 54.0, 1.2), ybound=(-54.0, 54.0, 1.2),
                       zbound=(-3.0, 3.0, 1.5), channels=16, edge_points=8),
    'det_z4': RigSpec(zbound=(-3.0, 3.0, 1.5)),
}


def create_frustum(image, feature, dbound):
    """``base.py:67-80``: (D, fH, fW, 3) of (u, v, depth)."""
    iH, iW = image
    fH, fW = feature
    ds = torch.arange(*dbound, dtype=torch.float).view(-1, 1, 1).expand(-1, fH, fW)
    D = ds.shape[0]
    xs = torch.linspace(0, iW - 1, fW, dtype=torch.float).view(1, 1, fW).expand(D, fH, fW)
    ys = torch.linspace(0, iH - 1, fH, dtype=torch.float).view(1, fH, 1).expand(D, fH, fW)
    return torch.stack((xs, ys, ds), -1)


def camera_rig(spec: RigSpec, gen: torch.Generator):
    """camera2lidar rotations (B, 6, 3, 3), translations (B, 6, 3) and
    intrinsics (B, 6, 3, 3).  Camera axes in the lidar frame: right
    (sin y, -cos y, 0), down (0, 0, -1), forward (cos y, sin y, 0)."""
    B, N = spec.batch, len(YAWS_DEG)
    yaw = torch.tensor(YAWS_DEG, dtype=torch.float64).repeat(B, 1)
    if spec.yaw_jitter_deg:
        yaw = yaw + (torch.rand(B, N, generator=gen, dtype=torch.float64) * 2 - 1) * spec.yaw_jitter_deg
    psi = yaw * math.pi / 180.0
    c, s = torch.cos(psi), torch.sin(psi)
    zero = torch.zeros_like(c)
    right = torch.stack((s, -c, zero), -1)
    down = torch.stack((zero, zero, -torch.ones_like(c)), -1)
    fwd = torch.stack((c, s, zero), -1)
    rots = torch.stack((right, down, fwd), -1).float()  # columns = camera axes
    trans = torch.tensor([0.0, 0.0, 1.5]).repeat(B, N, 1)
    if spec.trans_jitter_m:
        trans = trans + (torch.rand(B, N, 3, generator=gen) * 2 - 1) * spec.trans_jitter_m
    iH, iW = spec.image
    K = torch.tensor([[spec.focal, 0.0, iW / 2.0], [0.0, spec.focal, iH / 2.0], [0.0, 0.0, 1.0]])
    intrins = K.repeat(B, N, 1, 1)
    return rots, trans.float(), intrins


def get_geometry(frustum, rots, trans, intrins):
    """``base.py:82-126`` with identity post-rotation/translation and lidar
    augmentation: unproject (u*d, v*d, d), rotate by R K^-1, translate."""
    B, N = trans.shape[:2]
    pts = frustum.unsqueeze(-1)  # D fH fW 3 1
    pts = torch.cat((pts[..., :2, :] * pts[..., 2:3, :], pts[..., 2:3, :]), -2)
    combine = torch.linalg.solve(intrins.transpose(-1, -2), rots.transpose(-1, -2)).transpose(-1, -2)
    out = combine.reshape(B, N, 1, 1, 1, 3, 3).matmul(pts).squeeze(-1)
    return out + trans.reshape(B, N, 1, 1, 1, 3)


def camera_inputs(spec: RigSpec, seed: int = 1, augment: bool = True) -> dict:
    """The arguments of ``get_geometry`` (``base.py:82-126``) for the rig:
    frustum, camera2lidar rotations/translations, intrinsics and, with
    ``augment``, an image augmentation per camera (post_rots = scale s in
    [0.95, 1.05] times a rotation in +-5 degrees, post_trans a crop offset
    of up to 8 px) and a lidar augmentation per sample (extra_rots a yaw in
    +-10 degrees, extra_trans up to 0.5 m); identity/zero otherwise."""
    gen = torch.Generator().manual_seed(seed)
    frustum = create_frustum(spec.image, spec.feature, spec.dbound)
    rots, trans, intrins = camera_rig(spec, gen)
    B, N = spec.batch, len(YAWS_DEG)
    out = {'frustum': frustum, 'camera2lidar_rots': rots, 'camera2lidar_trans': trans,
           'intrins': intrins}
    if augment:
        s = 0.95 + 0.1 * torch.rand(B, N, generator=gen)
        th = (torch.rand(B, N, generator=gen) * 2 - 1) * (5.0 * math.pi / 180.0)
        pr = torch.zeros(B, N, 3, 3)
        pr[..., 0, 0] = s * torch.cos(th)
        pr[..., 0, 1] = -s * torch.sin(th)
        pr[..., 1, 0] = s * torch.sin(th)
        pr[..., 1, 1] = s * torch.cos(th)
        pr[..., 2, 2] = 1.0
        pt = torch.zeros(B, N, 3)
        pt[..., :2] = (torch.rand(B, N, 2, generator=gen) * 2 - 1) * 8.0
        yaw = (torch.rand(B, generator=gen) * 2 - 1) * (10.0 * math.pi / 180.0)
        er = torch.zeros(B, 3, 3)
        er[:, 0, 0] = torch.cos(yaw)
        er[:, 0, 1] = -torch.sin(yaw)
        er[:, 1, 0] = torch.sin(yaw)
        er[:, 1, 1] = torch.cos(yaw)
        er[:, 2, 2] = 1.0
        et = (torch.rand(B, 3, generator=gen) * 2 - 1) * 0.5
        out.update(post_rots=pr, post_trans=pt, extra_rots=er, extra_trans=et)
    else:
        out.update(post_rots=torch.eye(3).repeat(B, N, 1, 1), post_trans=torch.zeros(B, N, 3),
                   extra_rots=None, extra_trans=None)
    return out


@dataclass
class Case:
    name: str
    spec: RigSpec
    geom: torch.Tensor  # (B, N, D, fH, fW, 3) fp32 (CPU)
    x: torch.Tensor | None  # (B, N, D, fH, fW, C) channel-last contiguous
    xbound: tuple = field(default=())
    ybound: tuple = field(default=())
    zbound: tuple = field(default=())

    @property
    def n_points(self) -> int:
        return self.geom[..., 0].numel()


def make_geometry(spec: RigSpec, seed: int = 1) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    frustum = create_frustum(spec.image, spec.feature, spec.dbound)
    rots, trans, intrins = camera_rig(spec, gen)
    geom = get_geometry(frustum, rots, trans, intrins).contiguous()
    flat = geom.view(-1, 3)
    n = flat.shape[0]
    if spec.oob_fraction:
        k = int(n * spec.oob_fraction)
        sel = torch.randperm(n, generator=gen)[:k]
        sign = torch.where(torch.rand(k, generator=gen) < 0.5, -1.0, 1.0)
        flat[sel, 0] += sign * (60.0 + 140.0 * torch.rand(k, generator=gen))
    if spec.edge_points:
        # x just below the grid's low edge: q in (-1, 0) truncates to cell 0
        sel = torch.randperm(n, generator=gen)[: spec.edge_points]
        frac = 0.05 + 0.9 * torch.rand(spec.edge_points, generator=gen)
        flat[sel, 0] = torch.tensor(spec.xbound[0], dtype=torch.float32) - frac * spec.xbound[2]
        flat[sel, 1] = 0.5
        flat[sel, 2] = 0.0
    return geom


def make_features(spec: RigSpec, device='cpu', seed: int = 0) -> torch.Tensor:
    """x = softmax_D(logits) * context in (B, N, D, fH, fW, C) channel-last
    contiguous storage (values identical to the reference's
    ``rearrange(x, '(b n) c d h w -> b n d h w c')`` view)."""
    B, N = spec.batch, len(YAWS_DEG)
    fH, fW = spec.feature
    D = torch.arange(*spec.dbound, dtype=torch.float).shape[0]
    C = spec.channels
    gen = torch.Generator(device=device).manual_seed(seed)
    logits = torch.randn(B * N, D, fH, fW, generator=gen, device=device)
    context = torch.randn(B * N, C, fH, fW, generator=gen, device=device)
    depth = logits.softmax(dim=1)
    # (B*N, D, fH, fW, C) = depth[:, d, h, w] * context[:, c, h, w]
    x = depth.unsqueeze(-1) * context.permute(0, 2, 3, 1).unsqueeze(1)
    # the broadcast product follows its inputs' memory order; force channel-last
    x = x.contiguous().view(B, N, D, fH, fW, C)
    if spec.dtype != torch.float32:
        x = x.to(spec.dtype)
    return x


def make_case(name: str, device='cpu', seed: int = 0, features: bool = True) -> Case:
    """Geometry and (unless ``features`` is False: then ``x`` is None) the
    materialised feature of a named configuration."""
    spec = CASES[name]
    geom = make_geometry(spec)
    x = make_features(spec, device=device, seed=seed) if features else None
    return Case(name, spec, geom, x, spec.xbound, spec.ybound, spec.zbound)
