"""LSS view-transform pooling (geometry + camera features -> BEV) on MI355X.

Drop-in for the pooling half of ``models/vtransforms/base.py``:
  * :func:`gen_dx_bx`            -- ``base.py:19-23``
  * :class:`BevPoolTransform`    -- the ``dx``/``bx``/``nx`` parameters of
    ``BaseTransform.__init__`` (``base.py:57-60``) and its ``bev_pool(geom_feats, x)``
    method (``base.py:131-165``): quantise, batch index, kept mask,
    compaction, ``bev_pool``, Z-collapse;
  * :func:`lss_bev_pool`         -- the same as a function;
  * :func:`lss_bev_pool_depth`   -- the same for the LSS feature
    ``depth (x) context`` (``depth_lss.py:91-94``) without materialising it.

Everything between the geometry/feature tensors and the BEV map runs as HIP
kernels: the quantisation/kept-mask, the compaction (fused into the first
radix pass), the sort, the per-cell ranges, the pooled sums and the
Z-collapse (the output is written directly as (B, C*Dz, H, W)).  The gradient
flows to ``x`` only (the reference's ``.long()`` cuts it from the geometry),
with zero rows for dropped points, as autograd of ``x[kept]`` gives.

Like ``@force_fp32`` (``models/helper/amp.py:35-67``) the inputs are cast to
fp32 first.  ``x`` may be any (B, N, D, fH, fW, C) view: a channel-last
producer costs no copy; the reference's own view of channel-first storage
(``depth_lss.py:94``) is transposed into rows by one kernel (the copy
``base.py:136`` makes) and its gradient is written back channel-first without
a copy; other views are copied once.
"""
from __future__ import annotations

import weakref

import numpy as np
import torch
from torch import nn

from . import _pipeline as P


def gen_dx_bx(xbound, ybound, zbound):
    """``base.py:19-23``: dx = step, bx = lo + step/2 (double -> fp32),
    nx = int64((hi - lo) / step) with the division in double."""
    dx = torch.Tensor([row[2] for row in [xbound, ybound, zbound]])
    bx = torch.Tensor([row[0] + row[2] / 2.0 for row in [xbound, ybound, zbound]])
    nx = torch.LongTensor([(row[1] - row[0]) / row[2] for row in [xbound, ybound, zbound]])
    return dx, bx, nx


def host_grid(dx, bx, nx):
    """(offset, dx, nx) on the host: offset = bx - dx/2 evaluated with torch
    fp32 tensor arithmetic, exactly as ``base.py:139`` evaluates it.  Copies
    device tensors to the host (a synchronisation)."""
    dx32 = torch.as_tensor(dx).detach().to('cpu', torch.float32)
    bx32 = torch.as_tensor(bx).detach().to('cpu', torch.float32)
    offset = (bx32 - dx32 / 2.0).numpy().astype(np.float32)
    nxl = [int(v) for v in torch.as_tensor(nx).detach().cpu().tolist()]
    return offset, dx32.numpy().astype(np.float32), nxl


def planar_layout(x):
    """(stride_bn, stride_c, S) if the (B, N, D, fH, fW, C) tensor ``x`` is a
    view of planar storage, element (bn, c, s) at bn*stride_bn + c*stride_c + s
    with S = D*fH*fW and unit stride along s -- the layout of the reference's
    ``rearrange(x, '(b n) c d h w -> b n d h w c')`` (``depth_lss.py:94``);
    else None."""
    B, N, D, fH, fW, C = x.shape
    st = x.stride()
    S = D * fH * fW
    if C < 2 or S < 2 or st[4] != 1 or st[3] != fW or st[2] != fH * fW or st[5] < S:
        return None
    if B == 1 or N == 1:
        sbn = st[1] if B == 1 else st[0]
    elif st[0] == N * st[1]:
        sbn = st[1]
    else:
        return None
    return sbn, st[5], S


class _LSSBevPool(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, geom_feats, offset, dx, nx, index=None):
        B, N, D, fH, fW, C = x.shape
        X, Y, Z = nx
        planar = planar_layout(x) if x.numel() else None
        if planar is not None:
            # channel-first storage: one transposing kernel instead of the
            # reshape copy of base.py:136; the gradient goes back planar
            sbn, sc, S = planar
            x2 = P.planar_rows(x.as_strided((B * N, C, S), (sbn, sc, 1)))
        else:
            x2 = x.reshape(B * N * D * fH * fW, C)
            if x2.stride(1) != 1 and x2.shape[0]:
                x2 = x2.contiguous()
        if index is None:
            idx = P.index_from_geom(geom_feats.reshape(-1, 3), B, offset, dx, nx)
        else:
            idx = index
        out = torch.empty((B, Z * C, X, Y), dtype=torch.float32, device=x.device)
        # element (b, c, z, xy) of the (B, C, Dz, H, W) pool at channel z*C + c
        P.forward(idx, x2, out, Z * C * X * Y, X * Y, C * X * Y)
        ctx.pool_index = idx
        ctx.x_shape = x.shape
        ctx.planar = planar is not None
        return out

    @staticmethod
    def backward(ctx, g):
        idx = ctx.pool_index
        B, N, D, fH, fW, C = ctx.x_shape
        if g.dtype != torch.float32:
            g = g.float()
        if g.stride(3) != 1 or g.stride(2) != idx.W:
            g = g.contiguous()
        if ctx.planar:
            storage = torch.empty((B, N, C, D, fH, fW), dtype=torch.float32, device=g.device)
            P.backward_planar(idx, g, C, g.stride(0), g.stride(1), C * g.stride(1),
                              storage.view(B * N, C, D * fH * fW))
            return storage.permute(0, 1, 3, 4, 5, 2), None, None, None, None, None
        x_grad = torch.empty(ctx.x_shape, dtype=torch.float32, device=g.device)
        P.backward(idx, g, C, g.stride(0), g.stride(1), C * g.stride(1),
                   x_grad.view(-1, C))
        return x_grad, None, None, None, None, None


def lss_bev_pool(geom_feats, x, dx, bx, nx, *, grid=None):
    """``BaseTransform.bev_pool`` (``base.py:131-165``) as a function.

    geom_feats (B, N, D, fH, fW, 3), x (B, N, D, fH, fW, C) -> (B, C*Dz, H, W)
    fp32.  ``grid`` may pass a precomputed :func:`host_grid` triple to avoid
    reading device-resident dx/bx/nx back to the host on every call.
    ``geom_feats`` may instead be a :class:`CameraIndex` (the index stage
    computed from camera matrices by :func:`lss_index_cameras`).
    """
    if torch.is_floating_point(x):
        x = x.float()
    if x.dim() != 6:
        raise ValueError('expected x (B, N, D, H, W, C)')
    if isinstance(geom_feats, CameraIndex):
        P.require_gpu(x)
        geom_feats.check(x.shape[:5], grid)
        offset, d, n = geom_feats.grid
        return _LSSBevPool.apply(x, None, offset, d, tuple(n), geom_feats.index)
    P.require_gpu(geom_feats, x)
    geom_feats = geom_feats.float()
    if geom_feats.dim() != 6 or geom_feats.shape[-1] != 3:
        raise ValueError('expected geom_feats (B, N, D, H, W, 3) and x (B, N, D, H, W, C)')
    if geom_feats.shape[:5] != x.shape[:5]:
        raise ValueError('geom_feats and x must agree on (B, N, D, H, W)')
    offset, d, n = grid if grid is not None else host_grid(dx, bx, nx)
    return _LSSBevPool.apply(x, geom_feats, offset, d, tuple(n))


class _LSSBevPoolDepth(torch.autograd.Function):
    """Pooling of the outer product depth (x) context without materialising
    it: point p = (bn*D + d)*HW + hw carries depth[bn, d, hw] * context[bn, :, hw]."""

    @staticmethod
    def forward(ctx, depth, context, geom_feats, B, offset, dx, nx, index=None):
        BN, D, fH, fW = depth.shape
        C = context.shape[1]
        HW = fH * fW
        X, Y, Z = nx
        depth_flat = depth.contiguous().view(-1)
        rows = P.context_rows(context.reshape(BN, C, HW))
        if index is None:
            idx = P.index_from_geom(geom_feats.reshape(-1, 3), B, offset, dx, nx)
        else:
            idx = index
        out = torch.empty((B, Z * C, X, Y), dtype=torch.float32, device=depth.device)
        P.forward_depth(idx, depth_flat, rows, D, HW, out, Z * C * X * Y, X * Y, C * X * Y)
        ctx.pool_index = idx
        ctx.save_for_backward(depth_flat, rows)
        ctx.shapes = (BN, D, fH, fW, C)
        return out

    @staticmethod
    def backward(ctx, g):
        idx = ctx.pool_index
        depth_flat, rows = ctx.saved_tensors
        BN, D, fH, fW, C = ctx.shapes
        if g.dtype != torch.float32:
            g = g.float()
        if g.stride(3) != 1 or g.stride(2) != idx.W:
            g = g.contiguous()
        grad_depth = torch.empty((BN, D, fH, fW), dtype=torch.float32, device=g.device)
        grad_context = torch.empty((BN, C, fH, fW), dtype=torch.float32, device=g.device)
        P.backward_depth(idx, g, C, g.stride(0), g.stride(1), C * g.stride(1), depth_flat, rows,
                         D, fH * fW, grad_depth.view(-1), grad_context.view(BN, C, fH * fW))
        return grad_depth, grad_context, None, None, None, None, None, None


def lss_bev_pool_depth(geom_feats, depth, context, dx, bx, nx, *, grid=None):
    """``lss_bev_pool(geom_feats, x, ...)`` for the LSS feature
    ``x = depth.unsqueeze(1) * context.unsqueeze(2)`` rearranged to
    (B, N, D, fH, fW, C) (``depth_lss.py:91-94``), without forming ``x``.

    geom_feats (B, N, D, fH, fW, 3); depth (B*N, D, fH, fW) -- the softmaxed
    depth distribution; context (B*N, C, fH, fW), any view whose (fH, fW)
    plane is contiguous (the slice ``x[:, D:D+C]`` of the depth-net output
    costs no copy).  Returns the same (B, C*Dz, H, W) fp32 map, bit for bit,
    as pooling the materialised product; gradients flow to depth and
    context.  Channel counts the fused kernels do not take (C not a multiple
    of 4, or C > 256) pool the product formed on the GPU instead.
    """
    camera_index = geom_feats if isinstance(geom_feats, CameraIndex) else None
    if camera_index is not None:
        P.require_gpu(depth, context)
        shape = camera_index.shape
    else:
        P.require_gpu(geom_feats, depth, context)
        if geom_feats.dim() != 6 or geom_feats.shape[-1] != 3:
            raise ValueError('expected geom_feats (B, N, D, H, W, 3)')
        shape = tuple(geom_feats.shape[:5])
    if depth.dim() != 4 or context.dim() != 4:
        raise ValueError('expected depth (B*N, D, H, W) and context (B*N, C, H, W)')
    B, N, D, fH, fW = shape
    if tuple(depth.shape) != (B * N, D, fH, fW):
        raise ValueError('depth must be (B*N, D, H, W) matching geom_feats')
    if context.shape[0] != B * N or tuple(context.shape[2:]) != (fH, fW):
        raise ValueError('context must be (B*N, C, H, W) matching geom_feats')
    depth = depth.float()
    context = context.float()
    C = context.shape[1]
    if camera_index is not None:
        camera_index.check(shape, grid)
        offset, d, n = camera_index.grid
        geom_feats, index = None, camera_index.index
    else:
        geom_feats = geom_feats.float()
        offset, d, n = grid if grid is not None else host_grid(dx, bx, nx)
        index = None
    if C % 4 != 0 or C > 256 or C == 0:
        x = depth.unsqueeze(1) * context.unsqueeze(2)  # (BN, C, D, fH, fW)
        x = x.permute(0, 2, 3, 4, 1).reshape(B, N, D, fH, fW, C)
        return _LSSBevPool.apply(x, geom_feats, offset, d, tuple(n), index)
    return _LSSBevPoolDepth.apply(depth, context, geom_feats, B, offset, d, tuple(n), index)


def create_frustum(image_size, feature_size, dbound):
    """``base.py:67-80``: (D, fH, fW, 3) fp32 of (u, v, depth) -- image
    columns/rows by ``linspace`` over the feature grid, depths by ``arange``."""
    iH, iW = image_size
    fH, fW = feature_size
    ds = torch.arange(*dbound, dtype=torch.float).view(-1, 1, 1).expand(-1, fH, fW)
    D = ds.shape[0]
    xs = torch.linspace(0, iW - 1, fW, dtype=torch.float).view(1, 1, fW).expand(D, fH, fW)
    ys = torch.linspace(0, iH - 1, fH, dtype=torch.float).view(1, fH, 1).expand(D, fH, fW)
    return torch.stack((xs, ys, ds), -1)


class CameraIndex:
    """The index stage of one frustum (ranks, sorted keys, cell ranges),
    computed from camera matrices by :func:`lss_index_cameras`.  Pass it to
    :func:`lss_bev_pool`, :func:`lss_bev_pool_depth` or the
    :class:`BevPoolTransform` methods in place of ``geom_feats``; it can be
    reused for as long as the cameras are unchanged."""

    def __init__(self, index, shape, grid):
        self.index = index
        self.shape = tuple(int(v) for v in shape)  # (B, N, D, fH, fW)
        self.grid = grid  # host (offset, dx, nx)

    def check(self, shape, grid=None):
        """Shape of the features against the index; with a host ``grid``
        triple, its size against the index's (no device read)."""
        if tuple(int(v) for v in shape) != self.shape:
            raise ValueError(f'features {tuple(shape)} do not match the camera index {self.shape}')
        if grid is not None and list(grid[2]) != list(self.grid[2]):
            raise ValueError('the grid differs from the one the camera index was built on')


def lss_index_cameras(frustum, camera2lidar_rots, camera2lidar_trans, intrins, post_rots,
                      post_trans, dx, bx, nx, *, extra_rots=None, extra_trans=None, grid=None):
    """``get_geometry`` (``base.py:82-126``) fused into the quantisation: the
    frustum points are moved to the lidar frame and quantised inside one
    kernel, never stored.  fp32 with each operation rounded once (combine =
    rots inv(intrins) formed in double, rounded once); torch's matmul may
    round differently, so a point within rounding distance of a voxel face
    can fall in the neighbouring cell (the only difference from pooling
    ``get_geometry``'s tensor)."""
    P.require_gpu(camera2lidar_rots, camera2lidar_trans, intrins, post_rots, post_trans)
    dev = camera2lidar_trans.device
    B, N, _ = camera2lidar_trans.shape
    offset, d, n = grid if grid is not None else host_grid(dx, bx, nx)
    frustum = frustum.to(dev, torch.float32).contiguous()
    mats = (camera2lidar_rots, camera2lidar_trans, intrins, post_rots, post_trans, extra_rots,
            extra_trans)
    idx = P.index_from_cameras(frustum, mats, B, N, offset, d, n)
    D, fH, fW = frustum.shape[:3]
    return CameraIndex(idx, (B, N, D, fH, fW), (offset, d, n))


class BevPoolTransform(nn.Module):
    """The pooling state and method of ``BaseTransform`` (``base.py:26-66,
    131-165``): ``dx``, ``bx``, ``nx`` parameters from the x/y/z bounds and
    ``bev_pool(geom_feats, x)``.  A host copy of the grid is cached (and
    refreshed if the parameters are modified in place) so the forward never
    synchronises."""

    def __init__(self, xbound, ybound, zbound, cache_index=False):
        super().__init__()
        self.cache_index = cache_index
        self._index_cache = None
        self.xbound, self.ybound, self.zbound = xbound, ybound, zbound
        dx, bx, nx = gen_dx_bx(xbound, ybound, zbound)
        self.dx = nn.Parameter(dx, requires_grad=False)
        self.bx = nn.Parameter(bx, requires_grad=False)
        self.nx = nn.Parameter(nx, requires_grad=False)
        self._grid = host_grid(dx, bx, nx)
        self._grid_key = self._key()

    def _key(self):
        return tuple((p.data_ptr(), p._version) for p in (self.dx, self.bx, self.nx))

    def grid(self):
        key = self._key()
        if key != self._grid_key:
            self._grid = host_grid(self.dx, self.bx, self.nx)
            self._grid_key = key
        return self._grid

    def bev_pool(self, geom_feats, x):
        return lss_bev_pool(geom_feats, x, self.dx, self.bx, self.nx, grid=self.grid())

    def index_cameras(self, frustum, camera2lidar_rots, camera2lidar_trans, intrins, post_rots,
                      post_trans, extra_rots=None, extra_trans=None):
        """:func:`lss_index_cameras` on this grid.  With ``cache_index`` set,
        the last index is returned again while every input is the same
        tensor object at the same version (static cameras, e.g. inference
        with fixed calibration); any new or modified input recomputes it."""
        args = (frustum, camera2lidar_rots, camera2lidar_trans, intrins, post_rots, post_trans,
                extra_rots, extra_trans)
        if self.cache_index and self._index_cache is not None:
            key, idx = self._index_cache
            if len(key) == len(args) and all(
                    (a is None and k is None) or (k is not None and a is not None and k[0]() is a
                                                  and k[1] == a._version)
                    for k, a in zip(key, args)):
                return idx
        idx = lss_index_cameras(frustum, camera2lidar_rots, camera2lidar_trans, intrins,
                                post_rots, post_trans, self.dx, self.bx, self.nx,
                                extra_rots=extra_rots, extra_trans=extra_trans, grid=self.grid())
        if self.cache_index:
            self._index_cache = (tuple(None if a is None else (weakref.ref(a), a._version)
                                       for a in args), idx)
        return idx

    def bev_pool_depth(self, geom_feats, depth, context):
        return lss_bev_pool_depth(geom_feats, depth, context, self.dx, self.bx, self.nx,
                                  grid=self.grid())

    def forward(self, geom_feats, x):
        return self.bev_pool(geom_feats, x)


class LSSIndexExport:
    """Every index-stage quantity of a vtransform-level call, in original
    point indices, for parity checks: rank (-1 dropped), kept mask, the stable
    sort permutation of the kept points, their sorted ranks and the interval
    starts/lengths.  Synchronises."""

    def __init__(self, geom_feats, dx, bx, nx):
        P.require_gpu(geom_feats)
        offset, d, n = host_grid(dx, bx, nx)
        B = geom_feats.shape[0]
        idx = P.index_from_geom(geom_feats.float().reshape(-1, 3), B, offset, d, n)
        n_kept = int(P.read_meta(idx)[0])
        self.rank = idx.rank.long()
        self.kept = idx.rank >= 0
        keys = idx.keys[:n_kept]
        self.perm = (keys & 0xFFFFFFFF).long()
        self.sorted_ranks = (keys >> 32).long()
        self.starts, self.lengths, self.cells = P.intervals(idx)
        self.index = idx
