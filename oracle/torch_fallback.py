"""torch-CPU restatement of the reference's CPU fallback for the bev_pool path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the
HIP path and the CPU baseline of ``bench.py``.  Every function restates the
reference file:line it cites; none of it is imported by the library.

Pinning (see ``tests/test_oracle.py``):
  gen_dx_bx        closed form (double arithmetic -> fp32 / int64 truncation),
                   values for the det/seg/hires grids.
  quantize         hand-derived edge vectors (truncation of q in (-1, 0),
                   NaN/inf, the exact upper bound) + the C restatement.
  flatten_ranks    closed form on tiny inputs + the C restatement.
  bev_pool_cpu     the reference's known-answer fixture (exact), brute-force
                   Python loops, numpy.add.at, and the C sequential sum.
  sort_perm        brute-force sorted((rank, index)) on tiny inputs.
  intervals        brute-force run-length encoding on tiny inputs.
  backward         brute-force gather on tiny inputs + the C restatement.
  get_geometry     brute-force per-point float64 formula (R K^-1 by explicit
                   inverse) with augmentations, the closed-form projection
                   back onto the image for identity augmentation, and a planted
                   inverse-for-transpose mistake.
  pool_ranks       equal, bit for bit, to lss_bev_pool on the ranks of lss_index.
  lss_feature      brute-force loops (one fp32 product per element) and the
                   rearrange's index map on tiny inputs.
  lss_bev_pool_depth  brute-force sequential fp32 loops of depth*context per
                   cell; gradients against hand-written sums in float64 and
                   against finite differences.
"""
from __future__ import annotations

from typing import NamedTuple

import torch


# ---------------------------------------------------------------------------
# models/vtransforms/base.py:19-23
# ---------------------------------------------------------------------------
def gen_dx_bx(xbound, ybound, zbound):
    """dx = step, bx = lo + step/2 (Python double -> fp32), nx = (hi-lo)/step
    (double division, then int64 truncation) -- ``base.py:19-23``."""
    rows = [xbound, ybound, zbound]
    dx = torch.tensor([row[2] for row in rows], dtype=torch.float32)
    bx = torch.tensor([row[0] + row[2] / 2.0 for row in rows], dtype=torch.float32)
    nx = torch.tensor([int((row[1] - row[0]) / row[2]) for row in rows], dtype=torch.int64)
    return dx, bx, nx


# ---------------------------------------------------------------------------
# ops/bev_pool/src/bev_pool_triton.py:12-48, 219-227
# ---------------------------------------------------------------------------
def check_inputs(feats, coords, B, D, H, W) -> None:
    """``bev_pool_triton.py:12-31``: shape / dtype / size validation."""
    if feats.dim() != 2:
        raise ValueError('feats must have shape [N, C].')
    if coords.dim() != 2 or coords.size(-1) != 4:
        raise ValueError('coords must have shape [N, 4].')
    if feats.size(0) != coords.size(0):
        raise ValueError('feats and coords must have the same number of points.')
    if coords.dtype not in (torch.int32, torch.int64):
        raise TypeError('coords must have dtype torch.int32 or torch.int64.')
    if feats.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise TypeError('feats must have dtype torch.float16, torch.float32, or torch.bfloat16.')
    if min(B, D, H, W) <= 0:
        raise ValueError('B, D, H, W must be positive integers.')


def flatten_ranks(coords, B, D, H, W):
    """``bev_pool_triton.py:34-39``: rank = ((b*D + z)*H + x)*W + y in int64."""
    x = coords[:, 0].long()
    y = coords[:, 1].long()
    z = coords[:, 2].long()
    b = coords[:, 3].long()
    return ((b * D + z) * H + x) * W + y


def bev_pool_cpu(feats, coords, B, D, H, W):
    """``bev_pool_triton.py:42-48``: zeros + index_add_ (sequential in point
    order per cell) -> (B, D, H, W, C)."""
    ranks = flatten_ranks(coords, B, D, H, W)
    out = feats.new_zeros((B * D * H * W, feats.size(1)))
    out.index_add_(0, ranks, feats)
    return out.view(B, D, H, W, feats.size(1))


def bev_pool(feats, coords, B, D, H, W):
    """``bev_pool_triton.py:219-227`` (CPU branch): checks, fallback, then the
    ``permute(0, 4, 1, 2, 3).contiguous()`` to (B, C, D, H, W)."""
    B, D, H, W = int(B), int(D), int(H), int(W)
    check_inputs(feats, coords, B, D, H, W)
    out = bev_pool_cpu(feats, coords, B, D, H, W)
    return out.permute(0, 4, 1, 2, 3).contiguous()


# ---------------------------------------------------------------------------
# models/vtransforms/base.py:131-165
# ---------------------------------------------------------------------------
class Quantized(NamedTuple):
    coords: torch.Tensor  # (N_all, 4) int64 (x, y, z, b), before the kept mask
    kept: torch.Tensor  # (N_all,) bool


def quantize(geom_feats, dx, bx, nx) -> Quantized:
    """``base.py:139-156``: ((g - (bx - dx/2)) / dx).long() in fp32, batch
    index appended as column 3 (batch-major point order), kept mask
    0 <= q_k < nx[k]."""
    B = geom_feats.shape[0]
    n_per_batch = geom_feats[0].numel() // 3
    q = ((geom_feats - (bx - dx / 2.0)) / dx).long()
    q = q.reshape(-1, 3)
    batch_ix = torch.arange(B, dtype=torch.long).repeat_interleave(n_per_batch).view(-1, 1)
    coords = torch.cat((q, batch_ix), 1)
    kept = (
        (coords[:, 0] >= 0)
        & (coords[:, 0] < nx[0])
        & (coords[:, 1] >= 0)
        & (coords[:, 1] < nx[1])
        & (coords[:, 2] >= 0)
        & (coords[:, 2] < nx[2])
    )
    return Quantized(coords, kept)


def lss_bev_pool(geom_feats, x, dx, bx, nx):
    """``base.py:131-165`` with ``force_fp32`` (``models/helper/amp.py:35-67``):
    flatten x to (N_all, C), quantise, keep in-bounds points (order-preserving
    boolean gather), bev_pool to (B, C, Dz, H, W), collapse Z by
    ``cat(unbind(2), 1)`` -> (B, C*Dz, H, W).  Differentiable in x."""
    x = x.float()
    geom_feats = geom_feats.float()
    B, N, D, H, W, C = x.shape
    xf = x.reshape(B * N * D * H * W, C)
    q = quantize(geom_feats, dx, bx, nx)
    xk = xf[q.kept]
    ck = q.coords[q.kept]
    out = bev_pool(xk, ck, B, int(nx[2]), int(nx[0]), int(nx[1]))
    return torch.cat(out.unbind(dim=2), 1)


def get_geometry(frustum, camera2lidar_rots, camera2lidar_trans, intrins, post_rots,
                 post_trans, extra_rots=None, extra_trans=None, dtype=torch.float32):
    """``base.py:82-126`` in ``dtype``: undo the image augmentation
    (subtract post_trans, multiply by post_rots^T -- the transpose, as the
    reference writes it), scale (u, v) by depth, map by
    combine = linalg.solve(K^T, R^T)^T = R K^-1, add the translation, then the
    optional lidar augmentation.  (B, N, D, fH, fW, 3)."""
    f = lambda t: t.to(dtype)
    B, N, _ = camera2lidar_trans.shape
    points = f(frustum) - f(post_trans).view(B, N, 1, 1, 1, 3)
    points = f(post_rots).transpose(-1, -2).reshape(B, N, 1, 1, 1, 3, 3).matmul(
        points.unsqueeze(-1))
    points = torch.cat((points[..., :2, :] * points[..., 2:3, :], points[..., 2:3, :]), 5)
    combine = torch.linalg.solve(f(intrins).transpose(-1, -2),
                                 f(camera2lidar_rots).transpose(-1, -2)).transpose(-1, -2)
    points = combine.reshape(B, N, 1, 1, 1, 3, 3).matmul(points).squeeze(-1)
    points = points + f(camera2lidar_trans).view(B, N, 1, 1, 1, 3)
    if extra_rots is not None:
        points = f(extra_rots).view(B, 1, 1, 1, 1, 3, 3).matmul(points.unsqueeze(-1)).squeeze(-1)
    if extra_trans is not None:
        points = points + f(extra_trans).view(B, 1, 1, 1, 1, 3)
    return points


def pool_ranks(x2, rank, B, nx):
    """``base.py:157-165`` from the ranks on: keep rank >= 0 (order-preserving
    boolean gather), ``index_add_`` in point order into the
    (B, Dz, X, Y) grid (rank = ((b*Dz + z)*X + x)*Y + y), then the
    (B, C*Dz, X, Y) collapse.  x2 (N_all, C)."""
    X, Y, Z = (int(v) for v in nx)
    keep = rank >= 0
    C = x2.shape[1]
    out = x2.new_zeros((B * Z * X * Y, C))
    out.index_add_(0, rank[keep], x2[keep])
    out = out.view(B, Z, X, Y, C).permute(0, 4, 1, 2, 3)
    return torch.cat(out.unbind(dim=2), 1)


def lss_feature(depth, context, B, N):
    """``depth_lss.py:91-94``: x = depth.unsqueeze(1) * context.unsqueeze(2)
    -> (BN, C, D, fH, fW), then ``rearrange('(b n) c d h w -> b n d h w c')``."""
    x = depth.unsqueeze(1) * context.unsqueeze(2)
    BN, C, D, fH, fW = x.shape
    return x.permute(0, 2, 3, 4, 1).reshape(B, N, D, fH, fW, C)


def lss_bev_pool_depth(geom_feats, depth, context, dx, bx, nx, dtype=torch.float32):
    """The LSS feature (``lss_feature``) pooled by ``base.py:131-165``.
    ``dtype`` float32 is the reference (``force_fp32``); float64 gives the
    exact-arithmetic gradients the GPU's fp32 gradients are measured
    against.  Differentiable in depth and context."""
    B, N = geom_feats.shape[:2]
    x = lss_feature(depth.to(dtype), context.to(dtype), B, N)
    C = x.shape[-1]
    q = quantize(geom_feats.float(), dx, bx, nx)
    xk = x.reshape(-1, C)[q.kept]
    ck = q.coords[q.kept]
    out = bev_pool_cpu(xk, ck, B, int(nx[2]), int(nx[0]), int(nx[1]))
    out = out.permute(0, 4, 1, 2, 3)
    return torch.cat(out.unbind(dim=2), 1)


# ---------------------------------------------------------------------------
# sort permutation and intervals (ops/bev_pool/bev_pool_legacy.py:56-61,
# 102-104) on the (b, z, x, y) ranks of the kept points
# ---------------------------------------------------------------------------
def sort_perm(ranks):
    """Stable argsort of the ranks: the permutation a sequential per-cell sum
    in point order visits (``bev_pool_legacy.py:103`` made stable)."""
    return torch.sort(ranks, stable=True).indices


def intervals(sorted_ranks):
    """``bev_pool_legacy.py:56-61``: starts where r[i] != r[i-1] (int32),
    lengths by difference with the last one n - start."""
    n = sorted_ranks.shape[0]
    if n == 0:
        return torch.zeros(0, dtype=torch.int32), torch.zeros(0, dtype=torch.int32)
    kept = torch.ones(n, dtype=torch.bool)
    kept[1:] = sorted_ranks[1:] != sorted_ranks[:-1]
    starts = torch.where(kept)[0].int()
    lengths = torch.zeros_like(starts)
    lengths[:-1] = starts[1:] - starts[:-1]
    lengths[-1] = n - starts[-1]
    return starts, lengths


def backward_gather(grad, coords, B, D, H, W):
    """Gradient of ``bev_pool`` w.r.t. feats: index_add_'s backward is
    ``grad.index_select(0, ranks)`` on the (B*D*H*W, C) view of the
    channel-last gradient (``bev_pool_triton.py:102-150`` computes the same
    gather)."""
    ranks = flatten_ranks(coords, B, D, H, W)
    g = grad.permute(0, 2, 3, 4, 1).reshape(B * D * H * W, grad.shape[1])
    return g.index_select(0, ranks)


class LSSIndex(NamedTuple):
    rank: torch.Tensor  # (N_all,) int64, -1 for dropped points
    kept: torch.Tensor  # (N_all,) bool
    perm: torch.Tensor  # (N_kept,) int64 original point index, in sorted order
    sorted_ranks: torch.Tensor  # (N_kept,) int64
    starts: torch.Tensor  # (n_int,) int32
    lengths: torch.Tensor  # (n_int,) int32


def lss_index(geom_feats, dx, bx, nx) -> LSSIndex:
    """Every index-stage quantity of the vtransform path, in original point
    indices: rank (-1 dropped), kept mask, the stable sort permutation of the
    kept points, their sorted ranks and the interval starts/lengths."""
    q = quantize(geom_feats.float(), dx, bx, nx)
    B = geom_feats.shape[0]
    ranks = flatten_ranks(q.coords, B, int(nx[2]), int(nx[0]), int(nx[1]))
    rank = torch.where(q.kept, ranks, torch.full_like(ranks, -1))
    kept_idx = torch.nonzero(q.kept).squeeze(1)
    rk = ranks[kept_idx]
    order = sort_perm(rk)
    perm = kept_idx[order]
    sorted_ranks = rk[order]
    starts, lengths = intervals(sorted_ranks)
    return LSSIndex(rank, q.kept, perm, sorted_ranks, starts, lengths)


# ---------------------------------------------------------------------------
# legacy extension: ops/bev_pool/csrc/bev_pool_cpu.cpp:22-94 and the kernels
# of ops/bev_pool/csrc/bev_pool_cuda.cu:20-98, driven by
# ops/bev_pool/bev_pool_legacy.py:53-96
# ---------------------------------------------------------------------------
def legacy_cell(geom_feats, s, b, d, h, w):
    """Cell of the interval starting at row s (``bev_pool_cuda.cu:33-35``:
    ((gb*d + gz)*h + gx)*w + gy from geom_feats[s] = (gx, gy, gz, gb)), or
    None when the row or the cell lies outside the arrays (the reference
    reads / writes out of bounds there; the library skips the interval)."""
    if s < 0 or s >= geom_feats.shape[0]:
        return None
    gx, gy, gz, gb = (int(v) for v in geom_feats[s])
    if not (0 <= gx < h and 0 <= gy < w and 0 <= gz < d and 0 <= gb < b):
        return None
    return ((gb * d + gz) * h + gx) * w + gy


def _valid_interval(s, n_rows, n):
    return 0 <= s and 0 <= n_rows and s < n and s + n_rows <= n


def legacy_forward(x, geom_feats, interval_lengths, interval_starts, b, d, h, w):
    """``bev_pool_forward`` (``bev_pool_cpu.cpp:22-47`` + ``bev_pool_cuda.cu:20-42``):
    zeros (b, d, h, w, c); interval j stores psum = ((0 + x[s]) + x[s+1]) + ...
    (fp32, rows in order) at the cell of its first row.  Returns (out, n_bad)
    with n_bad the intervals skipped as invalid."""
    n, c = x.shape
    out = torch.zeros((b * d * h * w, c), dtype=torch.float32)
    n_bad = 0
    for j in range(int(interval_lengths.shape[0])):
        s, m = int(interval_starts[j]), int(interval_lengths[j])
        cell = legacy_cell(geom_feats, s, b, d, h, w) if _valid_interval(s, m, n) else None
        if cell is None:
            n_bad += 1
            continue
        psum = torch.zeros(c, dtype=torch.float32)
        for i in range(m):
            psum = psum + x[s + i]
        out[cell] = psum
    return out.view(b, d, h, w, c), n_bad


def legacy_backward(out_grad, geom_feats, interval_lengths, interval_starts, b, d, h, w):
    """``bev_pool_backward`` (``bev_pool_cpu.cpp:60-87`` + ``bev_pool_cuda.cu:61-84``):
    zeros (n, c), n = geom_feats rows; every row of interval j gets
    out_grad[cell]."""
    n, c = geom_feats.shape[0], out_grad.shape[4]
    g = out_grad.reshape(b * d * h * w, c)
    x_grad = torch.zeros((n, c), dtype=torch.float32)
    n_bad = 0
    for j in range(int(interval_lengths.shape[0])):
        s, m = int(interval_starts[j]), int(interval_lengths[j])
        cell = legacy_cell(geom_feats, s, b, d, h, w) if _valid_interval(s, m, n) else None
        if cell is None:
            n_bad += 1
            continue
        x_grad[s:s + m] = g[cell]
    return x_grad, n_bad


def runs(ranks):
    """``bev_pool_legacy.py:56-61`` on any rank array (not necessarily sorted):
    the same as :func:`intervals`."""
    return intervals(ranks)


def legacy_ranks(coords, B, D, H, W):
    """``bev_pool_legacy.py:102``: x*(W*D*B) + y*(D*B) + z*B + b."""
    c = coords.long()
    return c[:, 0] * (W * D * B) + c[:, 1] * (D * B) + c[:, 2] * B + c[:, 3]
