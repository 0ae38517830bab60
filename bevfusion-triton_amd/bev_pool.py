"""Op-level ``bev_pool(feats, coords, B, D, H, W)`` on MI355X.

Drop-in for ``ops/bev_pool/src/bev_pool_triton.py:219-227`` (re-exported by
``ops/bev_pool/__init__.py:1``): same arguments, same checks and exception
types (``:12-31``), same result -- a contiguous (B, C, D, H, W) tensor of
feats' dtype whose cell (b, z, x, y) holds the sum of the rows of feats whose
coords are (x, y, z, b); gradient to feats only.

Differences from the reference, by design:
  * the sum of each cell is accumulated in fp32 in increasing point order
    (the order of the reference's CPU ``index_add_``), so fp32 results are
    bit-identical to the CPU fallback and run-to-run deterministic (the
    reference's Triton path uses unordered atomics, ``:99``); fp16/bf16 inputs
    accumulate in fp32 and round once;
  * a coordinate whose flattened rank falls outside [0, B*D*H*W) is excluded
    on the device instead of being written out of bounds (the reference's
    Triton path does not check) and reported as the ``RuntimeError`` the CPU
    fallback's ``index_add_`` raises.  By default the report is asynchronous:
    the forward's last kernel writes the device counters into a slot of
    pinned host memory and then sets the slot's done flag; the next call of
    this module's functions (or :func:`check_errors`) polls that flag and
    raises once it is set, so a call never waits for the device.
    ``check_bounds='sync'`` waits and raises in the same call;
    ``check_bounds=False`` drops such points silently;
  * CPU tensors are rejected: the HIP path is the only implementation.
"""
from __future__ import annotations

from typing import SupportsInt

import torch

from . import _pipeline as P


def _check_inputs(feats, coords, B, D, H, W) -> None:
    """``bev_pool_triton.py:12-31``, message for message."""
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


def _flatten_ranks(coords, B, D, H, W):
    """``bev_pool_triton.py:34-39`` on the host (used only for error messages
    and by callers that want the ranks as a tensor)."""
    x = coords[:, 0].long()
    y = coords[:, 1].long()
    z = coords[:, 2].long()
    b = coords[:, 3].long()
    return ((b * D + z) * H + x) * W + y


class BevPoolFunction(torch.autograd.Function):
    """Counterpart of ``_BevPoolTritonFunction`` (``bev_pool_triton.py:153-216``):
    forward pools straight into the channel-first (B, C, D, H, W) layout (the
    reference's ``permute().contiguous()`` of ``:227`` is fused into the
    kernel's store) with one call of the library's op-level entry, which
    leaves the index (ranks, sorted keys, cell ranges: 12 bytes per point
    plus 8 per cell) in a buffer saved for the backward; the call's scratch
    (index-stage workspace and cell rows) is freed after each call.  Backward
    returns ``(x_grad, None x 6)``."""

    @staticmethod
    def forward(ctx, feats, coords, B, D, H, W, check_bounds=True):
        P.require_gpu(feats, coords)
        P.poll_errors()
        N, C = feats.shape
        ctx.feats_meta = (N, C, feats.dtype)
        ctx.sizes = (B, D, H, W)
        if C == 0:  # nothing to pool; the reference returns an empty (B, 0, D, H, W)
            ctx.index = None
            return feats.new_zeros((B, 0, D, H, W))
        P._check_sizes(N, B * D * H * W)
        feats2d = feats if feats.stride(1) == 1 or N == 0 else feats.contiguous()
        coords2d = coords if coords.stride(1) == 1 or N == 0 else coords.contiguous()
        index = P.op_index(N, B * D * H * W, feats.device)
        scratch = P.op_scratch(N, B * D * H * W, C, feats.device)
        out = torch.empty((B, C, D, H, W), dtype=feats.dtype, device=feats.device)
        if check_bounds == 'sync':
            P.op_forward(feats2d, coords2d, B, D, H, W, out, index, scratch)
            P.coords_report(coords2d, B, D, H, W)(P.op_meta(index).cpu().numpy())
        elif check_bounds:
            P.op_forward(feats2d, coords2d, B, D, H, W, out, index, scratch,
                         report=P.coords_report(coords2d, B, D, H, W))
        else:
            P.op_forward(feats2d, coords2d, B, D, H, W, out, index, scratch)
        ctx.index = index
        return out

    @staticmethod
    def backward(ctx, out_grad):
        P.poll_errors()
        N, C, dtype = ctx.feats_meta
        B, D, H, W = ctx.sizes
        if ctx.index is None:
            return out_grad.new_zeros((N, C), dtype=dtype), None, None, None, None, None, None
        g = out_grad
        if g.dtype != dtype:
            g = g.to(dtype)
        if g.stride(4) != 1 or g.stride(3) != W:
            g = g.contiguous()
        x_grad = torch.empty((N, C), dtype=dtype, device=g.device)
        scratch = P.backward_scratch(B * D * H * W, C, dtype, g.device)
        P.op_backward(g, C, N, B, D, H, W, x_grad, ctx.index, scratch)
        return x_grad, None, None, None, None, None, None


def bev_pool(feats: torch.Tensor, coords: torch.Tensor, B: SupportsInt, D: SupportsInt,
             H: SupportsInt, W: SupportsInt, *, check_bounds=True) -> torch.Tensor:
    """``bev_pool_triton.py:219-227``: (N, C) feats + (N, 4) coords (x, y, z, b)
    -> contiguous (B, C, D, H, W).  B, D, H, W may be 0-d integer tensors (the
    vtransform passes ``self.nx[k]``).  ``check_bounds``: True (report
    out-of-grid coords asynchronously, no host synchronisation), ``'sync'``
    (synchronise and raise in this call) or False."""
    B, D, H, W = int(B), int(D), int(H), int(W)
    _check_inputs(feats, coords, B, D, H, W)
    if check_bounds not in (True, False, 'sync'):
        raise ValueError("check_bounds must be True, False or 'sync'")
    return BevPoolFunction.apply(feats, coords, B, D, H, W, check_bounds)


def check_errors() -> None:
    """Wait for the device and raise any deferred error of earlier calls
    (out-of-grid coordinates, invalid legacy intervals)."""
    P.poll_errors(block=True)


class BevPoolIndexExport:
    """Every index-stage quantity of one op-level call, for parity checks:
    ranks (-1 = invalid), the stable sort permutation, sorted ranks and the
    interval starts/lengths (``bev_pool_legacy.py:56-61`` semantics on
    (b, z, x, y) ranks).  Synchronises."""

    def __init__(self, coords, B, D, H, W):
        P.require_gpu(coords)
        idx = P.index_from_coords(coords, int(B), int(D), int(H), int(W))
        meta = P.read_meta(idx)
        n_kept = int(meta[0])
        self.rank = idx.rank.long()
        keys = idx.keys[:n_kept]
        self.perm = (keys & 0xFFFFFFFF).long()
        self.sorted_ranks = (keys >> 32).long()
        self.starts, self.lengths, self.cells = P.intervals(idx)
        self.n_bad = int(meta[2])
        self.index = idx
