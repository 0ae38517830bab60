"""Drop-in for the reference's legacy pooling module,
``ops/bev_pool/bev_pool_legacy.py`` (the mit-han-lab style implementation
the reference's tests compare the Triton path against,
``tests/test_ops/test_bev_pool.py:50-54, 87-119``).

  ext_module.bev_pool_forward / bev_pool_backward
                                        bev_pool_legacy.py:10-19, the pybind
                                        functions of csrc/bev_pool_cpu.cpp:22-94
  QuickCumsumCuda.apply(x, geom_feats, ranks, B, D, H, W)
                                        bev_pool_legacy.py:53-96
  bev_pool(feats, coords, B, D, H, W)   bev_pool_legacy.py:99-108

``ext_module`` and ``QuickCumsumCuda`` run on the caller's intervals: the runs
of equal ``ranks`` (``bev_pool_legacy.py:56-61``) are found on the device
(``bevpool_runs``, no host synchronisation where the reference calls
``torch.where``), and each run is summed in row order into the cell of its
first row's coordinates (``bevpool_legacy_forward``), exactly the legacy
kernel's arithmetic.  Like the legacy extension (``csrc/bev_pool_cpu.cpp:33``
reads ``data_ptr<float>``), only fp32 features are accepted.

``bev_pool`` sorts by its own (x, y, z, b) rank with a non-stable ``argsort``
in the reference, so the order of points within a cell is unspecified there;
here it runs the op-level path, which sums each cell in increasing point
order -- one of the orders the legacy path may produce and the order of the
reference's CPU fallback -- so results are deterministic and bit-identical to
the op-level ``bev_pool``.

Difference from the reference: an interval whose rows or cell lie outside the
arrays is skipped (the reference reads and writes out of bounds) and reported
as a ``RuntimeError`` by the next call of the library once the device has
passed this one (``check_errors()`` waits for it).
"""
from __future__ import annotations

import types

import torch

from . import _lib as L
from . import _pipeline as P
from .bev_pool import BevPoolFunction

__all__ = ['QuickCumsumCuda', 'bev_pool', 'ext_module']


def _require_dtype(t, dtype, name):
    """``Tensor.data_ptr<T>()``'s check in csrc/bev_pool_cpu.cpp:33-36, 71-74."""
    if t.dtype != dtype:
        want = {torch.float32: 'Float', torch.int32: 'Int'}[dtype]
        got = {torch.float16: 'Half', torch.bfloat16: 'BFloat16', torch.float64: 'Double',
               torch.int64: 'Long', torch.int16: 'Short', torch.int8: 'Char',
               torch.uint8: 'Byte', torch.bool: 'Bool', torch.float32: 'Float',
               torch.int32: 'Int'}.get(t.dtype, str(t.dtype))
        raise RuntimeError(f'expected scalar type {want} but found {got} ({name})')


def _require_fp32(x):
    _require_dtype(x, torch.float32, 'x')


def _interval_report(what):
    def report(meta):
        if meta[L.META_N_BAD]:
            raise RuntimeError(f'{what}: {int(meta[L.META_N_BAD])} intervals whose rows or cell lie '
                               f'outside the input were skipped')
    return report


def _legacy_call(fn, src, n, C, geom_feats, starts, lengths, n_intervals, count_dev, b, d, h, w,
                 dst, what):
    meta = torch.zeros(L.META_LEN, dtype=torch.int32, device=dst.device)
    with torch.cuda.device(dst.device):
        L.check(
            fn(L.ptr(src), n, C, L.ptr(geom_feats), L.ptr(starts), L.ptr(lengths), n_intervals,
               L.ptr(count_dev), b, d, h, w, L.ptr(dst), L.ptr(meta),
               L.stream_handle(dst.device)),
            what,
        )
    P.defer_check(meta, _interval_report(what))


def _interval_arrays(geom_feats, interval_lengths, interval_starts, n_rows):
    _require_dtype(geom_feats, torch.int32, 'geom_feats')
    if geom_feats.dim() != 2 or geom_feats.shape[1] != 4 or geom_feats.shape[0] < n_rows:
        raise RuntimeError(f'geom_feats must be (n, 4) with n >= {n_rows} rows, got '
                           f'{tuple(geom_feats.shape)}')
    _require_dtype(interval_lengths, torch.int32, 'interval_lengths')
    _require_dtype(interval_starts, torch.int32, 'interval_starts')
    n_int = interval_lengths.size(0)
    if interval_starts.numel() < n_int:
        raise RuntimeError(f'interval_starts holds {interval_starts.numel()} entries, '
                           f'interval_lengths {n_int}')
    P.require_gpu(geom_feats, interval_lengths, interval_starts)
    return (geom_feats.contiguous(), interval_starts.contiguous(), interval_lengths.contiguous(),
            n_int)


def _bev_pool_forward(x, geom_feats, interval_lengths, interval_starts, b, d, h, w):
    """``bev_pool_forward`` (csrc/bev_pool_cpu.cpp:22-47): (b, d, h, w, c) fp32,
    zero outside the intervals' cells; interval j's cell holds the row-order
    sum of x[starts[j] : starts[j] + lengths[j]]."""
    _require_fp32(x)
    P.require_gpu(x)
    P.poll_errors()
    if x.dim() != 2:
        raise RuntimeError(f'x must be (n, c), got {tuple(x.shape)}')
    geom_feats, starts, lengths, n_int = _interval_arrays(geom_feats, interval_lengths,
                                                         interval_starts, x.shape[0])
    n, c = x.shape
    b, d, h, w = int(b), int(d), int(h), int(w)
    out = torch.empty((b, d, h, w, c), dtype=x.dtype, device=x.device)
    _legacy_call(L.library().bevpool_legacy_forward, x.contiguous(), n, c, geom_feats, starts,
                 lengths, n_int, None, b, d, h, w, out, 'bev_pool_forward')
    return out


def _bev_pool_backward(out_grad, geom_feats, interval_lengths, interval_starts, b, d, h, w):
    """``bev_pool_backward`` (csrc/bev_pool_cpu.cpp:60-87): (n, c) fp32 with
    n = geom_feats.size(0), c = out_grad.size(4); each interval's rows get
    its cell's gradient row, other rows are zero."""
    _require_dtype(out_grad, torch.float32, 'out_grad')
    P.require_gpu(out_grad)
    P.poll_errors()
    geom_feats, starts, lengths, n_int = _interval_arrays(geom_feats, interval_lengths,
                                                         interval_starts, 0)
    n, c = geom_feats.size(0), out_grad.size(4)
    b, d, h, w = int(b), int(d), int(h), int(w)
    if tuple(out_grad.shape) != (b, d, h, w, c):
        raise RuntimeError(f'out_grad must be (b, d, h, w, c) = {(b, d, h, w, c)}, got '
                           f'{tuple(out_grad.shape)}')
    x_grad = torch.empty((n, c), dtype=out_grad.dtype, device=out_grad.device)
    _legacy_call(L.library().bevpool_legacy_backward, out_grad.contiguous(), n, c, geom_feats,
                 starts, lengths, n_int, None, b, d, h, w, x_grad, 'bev_pool_backward')
    return x_grad


# The reference's lazily built pybind extension (bev_pool_legacy.py:10-19);
# its two functions take the same arguments in the same order.
ext_module = types.SimpleNamespace(bev_pool_forward=_bev_pool_forward,
                                   bev_pool_backward=_bev_pool_backward)


def _runs(ranks):
    """Run starts and lengths of ``ranks`` on the device (capacity n, count
    in meta[BEVPOOL_META_N_INTERVALS]): bev_pool_legacy.py:56-61."""
    if ranks.dtype not in (torch.int32, torch.int64):
        raise TypeError(f'ranks must be int32 or int64, got {ranks.dtype}')
    r = ranks.contiguous()
    n = r.numel()
    starts = torch.empty(max(n, 1), dtype=torch.int32, device=r.device)
    lengths = torch.empty(max(n, 1), dtype=torch.int32, device=r.device)
    meta = torch.empty(L.META_LEN, dtype=torch.int32, device=r.device)
    lib = L.library()
    ws = torch.empty(max(int(lib.bevpool_runs_workspace_bytes(n)), 256), dtype=torch.uint8,
                     device=r.device)
    with torch.cuda.device(r.device):
        L.check(lib.bevpool_runs(L.ptr(r), r.element_size(), n, L.ptr(starts), L.ptr(lengths),
                                 L.ptr(meta), L.ptr(ws), ws.numel(), L.stream_handle(r.device)),
                'bevpool_runs')
    return starts, lengths, meta


class QuickCumsumCuda(torch.autograd.Function):
    """``bev_pool_legacy.py:53-96``: x (n, c) fp32 and geom_feats (n, 4) sorted
    so that equal ``ranks`` are adjacent; each run of equal ranks is summed in
    row order into the cell of its first row.  Returns the (B, D, H, W, C)
    pooled grid; the gradient flows to x."""

    @staticmethod
    def forward(ctx, x, geom_feats, ranks, B, D, H, W):
        _require_fp32(x)
        P.require_gpu(x, geom_feats, ranks)
        P.poll_errors()
        n, c = x.shape
        B, D, H, W = int(B), int(D), int(H), int(W)
        if ranks.numel() != n or geom_feats.dim() != 2 or tuple(geom_feats.shape) != (n, 4):
            raise ValueError('x (n, c), geom_feats (n, 4) and ranks (n,) must have the same '
                             'number of rows')
        starts, lengths, meta = _runs(ranks)
        geom_i = geom_feats.int().contiguous()
        count = meta[L.META_N_INTERVALS:L.META_N_INTERVALS + 1]
        out = torch.empty((B, D, H, W, c), dtype=x.dtype, device=x.device)
        _legacy_call(L.library().bevpool_legacy_forward, x.contiguous(), n, c, geom_i, starts,
                     lengths, n, count, B, D, H, W, out, 'QuickCumsumCuda')
        ctx.save_for_backward(starts, lengths, geom_i, count)
        ctx.saved_shapes = B, D, H, W
        return out

    @staticmethod
    def backward(ctx, out_grad):
        starts, lengths, geom_i, count = ctx.saved_tensors
        B, D, H, W = ctx.saved_shapes
        P.poll_errors()
        g = out_grad.float().contiguous()
        n, c = geom_i.shape[0], g.shape[4]
        x_grad = torch.empty((n, c), dtype=torch.float32, device=g.device)
        _legacy_call(L.library().bevpool_legacy_backward, g, n, c, geom_i, starts, lengths, n,
                     count, B, D, H, W, x_grad, 'QuickCumsumCuda backward')
        return x_grad, None, None, None, None, None, None


def bev_pool(feats, coords, B, D, H, W):
    """``bev_pool_legacy.py:99-108``: (B, C, D, H, W) contiguous pooled grid
    of fp32 ``feats`` at (x, y, z, b) ``coords``; gradient to ``feats``."""
    # the legacy module's own check and exception type (bev_pool_legacy.py:100)
    assert feats.shape[0] == coords.shape[0]
    _require_fp32(feats)
    return BevPoolFunction.apply(feats, coords, int(B), int(D), int(H), int(W), True)
