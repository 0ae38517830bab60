"""Device pipeline of the pooling path: index stage, forward and backward.

Thin torch-side plumbing over the C ABI (``include/bevpool.h``): it allocates
outputs and scratch with torch's caching allocator on the tensors' device,
passes raw pointers plus torch's current HIP stream, and keeps the device
index (ranks, sorted keys, per-cell ranges) for the backward.  Nothing here
synchronises the device except :func:`read_meta` (used for error reporting
and the optional interval export).
"""
from __future__ import annotations

import threading

import numpy as np
import torch

from . import _lib as L

_INT32_MAX = 2**31 - 1


def require_gpu(*tensors) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                'bevfusion-triton_amd runs the bev_pool path on a ROCm GPU only '
                f'(got a tensor on {t.device}); there is no CPU fallback'
            )


class PoolIndex:
    """Device-resident index of one pooling call.

    rank        int32 (n_points,)  flattened (b, z, x, y) cell, -1 if dropped
    keys        int64 (n_points,)  first n_kept: sorted (rank << 32 | point)
    cell_start  int32 (n_cells,)   sorted range [start, end) of each cell
    cell_end    int32 (n_cells,)
    meta        int32 (8,)         device counters (n_kept, n_intervals, ...)
    """

    __slots__ = ('rank', 'keys', 'cell_start', 'cell_end', 'meta', 'n_points', 'B', 'D', 'H',
                 'W', 'device')

    def __init__(self, n_points, B, D, H, W, device):
        self.n_points, self.B, self.D, self.H, self.W = int(n_points), int(B), int(D), int(H), int(W)
        self.device = device
        n_cells = self.n_cells
        self.rank = torch.empty(self.n_points, dtype=torch.int32, device=device)
        self.keys = torch.empty(self.n_points, dtype=torch.int64, device=device)
        self.cell_start = torch.empty(n_cells, dtype=torch.int32, device=device)
        self.cell_end = torch.empty(n_cells, dtype=torch.int32, device=device)
        self.meta = torch.empty(L.META_LEN, dtype=torch.int32, device=device)

    @property
    def n_cells(self) -> int:
        return self.B * self.D * self.H * self.W

    def workspace(self):
        nbytes = L.library().bevpool_index_workspace_bytes(self.n_points, self.n_cells)
        return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=self.device)


def _check_sizes(n_points: int, n_cells: int) -> None:
    if n_points > _INT32_MAX:
        raise ValueError(f'{n_points} points exceed the 2^31-1 limit of the int32 index')
    if n_cells > _INT32_MAX:
        raise ValueError(f'B*D*H*W = {n_cells} exceeds the 2^31-1 limit of the int32 ranks')


def _sort(idx: PoolIndex, ws, stream) -> None:
    lib = L.library()
    L.check(
        lib.bevpool_sort(
            L.ptr(idx.rank), idx.n_points, idx.n_cells, L.ptr(idx.keys), L.ptr(idx.cell_start),
            L.ptr(idx.cell_end), L.ptr(idx.meta), L.ptr(ws), ws.numel(), stream,
        ),
        'bevpool_sort',
    )


def index_from_geom(geom2d, B: int, offset, dx, nx) -> PoolIndex:
    """Quantise (N_all, 3) fp32 geometry in batch-major point order, keep the
    in-bounds points, stable-sort their ranks and build per-cell ranges.

    offset, dx: 3 fp32 values (offset = fp32(bx) - fp32(dx)/2); nx: 3 ints.
    Output grid (D, H, W) = (nx[2], nx[0], nx[1]).
    """
    require_gpu(geom2d)
    if geom2d.dtype != torch.float32:
        raise TypeError('geometry must be float32')
    if geom2d.dim() != 2 or geom2d.shape[1] != 3:
        raise ValueError('geometry must be (N, 3)')
    if geom2d.stride(1) != 1:
        geom2d = geom2d.contiguous()
    n_points = geom2d.shape[0]
    nx = [int(v) for v in nx]
    B = int(B)
    _check_sizes(n_points, B * nx[0] * nx[1] * nx[2])
    if n_points % B:
        raise ValueError('the point count must be a multiple of the batch size')
    idx = PoolIndex(n_points, B, nx[2], nx[0], nx[1], geom2d.device)
    ws = idx.workspace()
    stream = L.stream_handle(geom2d.device)
    lib = L.library()
    off = np.asarray(offset, dtype=np.float32)
    d = np.asarray(dx, dtype=np.float32)
    with torch.cuda.device(geom2d.device):
        _quantize(lib, geom2d, n_points, B, off, d, nx, idx, ws, stream)
        _sort(idx, ws, stream)
    return idx


def index_from_cameras(frustum, mats, B: int, N: int, offset, dx, nx) -> PoolIndex:
    """As :func:`index_from_geom` with the geometry computed inside the
    quantisation from the frustum (D, fH, fW, 3) and the camera matrices
    ``mats`` = (rots, trans, intrins, post_rots, post_trans, extra_rots,
    extra_trans) (see ``bevpool_quantize_cameras``; the extras may be None)."""
    require_gpu(frustum, *[m for m in mats if m is not None])
    D, fH, fW, three = frustum.shape
    if three != 3:
        raise ValueError('frustum must be (D, fH, fW, 3)')
    frustum = frustum.float().contiguous()
    shapes = ((B * N, 3, 3), (B * N, 3), (B * N, 3, 3), (B * N, 3, 3), (B * N, 3), (B, 3, 3),
              (B, 3))
    flat = []
    for m, shp in zip(mats, shapes):
        if m is None:
            flat.append(None)
            continue
        m = m.float().reshape(shp).contiguous()
        flat.append(m)
    if any(m is None for m in flat[:5]):
        raise ValueError('rots, trans, intrins, post_rots and post_trans are required')
    nx = [int(v) for v in nx]
    n_points = B * N * D * fH * fW
    _check_sizes(n_points, B * nx[0] * nx[1] * nx[2])
    idx = PoolIndex(n_points, B, nx[2], nx[0], nx[1], frustum.device)
    ws = idx.workspace()
    stream = L.stream_handle(frustum.device)
    lib = L.library()
    off = np.asarray(offset, dtype=np.float32)
    d = np.asarray(dx, dtype=np.float32)
    with torch.cuda.device(frustum.device):
        L.check(
            lib.bevpool_quantize_cameras(
                L.ptr(frustum), D, fH, fW, *[L.ptr(m) for m in flat], N, B,
                L._f3(*[float(v) for v in off]), L._f3(*[float(v) for v in d]), L._i3(*nx),
                L.ptr(idx.rank), L.ptr(idx.meta), L.ptr(ws), ws.numel(), stream,
            ),
            'bevpool_quantize_cameras',
        )
        _sort(idx, ws, stream)
    return idx


def _quantize(lib, geom2d, n_points, B, off, d, nx, idx, ws, stream):
    L.check(
        lib.bevpool_quantize_geom(
            L.ptr(geom2d), n_points, geom2d.stride(0) if n_points else 3,
            max(1, n_points // B), B,
            L._f3(*[float(v) for v in off]), L._f3(*[float(v) for v in d]), L._i3(*nx),
            L.ptr(idx.rank), L.ptr(idx.meta), L.ptr(ws), ws.numel(), stream,
        ),
        'bevpool_quantize_geom',
    )


def index_from_coords(coords, B: int, D: int, H: int, W: int) -> PoolIndex:
    """Op-level ranks from (N, 4) int32/int64 coords (x, y, z, b), then the
    same sort and per-cell ranges.  Invalid ranks are excluded and counted in
    meta (see :func:`raise_on_bad_coords`)."""
    require_gpu(coords)
    if coords.stride(1) != 1:
        coords = coords.contiguous()
    n_points = coords.shape[0]
    _check_sizes(n_points, B * D * H * W)
    idx = PoolIndex(n_points, B, D, H, W, coords.device)
    ws = idx.workspace()
    stream = L.stream_handle(coords.device)
    with torch.cuda.device(coords.device):
        _coord_ranks(coords, n_points, B, D, H, W, idx, ws, stream)
        _sort(idx, ws, stream)
    return idx


def _coord_ranks(coords, n_points, B, D, H, W, idx, ws, stream):
    L.check(
        L.library().bevpool_coord_ranks(
            L.ptr(coords), coords.element_size(), n_points, coords.stride(0) if n_points else 4,
            B, D, H, W, L.ptr(idx.rank), L.ptr(idx.meta), L.ptr(ws), ws.numel(), stream,
        ),
        'bevpool_coord_ranks',
    )


def read_meta(idx: PoolIndex) -> np.ndarray:
    """Device counters on the host (synchronises the stream)."""
    return idx.meta.cpu().numpy()


def raise_on_bad_coords(idx: PoolIndex, coords) -> None:
    """Raise the error the reference CPU fallback's index_add_ raises
    (``RuntimeError: index ... is out of bounds``) when a coordinate's rank
    lies outside [0, B*D*H*W).  Synchronises."""
    meta = read_meta(idx)
    if meta[L.META_N_BAD]:
        p = int(meta[L.META_FIRST_BAD])
        x, y, z, b = (int(v) for v in coords[p].tolist())
        r = ((b * idx.D + z) * idx.H + x) * idx.W + y
        raise RuntimeError(
            f'index {r} is out of bounds for dimension 0 with size {idx.n_cells} '
            f'(point {p}, coords (x={x}, y={y}, z={z}, b={b}))'
        )


def intervals(idx: PoolIndex):
    """(starts, lengths, cells) int32 of the occupied cells in rank order
    (synchronises once to read the interval count)."""
    n = idx.n_points
    cap = max(1, n)
    starts = torch.empty(cap, dtype=torch.int32, device=idx.device)
    lengths = torch.empty(cap, dtype=torch.int32, device=idx.device)
    cells = torch.empty(cap, dtype=torch.int32, device=idx.device)
    ws = idx.workspace()
    with torch.cuda.device(idx.device):
        _intervals(idx, n, starts, lengths, cells, ws)
    m = int(read_meta(idx)[L.META_N_INTERVALS])
    return starts[:m], lengths[:m], cells[:m]


def _intervals(idx, n, starts, lengths, cells, ws):
    L.check(
        L.library().bevpool_intervals(
            L.ptr(idx.keys), n, L.ptr(idx.cell_end), L.ptr(starts), L.ptr(lengths), L.ptr(cells),
            L.ptr(idx.meta), L.ptr(ws), ws.numel(), L.stream_handle(idx.device),
        ),
        'bevpool_intervals',
    )


def forward(idx: PoolIndex, feats2d, out, stride_b: int, stride_c: int, stride_z: int) -> None:
    """Pool (n_points, C) rows into `out` (element (b, c, z, xy) at
    b*stride_b + c*stride_c + z*stride_z + xy)."""
    dtype = L.DTYPE_CODES[feats2d.dtype]
    C = feats2d.shape[1]
    if feats2d.stride(1) != 1 and idx.n_points:
        feats2d = feats2d.contiguous()
    lib = L.library()
    scratch_bytes = lib.bevpool_forward_scratch_bytes(idx.n_cells, C)
    scratch = torch.empty(max(int(scratch_bytes), 256), dtype=torch.uint8, device=idx.device)
    with torch.cuda.device(idx.device):
        _forward_call(lib, idx, feats2d, dtype, C, out, stride_b, stride_c, stride_z, scratch)


def _forward_call(lib, idx, feats2d, dtype, C, out, stride_b, stride_c, stride_z, scratch):
    L.check(
        lib.bevpool_forward(
            L.ptr(feats2d), dtype, feats2d.stride(0) if idx.n_points else C, C, idx.n_points,
            L.ptr(idx.keys), L.ptr(idx.cell_start), L.ptr(idx.cell_end), L.ptr(idx.meta), idx.B,
            idx.D, idx.H * idx.W, stride_b, stride_c, stride_z, L.ptr(out), L.ptr(scratch),
            scratch.numel(), L.stream_handle(idx.device),
        ),
        'bevpool_forward',
    )


def backward(idx: PoolIndex, grad, C: int, stride_b: int, stride_c: int, stride_z: int,
             x_grad) -> None:
    """x_grad (n_points, C) <- grad (element (b, c, z, xy) at the strides)."""
    dtype = L.DTYPE_CODES[grad.dtype]
    lib = L.library()
    scratch_bytes = lib.bevpool_backward_scratch_bytes(idx.n_cells, C, dtype)
    scratch = torch.empty(max(int(scratch_bytes), 256), dtype=torch.uint8, device=idx.device)
    with torch.cuda.device(idx.device):
        _backward_call(lib, idx, grad, dtype, C, stride_b, stride_c, stride_z, x_grad, scratch)


def _backward_call(lib, idx, grad, dtype, C, stride_b, stride_c, stride_z, x_grad, scratch):
    L.check(
        lib.bevpool_backward(
            L.ptr(grad), dtype, stride_b, stride_c, stride_z, C, L.ptr(idx.rank), idx.n_points,
            L.ptr(idx.cell_start), L.ptr(idx.cell_end), idx.B, idx.D, idx.H * idx.W,
            L.ptr(x_grad), x_grad.stride(0) if idx.n_points else C, 1, L.ptr(scratch),
            scratch.numel(), L.stream_handle(idx.device),
        ),
        'bevpool_backward',
    )


# ---- depth-weighted (fused depth x context) pooling -------------------------

def planar_rows(src3d):
    """(BN, C, S) fp32 planar tensor (S contiguous, any batch/channel strides)
    -> (BN*S, C) channel-last rows."""
    BN, C, S = src3d.shape
    if src3d.stride(2) != 1:
        src3d = src3d.contiguous()
    rows = torch.empty((BN * S, C), dtype=torch.float32, device=src3d.device)
    with torch.cuda.device(src3d.device):
        L.check(
            L.library().bevpool_planar_rows(
                L.ptr(src3d), src3d.stride(0), src3d.stride(1), BN, C, S, L.ptr(rows),
                L.stream_handle(src3d.device),
            ),
            'bevpool_planar_rows',
        )
    return rows


context_rows = planar_rows  # the depth-net context is planar with S = fH*fW


def backward_planar(idx: PoolIndex, grad, C: int, stride_b: int, stride_c: int, stride_z: int,
                    x_grad3d) -> None:
    """Gradient of the pooling written straight into a planar (BN, C, S) fp32
    tensor (S contiguous)."""
    BN, _, S = x_grad3d.shape
    lib = L.library()
    scratch_bytes = lib.bevpool_backward_scratch_bytes(idx.n_cells, C, L.F32)
    scratch = torch.empty(max(int(scratch_bytes), 256), dtype=torch.uint8, device=idx.device)
    with torch.cuda.device(idx.device):
        L.check(
            lib.bevpool_backward_planar(
                L.ptr(grad), stride_b, stride_c, stride_z, C, L.ptr(idx.rank), idx.n_points,
                L.ptr(idx.cell_start), L.ptr(idx.cell_end), idx.B, idx.D, idx.H * idx.W, S,
                L.ptr(x_grad3d), x_grad3d.stride(0), x_grad3d.stride(1), L.ptr(scratch),
                scratch.numel(), L.stream_handle(idx.device),
            ),
            'bevpool_backward_planar',
        )


def forward_depth(idx: PoolIndex, depth_flat, rows, D: int, HW: int, out, stride_b: int,
                  stride_c: int, stride_z: int) -> None:
    """Pool depth[p] * rows[pix(p)] into `out` (fp32, strides as forward)."""
    C = rows.shape[1]
    lib = L.library()
    scratch_bytes = lib.bevpool_forward_scratch_bytes(idx.n_cells, C)
    scratch = torch.empty(max(int(scratch_bytes), 256), dtype=torch.uint8, device=idx.device)
    with torch.cuda.device(idx.device):
        L.check(
            lib.bevpool_forward_depth(
                L.ptr(depth_flat), L.ptr(rows), C, idx.n_points, D, HW, L.ptr(idx.keys),
                L.ptr(idx.cell_start), L.ptr(idx.cell_end), L.ptr(idx.meta), idx.B, idx.D,
                idx.H * idx.W, stride_b, stride_c, stride_z, L.ptr(out), L.ptr(scratch),
                scratch.numel(), L.stream_handle(idx.device),
            ),
            'bevpool_forward_depth',
        )


def backward_depth(idx: PoolIndex, grad, C: int, stride_b: int, stride_c: int, stride_z: int,
                   depth_flat, rows, D: int, HW: int, grad_depth, grad_context3d) -> None:
    """grad_depth (n_points,) and grad_context (BN, C, HW) <- grad."""
    lib = L.library()
    scratch_bytes = lib.bevpool_backward_scratch_bytes(idx.n_cells, C, L.F32)
    scratch = torch.empty(max(int(scratch_bytes), 256), dtype=torch.uint8, device=idx.device)
    with torch.cuda.device(idx.device):
        L.check(
            lib.bevpool_backward_depth(
                L.ptr(grad), stride_b, stride_c, stride_z, C, L.ptr(idx.rank), idx.n_points, D,
                HW, L.ptr(depth_flat), L.ptr(rows), L.ptr(idx.cell_start), L.ptr(idx.cell_end),
                idx.B, idx.D, idx.H * idx.W, L.ptr(grad_depth), L.ptr(grad_context3d),
                grad_context3d.stride(0), grad_context3d.stride(1), L.ptr(scratch),
                scratch.numel(), L.stream_handle(idx.device),
            ),
            'bevpool_backward_depth',
        )


# ---- deferred (asynchronous) error reports ----------------------------------
#
# The device counts invalid inputs (coords outside the grid, intervals outside
# the arrays) in a meta array.  Reading it at once would synchronise the host
# with the device on every call; instead a kernel of the call (the op-level
# forward's last kernel, or bevpool_meta_report's single block) writes the
# counters into a slot of pinned host memory and then sets the slot's done
# flag, which the host polls -- at the next call of the library's autograd
# functions, or at check_errors().  No event, copy or second stream is
# involved.  An error therefore surfaces one call late, the way an
# asynchronous device error does.

class _Pending:
    __slots__ = ('host', 'report', 'slot')

    def __init__(self, host, report, slot):
        self.host, self.report, self.slot = host, report, slot


_pending = []
# guards _pending and the slots' free lists: the autograd engine runs
# backward calls (which poll) on its own threads
_lock = threading.RLock()


class _ReadBack:
    """Per-device pinned host buffer of ``_SLOTS`` report slots (the
    counters, then the done flag; 64 bytes apart)."""

    _SLOTS = 64
    _STRIDE = 16  # int32 per slot (>= REPORT_LEN)

    def __init__(self, device):
        self.device = device
        self.host = torch.zeros((self._SLOTS, self._STRIDE), dtype=torch.int32, pin_memory=True)
        self.view = self.host.numpy()  # the same pinned memory, read without torch dispatch
        self.base = self.host.data_ptr()
        self.free = list(range(self._SLOTS))


_readback = {}


def report_slot(device):
    """A free pinned slot for a deferred report on ``device``, its done flag
    cleared: (state, slot, host address).  Drains the pending reports when
    every slot is taken."""
    with _lock:
        rb = _readback.get(device)
        if rb is None:
            rb = _readback[device] = _ReadBack(device)
        if not rb.free:
            poll_errors(block=True)  # every slot awaits its kernel: drain them
        slot = rb.free.pop()
        rb.view[slot, L.META_LEN] = 0
        return rb, slot, rb.base + slot * 4 * _ReadBack._STRIDE


def release_slot(rb, slot) -> None:
    """Return a slot whose report was never queued (the call failed)."""
    with _lock:
        rb.free.append(slot)


def defer_report(rb, slot, report) -> None:
    """Queue ``report(host_meta)`` for slot ``slot``, which work already
    queued on the current stream fills."""
    with _lock:
        _pending.append(_Pending(rb, report, slot))


def defer_check(meta, report) -> None:
    """Queue a check of the device counters ``meta`` (int32, written by work
    already queued on the current stream): a single-block kernel on that
    stream copies them into a pinned host slot and sets its done flag.
    ``report(host_meta)`` raises if they show an error.  Skipped while the
    stream is being captured into a graph."""
    if torch.cuda.is_current_stream_capturing():
        return
    device = meta.device
    rb, slot, addr = report_slot(device)
    with torch.cuda.device(device):
        st = L.library().bevpool_meta_report(L.ptr(meta), addr, L.stream_handle(device))
        if st:
            release_slot(rb, slot)
        L.check(st, 'bevpool_meta_report')
    defer_report(rb, slot, report)


def poll_errors(block: bool = False) -> None:
    """Raise the first deferred error whose device work has finished (all
    queued ones when ``block``; that waits for the devices)."""
    if not _pending:
        return
    if block:
        with _lock:
            devices = {p.host.device for p in _pending}
        for dev in devices:
            torch.cuda.synchronize(dev)
    with _lock:
        done = []
        keep = []
        for p in _pending:
            (done if p.host.view[p.slot, L.META_LEN] else keep).append(p)
        if not done:
            return
        _pending[:] = keep
        finished = []
        for p in done:
            finished.append((p.report, p.host.view[p.slot, :L.META_LEN].copy()))
            p.host.free.append(p.slot)
    first = None
    for report, meta in finished:
        try:
            report(meta)
        except RuntimeError as e:  # report every finished slot; raise the first error
            if first is None:
                first = e
    if first is not None:
        raise first


def coords_report(coords, B, D, H, W):
    """Report of an op-level call: the CPU fallback's ``index_add_`` error
    (``bev_pool_triton.py:47``) for the first coordinate whose rank lies
    outside [0, B*D*H*W)."""

    def report(meta):
        if meta[L.META_N_BAD]:
            p = int(meta[L.META_FIRST_BAD])
            x, y, z, b = (int(v) for v in coords[p].tolist())
            r = ((b * D + z) * H + x) * W + y
            raise RuntimeError(
                f'index {r} is out of bounds for dimension 0 with size {B * D * H * W} '
                f'(point {p}, coords (x={x}, y={y}, z={z}, b={b}); '
                f'{int(meta[L.META_N_BAD])} such points were excluded)'
            )

    return report


# ---- one-call op level ------------------------------------------------------

def op_index(n_points: int, n_cells: int, device):
    """The op-level index buffer (meta counters, ranks, sorted keys, cell
    ranges): written by :func:`op_forward`, read by :func:`op_backward`."""
    nbytes = L.library().bevpool_op_index_bytes(n_points, n_cells)
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def op_scratch(n_points: int, n_cells: int, C: int, device):
    """Scratch of one op-level call (index-stage workspace and cell rows);
    enough for the forward and for the backward."""
    nbytes = L.library().bevpool_op_scratch_bytes(n_points, n_cells, C)
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def backward_scratch(n_cells: int, C: int, dtype, device):
    """Scratch of one backward call (the gradient rows of the cells)."""
    nbytes = L.library().bevpool_backward_scratch_bytes(n_cells, C, L.DTYPE_CODES[dtype])
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def op_meta(index):
    """The meta counters at the start of an op-level index buffer."""
    return index[:4 * L.META_LEN].view(torch.int32)


def op_forward(feats2d, coords, B, D, H, W, out, index, scratch, report=None) -> None:
    """The one-call op-level forward.  ``index`` is kept for the backward;
    ``scratch`` is needed only during the call.  ``report``: None, or a
    callable ``report(host_meta)`` run on the meta counters once the device
    has passed this call (the call's last kernel writes them and a done flag
    into a pinned slot; no host synchronisation).  Not queued while the
    stream is being captured."""
    n, C = feats2d.shape
    device = feats2d.device
    slot = None
    if report is not None and not torch.cuda.is_current_stream_capturing():
        rb, slot, addr = report_slot(device)
    with torch.cuda.device(device):
        st = L.library().bevpool_op_forward(
            L.ptr(feats2d), L.DTYPE_CODES[feats2d.dtype], feats2d.stride(0) if n else C, C,
            L.ptr(coords), coords.element_size(), coords.stride(0) if n else 4, n, B, D, H,
            W, L.ptr(out), L.ptr(index), index.numel(), L.ptr(scratch), scratch.numel(),
            addr if slot is not None else None, L.stream_handle(device),
        )
        if st and slot is not None:
            release_slot(rb, slot)
        L.check(st, 'bevpool_op_forward')
    if slot is not None:
        defer_report(rb, slot, report)


def op_backward(grad, C, n, B, D, H, W, x_grad, index, scratch, zero_dropped=True) -> None:
    with torch.cuda.device(grad.device):
        L.check(
            L.library().bevpool_op_backward(
                L.ptr(grad), L.DTYPE_CODES[grad.dtype], grad.stride(0), grad.stride(1),
                grad.stride(2), C, n, B, D, H, W, L.ptr(x_grad),
                x_grad.stride(0) if n else C, 1 if zero_dropped else 0, L.ptr(index),
                index.numel(), L.ptr(scratch), scratch.numel(), L.stream_handle(grad.device),
            ),
            'bevpool_op_backward',
        )
