"""Drop-in for the reference's legacy pooling module,
``ops/bev_pool/bev_pool_legacy.py`` (the mit-han-lab style implementation
the reference's tests compare the Triton path against,
``tests/test_ops/test_bev_pool.py:87-119``).

  bev_pool(feats, coords, B, D, H, W)   bev_pool_legacy.py:99-108
  QuickCumsumCuda.apply(x, geom_feats, ranks, B, D, H, W)
                                        bev_pool_legacy.py:53-96

The legacy path sorts the points by its own (x, y, z, b) rank with a
non-stable ``argsort`` and sums each run of equal ranks in sorted order; the
order of points within a cell is therefore unspecified there.  Here each
cell is summed in increasing point order (the stable order), which is one of
the orders the legacy path may produce and the order of the reference's CPU
fallback, so results are deterministic and bit-identical to the op-level
``bev_pool``.  Like the legacy extension (``csrc/bev_pool_cpu.cpp:33`` reads
``data_ptr<float>``), only fp32 features are accepted.
"""
from __future__ import annotations

import torch

from .bev_pool import BevPoolFunction

__all__ = ['QuickCumsumCuda', 'bev_pool']


def _require_fp32(x):
    if x.dtype != torch.float32:
        raise RuntimeError(f'expected scalar type Float but found {x.dtype}')


class QuickCumsumCuda(torch.autograd.Function):
    """``bev_pool_legacy.py:53-96``: features and coords already sorted so
    that equal cells are adjacent; returns the (B, D, H, W, C) pooled grid.
    ``ranks`` only marks the runs in the reference; here the cells come from
    ``geom_feats`` directly (for ranks consistent with the coords, as the
    legacy ``bev_pool`` passes them, the runs are the same)."""

    @staticmethod
    def forward(ctx, x, geom_feats, ranks, B, D, H, W):
        _require_fp32(x)
        out = BevPoolFunction.forward(ctx, x, geom_feats, int(B), int(D), int(H), int(W), True)
        return out.permute(0, 2, 3, 4, 1).contiguous()

    @staticmethod
    def backward(ctx, out_grad):
        g = out_grad.permute(0, 4, 1, 2, 3)  # (B, C, D, H, W) view, strides handled below
        grads = BevPoolFunction.backward(ctx, g)
        return grads[0], None, None, None, None, None, None


def bev_pool(feats, coords, B, D, H, W):
    """``bev_pool_legacy.py:99-108``: (B, C, D, H, W) contiguous pooled grid
    of fp32 ``feats`` at (x, y, z, b) ``coords``; gradient to ``feats``."""
    # the legacy module's own check and exception type (bev_pool_legacy.py:100)
    assert feats.shape[0] == coords.shape[0]
    _require_fp32(feats)
    return BevPoolFunction.apply(feats, coords, int(B), int(D), int(H), int(W))
