"""Pins the oracle of the depth-weighted pooling (``oracle/torch_fallback.py``
``lss_feature`` / ``lss_bev_pool_depth``, restating ``depth_lss.py:91-94`` and
``base.py:131-165``) against brute-force loops that share none of its code:
ranks come from the independent C restatement, products are single fp32
multiplications in numpy, sums are sequential fp32 additions in point order,
and the gradients are the hand-written sums of the chain rule in float64.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import seq
from oracle import torch_fallback as ref

BOUNDS = ((-2.0, 2.0, 1.0), (-1.5, 1.5, 1.0), (-10.0, 10.0, 20.0))  # 4 x 3 x 1 grid


def tiny_inputs(seed, B=2, N=2, D=3, fH=2, fW=3, C=5):
    rng = np.random.default_rng(seed)
    geom = rng.uniform(-2.6, 2.6, size=(B, N, D, fH, fW, 3)).astype(np.float32)
    geom[..., 2] = rng.uniform(-12.0, 12.0, size=geom.shape[:-1]).astype(np.float32)
    # a few collisions: several points of one ray land in one cell
    geom[0, 0, :, 0, 0, :] = np.array([0.1, 0.2, 0.0], np.float32)
    logits = rng.standard_normal((B * N, D, fH, fW)).astype(np.float32)
    depth = torch.from_numpy(logits).softmax(dim=1).numpy()
    context = rng.standard_normal((B * N, C, fH, fW)).astype(np.float32)
    return geom, depth, context


def c_ranks(geom, B):
    dx, bx, nx = ref.gen_dx_bx(*BOUNDS)
    offset = (bx - dx / 2.0).numpy()
    n = geom[..., 0].size
    return seq.quantize_geom(geom, n // B, offset, dx.numpy(), nx.numpy()), nx


def brute_feature(depth, context, B, N):
    BN, D, fH, fW = depth.shape
    C = context.shape[1]
    x = np.zeros((B, N, D, fH, fW, C), np.float32)
    for bn in range(BN):
        b, n = divmod(bn, N)
        for d in range(D):
            for h in range(fH):
                for w in range(fW):
                    for c in range(C):
                        x[b, n, d, h, w, c] = np.float32(depth[bn, d, h, w]) * np.float32(
                            context[bn, c, h, w])
    return x


@pytest.mark.parametrize('seed', [0, 1, 2])
def test_lss_feature_brute_force(seed):
    geom, depth, context = tiny_inputs(seed)
    B, N = geom.shape[:2]
    x = ref.lss_feature(torch.from_numpy(depth), torch.from_numpy(context), B, N)
    expect = brute_feature(depth, context, B, N)
    np.testing.assert_array_equal(x.numpy().view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize('seed', [0, 1, 2, 3])
def test_lss_bev_pool_depth_brute_force(seed):
    geom, depth, context = tiny_inputs(seed)
    B, N, D, fH, fW = geom.shape[:5]
    C = context.shape[1]
    rank, nx = c_ranks(geom, B)
    X, Y, Z = (int(v) for v in nx)
    assert (rank < 0).any() and (rank >= 0).any()
    acc = np.zeros((B * Z * X * Y, C), np.float32)
    HW = fH * fW
    for p in range(rank.size):  # point order = (b, n, d, h, w)
        if rank[p] < 0:
            continue
        bn, rem = divmod(p, D * HW)
        d, hw = divmod(rem, HW)
        h, w = divmod(hw, fW)
        for c in range(C):
            acc[rank[p], c] = np.float32(acc[rank[p], c] + np.float32(
                depth[bn, d, h, w] * context[bn, c, h, w]))
    expect = acc.reshape(B, Z, X, Y, C).transpose(0, 1, 4, 2, 3).reshape(B, Z * C, X, Y)
    dx, bx, nx_t = ref.gen_dx_bx(*BOUNDS)
    out = ref.lss_bev_pool_depth(torch.from_numpy(geom), torch.from_numpy(depth),
                                 torch.from_numpy(context), dx, bx, nx_t)
    np.testing.assert_array_equal(out.numpy().view(np.uint32), expect.view(np.uint32))
    # the materialised-feature path of the oracle agrees bit for bit
    x = ref.lss_feature(torch.from_numpy(depth), torch.from_numpy(context), B, N)
    out2 = ref.lss_bev_pool(torch.from_numpy(geom), x, dx, bx, nx_t)
    assert torch.equal(out.view(torch.int32), out2.view(torch.int32))


@pytest.mark.parametrize('seed', [0, 4])
def test_lss_bev_pool_depth_gradients(seed):
    geom, depth, context = tiny_inputs(seed)
    B, N, D, fH, fW = geom.shape[:5]
    C = context.shape[1]
    rank, nx = c_ranks(geom, B)
    X, Y, Z = (int(v) for v in nx)
    dx, bx, nx_t = ref.gen_dx_bx(*BOUNDS)
    dt = torch.from_numpy(depth).double().requires_grad_(True)
    ct = torch.from_numpy(context).double().requires_grad_(True)
    out = ref.lss_bev_pool_depth(torch.from_numpy(geom), dt, ct, dx, bx, nx_t,
                                 dtype=torch.float64)
    g = np.random.default_rng(seed + 10).standard_normal(out.shape)
    (out * torch.from_numpy(g)).sum().backward()
    # chain rule by hand: G[rank, c] is the output gradient of cell `rank`
    G = g.reshape(B, Z, C, X, Y).transpose(0, 1, 3, 4, 2).reshape(-1, C)
    gd = np.zeros(depth.shape)
    gc = np.zeros(context.shape)
    HW = fH * fW
    for p in range(rank.size):
        if rank[p] < 0:
            continue
        bn, rem = divmod(p, D * HW)
        d, hw = divmod(rem, HW)
        h, w = divmod(hw, fW)
        for c in range(C):
            gd[bn, d, h, w] += G[rank[p], c] * float(context[bn, c, h, w])
            gc[bn, c, h, w] += G[rank[p], c] * float(depth[bn, d, h, w])
    np.testing.assert_allclose(dt.grad.numpy(), gd, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ct.grad.numpy(), gc, rtol=1e-12, atol=1e-12)
    # dropped points get no depth gradient
    flat = dt.grad.numpy().reshape(-1)
    assert np.all(flat[rank < 0] == 0.0)


def test_lss_bev_pool_depth_finite_differences():
    geom, depth, context = tiny_inputs(5, C=3)
    dx, bx, nx = ref.gen_dx_bx(*BOUNDS)
    gt = torch.from_numpy(geom)

    def f(d, c):
        return ref.lss_bev_pool_depth(gt, d, c, dx, bx, nx, dtype=torch.float64)

    d = torch.from_numpy(depth).double().requires_grad_(True)
    c = torch.from_numpy(context).double().requires_grad_(True)
    assert torch.autograd.gradcheck(f, (d, c), eps=1e-6, atol=1e-7)


def test_planted_depth_mistakes_are_caught():
    """A transposed (h, w) pixel map or a depth/context swap of the
    broadcast changes the pooled map of the brute-force check."""
    geom, depth, context = tiny_inputs(0, fH=2, fW=3)
    B, N = geom.shape[:2]
    good = brute_feature(depth, context, B, N)
    # pixel map with h and w exchanged (reshape instead of permute)
    bad_ctx = np.ascontiguousarray(context.reshape(context.shape[0], -1, 3, 2)
                                   .transpose(0, 1, 3, 2)).reshape(context.shape)
    bad = ref.lss_feature(torch.from_numpy(depth), torch.from_numpy(bad_ctx), B, N).numpy()
    assert not np.array_equal(bad, good)
    # rearrange to (b n) d h w c with b and n exchanged
    x = ref.lss_feature(torch.from_numpy(depth), torch.from_numpy(context), B, N).numpy()
    assert not np.array_equal(x.transpose(1, 0, 2, 3, 4, 5), good)
