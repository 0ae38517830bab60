"""Pins the oracle's restatement of the reference's legacy extension
(``ops/bev_pool/csrc/bev_pool_cpu.cpp:22-94``, kernels
``bev_pool_cuda.cu:20-98``; ``oracle.torch_fallback.legacy_forward`` /
``legacy_backward`` / ``runs``) against things other than itself: the
reference's known-answer fixture, the CPU fallback (itself pinned by brute
force in ``test_oracle.py``) on the runs ``bev_pool_legacy.py`` builds, and
numpy brute-force loops on arbitrary intervals.  Planted mistakes (the
interval's last row giving the cell, a reversed summation, a dropped first
row) are shown to fail these pins."""
from __future__ import annotations

import json

import numpy as np
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from conftest import GOLDEN
from oracle import torch_fallback as ref


def _known():
    k = json.loads((GOLDEN / 'known_case.json').read_text())
    return (torch.tensor(k['feats'], dtype=torch.float32),
            torch.tensor(k['coords'], dtype=torch.int32), (k['B'], k['D'], k['H'], k['W']),
            torch.tensor(k['expected'], dtype=torch.float32))


def test_known_case_through_legacy_runs():
    """bev_pool_legacy.py:99-108 on the reference's fixture
    (tests/test_ops/test_bev_pool.py:57-84): legacy ranks, sort, runs, the
    extension's forward, permute -- the fixture's expected grid."""
    feats, coords, (B, D, H, W), expected = _known()
    ranks = ref.legacy_ranks(coords, B, D, H, W)
    order = torch.sort(ranks, stable=True).indices
    starts, lengths = ref.runs(ranks[order])
    assert starts.tolist() == [0, 2] and lengths.tolist() == [2, 1]
    out, bad = ref.legacy_forward(feats[order], coords[order].int(), lengths, starts, B, D, H, W)
    assert bad == 0
    assert torch.equal(out.permute(0, 4, 1, 2, 3).contiguous(), expected)


@st.composite
def grids(draw):
    B, D, H, W = (draw(st.integers(1, 3)) for _ in range(4))
    N = draw(st.integers(0, 40))
    C = draw(st.integers(1, 5))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    coords = np.stack([rng.integers(0, H, N), rng.integers(0, W, N), rng.integers(0, D, N),
                       rng.integers(0, B, N)], 1).astype(np.int32)
    feats = (rng.standard_normal((N, C)) * 10.0 ** rng.integers(-3, 6, (N, C))).astype(np.float32)
    return feats, coords, (B, D, H, W), rng


@settings(max_examples=60, deadline=None)
@given(grids())
def test_legacy_forward_on_sorted_runs_equals_fallback(inp):
    """The legacy module's own flow (sort by the legacy rank, one run per
    cell, bev_pool_legacy.py:56-73, 102-106) with a stable sort gives the CPU
    fallback's index_add_ sums bit for bit (both add a cell's points in point
    order from +0.0)."""
    feats, coords, sizes, _ = inp
    f, c = torch.from_numpy(feats), torch.from_numpy(coords)
    ranks = ref.legacy_ranks(c, *sizes)
    order = torch.sort(ranks, stable=True).indices
    starts, lengths = ref.runs(ranks[order])
    out, bad = ref.legacy_forward(f[order], c[order], lengths, starts, *sizes)
    assert bad == 0
    fb = ref.bev_pool_cpu(f, c, *sizes)
    assert torch.equal(out.view(torch.int32), fb.view(torch.int32))


def brute_legacy(x, geom, starts, lengths, sizes, reverse=False, last_row=False, skip_first=False):
    """Per-channel scalar loops, np.float32 rounding after every add."""
    B, D, H, W = sizes
    n, C = x.shape
    out = np.zeros((B * D * H * W, C), np.float32)
    bad = 0
    for s, m in zip(starts.tolist(), lengths.tolist()):
        if not (0 <= s < n and 0 <= m and s + m <= n):
            bad += 1
            continue
        r = s + m - 1 if (last_row and m > 0) else s
        gx, gy, gz, gb = (int(v) for v in geom[r])
        if not (0 <= gx < H and 0 <= gy < W and 0 <= gz < D and 0 <= gb < B):
            bad += 1
            continue
        cell = ((gb * D + gz) * H + gx) * W + gy
        rows = list(range(s, s + m))
        if reverse:
            rows = rows[::-1]
        if skip_first:
            rows = rows[1:]
        for c in range(C):
            acc = np.float32(0.0)
            for i in rows:
                acc = np.float32(acc + x[i, c])
            out[cell, c] = acc
    return out.reshape(B, D, H, W, C), bad


@st.composite
def arbitrary_intervals(draw):
    feats, coords, sizes, rng = draw(grids())
    n = feats.shape[0]
    k = draw(st.integers(0, 8))
    starts = rng.integers(-2, n + 3, k).astype(np.int32)
    lengths = rng.integers(-1, 6, k).astype(np.int32)
    return feats, coords, sizes, starts, lengths


@settings(max_examples=80, deadline=None)
@given(arbitrary_intervals())
def test_legacy_forward_brute_force(inp):
    """Arbitrary (also invalid, empty and coarse) intervals: the cell of the
    first row, the rows summed in order, invalid intervals skipped."""
    feats, coords, sizes, starts, lengths = inp
    out, bad = ref.legacy_forward(torch.from_numpy(feats), torch.from_numpy(coords),
                                  torch.from_numpy(lengths), torch.from_numpy(starts), *sizes)
    exp, ebad = brute_legacy(feats, coords, starts, lengths, sizes)
    # two intervals of one cell race in the reference; both restatements
    # here are sequential, so the later interval wins in both
    assert bad == ebad
    np.testing.assert_array_equal(out.numpy().view(np.uint32), exp.view(np.uint32))


@settings(max_examples=60, deadline=None)
@given(arbitrary_intervals())
def test_legacy_backward_brute_force(inp):
    feats, coords, sizes, starts, lengths = inp
    B, D, H, W = sizes
    n, C = feats.shape
    g = np.random.default_rng(5).standard_normal((B, D, H, W, C)).astype(np.float32)
    xg, bad = ref.legacy_backward(torch.from_numpy(g), torch.from_numpy(coords),
                                  torch.from_numpy(lengths), torch.from_numpy(starts), *sizes)
    exp = np.zeros((n, C), np.float32)
    ebad = 0
    gf = g.reshape(-1, C)
    for s, m in zip(starts.tolist(), lengths.tolist()):
        if not (0 <= s < n and 0 <= m and s + m <= n):
            ebad += 1
            continue
        gx, gy, gz, gb = (int(v) for v in coords[s])
        if not (0 <= gx < H and 0 <= gy < W and 0 <= gz < D and 0 <= gb < B):
            ebad += 1
            continue
        for i in range(s, s + m):
            exp[i] = gf[((gb * D + gz) * H + gx) * W + gy]
    assert bad == ebad
    np.testing.assert_array_equal(xg.numpy(), exp)


@settings(max_examples=60, deadline=None)
@given(st.lists(st.integers(-3, 3), max_size=30))
def test_runs_brute_force(values):
    """bev_pool_legacy.py:56-61 on any (unsorted) rank array: a run starts
    where the value changes."""
    r = torch.tensor(values, dtype=torch.int64)
    starts, lengths = ref.runs(r)
    bs, bl = [], []
    for i, v in enumerate(values):
        if i == 0 or v != values[i - 1]:
            bs.append(i)
            bl.append(1)
        else:
            bl[-1] += 1
    assert starts.tolist() == bs and lengths.tolist() == bl


def test_planted_mistakes_are_caught():
    """The pins above fail for plausible mistakes: the interval's cell taken
    from its last row, the rows added in reverse, the first row dropped."""
    rng = np.random.default_rng(11)
    sizes = (1, 1, 4, 4)
    coords = np.stack([rng.integers(0, 4, 12), rng.integers(0, 4, 12), np.zeros(12, int),
                       np.zeros(12, int)], 1).astype(np.int32)
    feats = (rng.standard_normal((12, 3)) * 10.0 ** rng.integers(-3, 6, (12, 3))).astype(np.float32)
    starts = np.array([0, 5], np.int32)
    lengths = np.array([5, 7], np.int32)  # coarse runs: rows of several cells
    good, _ = ref.legacy_forward(torch.from_numpy(feats), torch.from_numpy(coords),
                                 torch.from_numpy(lengths), torch.from_numpy(starts), *sizes)
    for kw in ({'last_row': True}, {'reverse': True}, {'skip_first': True}):
        bad, _ = brute_legacy(feats, coords, starts, lengths, sizes, **kw)
        assert not np.array_equal(good.numpy().view(np.uint32), bad.view(np.uint32)), kw
    # and the known case catches a dropped first row
    f, c, s, expected = _known()
    bad, _ = brute_legacy(f.numpy(), c.numpy(), np.array([0, 2], np.int32),
                          np.array([2, 1], np.int32), s, skip_first=True)
    assert not np.array_equal(bad.transpose(0, 4, 1, 2, 3), expected.numpy())
