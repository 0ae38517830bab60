"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

Nothing here runs or imports the reference.  The fixtures are data:

known_case.json
    The reference's only value-pinning fixture, the inputs and expected
    output of tests/test_ops/test_bev_pool.py:57-84 (3 points, C=2, B=1,
    D=1, H=2, W=1), plus its input-rejection cases (:122-131).

quantize_edges.json
    Expected cell / kept flag of hand-picked geometry points for the det grid
    (models/vtransforms/base.py:139-156), derived here WITHOUT float
    hardware: every fp32 operation of ((g - (bx - dx/2)) / dx) is evaluated
    exactly with fractions.Fraction and rounded to nearest-even fp32 by
    `round_f32`, then truncated toward zero as `.long()` does.

order_case.json
    Pooling of values whose fp32 sum depends on the summation order, with
    expected sums worked out by hand for the increasing-point-index order.
"""
from __future__ import annotations

import json
import math
import struct
from fractions import Fraction
from pathlib import Path

HERE = Path(__file__).resolve().parent


# ---------------------------------------------------------------------------
# exact fp32 arithmetic
# ---------------------------------------------------------------------------
def f32_bits(v: float) -> int:
    return struct.unpack('<I', struct.pack('<f', v))[0]


def f32_value(bits: int) -> Fraction:
    """Exact rational value of a finite fp32 bit pattern."""
    sign = -1 if bits >> 31 else 1
    e = (bits >> 23) & 0xFF
    m = bits & 0x7FFFFF
    if e == 0:
        return sign * Fraction(m, 1 << 149)
    return sign * Fraction(m | 0x800000, 1) * Fraction(2) ** (e - 150)


def round_f32(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 value (ties to even).
    Only the normal range is needed here."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)  # q integer count of ulps, r remainder
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp


def f32(x) -> Fraction:
    """fp32 value nearest to a decimal literal (Python float -> fp32, as
    torch.Tensor([...]) does: double first, then nearest-even to fp32)."""
    return round_f32(Fraction(float(x)))


def trunc_long(q: Fraction):
    """torch .long() of a finite fp32 value: truncation toward zero."""
    return int(q) if q >= 0 else -int(-q)


def det_grid():
    # base.py:19-23 with swint_v0p075.yaml:26-27 and depth_lss.yaml:13
    bounds = [(-54.0, 54.0, 0.3), (-54.0, 54.0, 0.3), (-10.0, 10.0, 20.0)]
    dx = [f32(b[2]) for b in bounds]
    bx = [f32(b[0] + b[2] / 2.0) for b in bounds]
    nx = [int((b[1] - b[0]) / b[2]) for b in bounds]
    # base.py:139: (bx - dx / 2.0) in fp32: dx/2 is exact, the subtraction rounds
    offset = [round_f32(bx[k] - dx[k] / 2) for k in range(3)]
    return bounds, dx, nx, offset


def quantize_edges():
    bounds, dx, nx, offset = det_grid()
    # (label, x, y, z) geometry in metres (fp32 values of the decimal literals)
    pts = [
        ('origin corner', -54.0, -54.0, -10.0),
        ('x just below the low edge (q in (-1,0)) -> cell 0', -54.05, 0.0, 0.0),
        ('x = -54.3 m: q = -0.99999... -> cell 0 (kept)', -54.3, 0.0, 0.0),
        ('x = -54.31 m: q < -1 -> dropped', -54.31, 0.0, 0.0),
        ('x = 1 m -> cell 183; y = 0 m: q = 179.99999... rounds to 180.0', 1.0, 0.0, 0.0),
        ('x = +54 m: q rounds to 360.0 -> dropped', 54.0, 10.0, 0.0),
        ('x = +54.01 m: q > 360 -> dropped', 54.01, 10.0, 0.0),
        ('x = 53.99 m: last cell 359', 53.99, 10.0, 0.0),
        ('z = +10 m: q = 1 -> dropped', 0.0, 0.0, 10.0),
        ('z = 9.999 m: kept', 0.0, 0.0, 9.999),
        ('z = -10.5 m: q in (-1,0) -> kept', 0.0, 0.0, -10.5),
        ('z = -30 m: q = -1 -> dropped', 0.0, 0.0, -30.0),
        ('interior point', 12.345, -23.456, 1.25),
    ]
    out = []
    for label, *g in pts:
        gf = [f32(v) for v in g]
        q = []
        for k in range(3):
            diff = round_f32(gf[k] - offset[k])
            q.append(round_f32(diff / dx[k]))
        qi = [trunc_long(v) for v in q]
        kept = all(0 <= qi[k] < nx[k] for k in range(3))
        rank = ((0 * nx[2] + qi[2]) * nx[0] + qi[0]) * nx[1] + qi[1] if kept else -1
        out.append({
            'label': label,
            'geom_f32_bits': [f32_bits(float(v)) for v in gf],
            'q': [float(v) for v in q],
            'cell_xyz': qi,
            'kept': kept,
            'rank': rank,
        })
    # non-finite geometry is dropped (NaN and +-inf compare false / out of range)
    for label, v in [('NaN x', float('nan')), ('+inf y', float('inf')), ('-inf z', float('-inf'))]:
        g = [1.0, 1.0, 1.0]
        g[['NaN x', '+inf y', '-inf z'].index(label)] = v
        out.append({'label': label, 'geom_f32_bits': [f32_bits(c) for c in g], 'q': None,
                    'cell_xyz': None, 'kept': False, 'rank': -1})
    return {
        'grid': {'xbound': list(bounds[0]), 'ybound': list(bounds[1]), 'zbound': list(bounds[2]),
                 'dx_f32_bits': [f32_bits(float(v)) for v in dx],
                 'offset_f32_bits': [f32_bits(float(v)) for v in offset], 'nx': nx},
        'points': out,
    }


def known_case():
    # tests/test_ops/test_bev_pool.py:57-84 and :122-131 (data only)
    return {
        'feats': [[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]],
        'coords': [[0, 0, 0, 0], [0, 0, 0, 0], [1, 0, 0, 0]],
        'B': 1, 'D': 1, 'H': 2, 'W': 1,
        'expected': [[[[[4.0], [5.0]]], [[[6.0], [6.0]]]]],
        'expected_shape': [1, 2, 1, 2, 1],
        'reject': [
            {'feats_dtype': 'int32', 'coords_dtype': 'int32', 'error': 'TypeError'},
            {'feats_dtype': 'float32', 'coords_dtype': 'float32', 'error': 'TypeError'},
        ],
    }


def order_case():
    """One channel, B=D=1, H=1, W=3 (cells y=0,1,2).  Points in index order:
         p0 -> y=1: 1e8       p1 -> y=0: -0.0     p2 -> y=1: -1e8
         p3 -> y=2: 1.0       p4 -> y=1: 1.0      p5 -> y=2: 2**-24
         p6 -> y=2: 2**-24
    Cell y=1 in point order: ((0 + 1e8) + -1e8) + 1 = 1.0; any order that adds
    1 before -1e8 loses it (1e8 + 1 rounds back to 1e8) and gives 0.0.
    Cell y=0: 0 + (-0.0) = +0.0 (the accumulator starts at +0.0).
    Cell y=2: ((0 + 1) + 2^-24) + 2^-24 = 1.0 (each 2^-24 is half an ulp of
    1 and ties to even); adding the two small values first gives 1 + 2^-23.
    """
    feats = [[1e8], [-0.0], [-1e8], [1.0], [1.0], [2.0 ** -24], [2.0 ** -24]]
    coords = [[0, 1, 0, 0], [0, 0, 0, 0], [0, 1, 0, 0], [0, 2, 0, 0], [0, 1, 0, 0],
              [0, 2, 0, 0], [0, 2, 0, 0]]
    return {
        'feats_f32_bits': [[f32_bits(v[0])] for v in feats],
        'coords': coords, 'B': 1, 'D': 1, 'H': 1, 'W': 3,
        'expected_f32_bits': [f32_bits(0.0), f32_bits(1.0), f32_bits(1.0)],
        'wrong_order_f32_bits': {'y=1 reversed': f32_bits(0.0),
                                 'y=2 small-first': f32_bits(1.0 + 2.0 ** -23)},
    }


def main():
    for name, obj in [('known_case.json', known_case()), ('quantize_edges.json', quantize_edges()),
                      ('order_case.json', order_case())]:
        (HERE / name).write_text(json.dumps(obj, indent=1) + '\n')
        print('wrote', HERE / name)


if __name__ == '__main__':
    main()
