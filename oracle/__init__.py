"""CPU oracle for the LSS ``bev_pool`` path -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import, call or link anything under ``oracle/``; the library path
(``bevfusion-triton_amd``) never does and fails loudly when its HIP library is
missing.

Contents
--------
``torch_fallback``  torch-CPU restatement of the reference's CPU fallback
                    (``ops/bev_pool/src/bev_pool_triton.py:12-48, 219-227``)
                    and of the vtransform quantise / kept-mask / compaction /
                    Z-collapse (``models/vtransforms/base.py:19-23, 131-165``),
                    plus the stable sort permutation and the interval
                    boundaries (``ops/bev_pool/bev_pool_legacy.py:56-61``)
                    applied to (b, z, x, y) ranks.
``seq``             ctypes front end of ``bevpool_seq.c``: an independent,
                    strictly sequential plain-C restatement of the same path
                    (quantise with x86 ``.long()`` semantics, ranks, stable
                    counting sort, intervals, point-order forward sums and the
                    backward gather).  Built by ``oracle/Makefile`` into
                    ``oracle/_build/liboracle_seq.so``.

How each function is pinned (checked against something other than itself)
is listed in the docstrings and exercised by ``tests/test_oracle.py``:
the reference's known-answer fixture (``tests/test_ops/test_bev_pool.py:57-84``,
committed as ``tests/golden/known_case.json``), the reference's input
rejection cases (``:122-131``), hand-derived closed-form vectors
(``tests/golden/quantize_edges.json``), brute-force pure-Python loops on tiny
inputs, ``numpy.add.at`` and the independent C restatement.
"""
