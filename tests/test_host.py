"""CPU tests of the host side: the C ABI library loads and exports every
symbol include/bevpool.h declares, argument validation returns the documented
status codes (these calls fail before any HIP call, so no GPU is needed), and
the Python surface mirrors the reference's checks and exception types."""
from __future__ import annotations

import ctypes
import json
import re

import numpy as np
import pytest
import torch

from conftest import GOLDEN, ROOT

HEADER = ROOT / 'include' / 'bevpool.h'


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(bevpool_\w+)\s*\(', text)))


def test_header_and_binding_agree(pkg):
    from bevfusion_triton_amd import _lib

    assert header_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.library()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.bevpool_abi_version() == 4
    assert lib.bevpool_last_error() == b''


C_CALLER = r"""
#include <stdio.h>
#include <string.h>
#include "bevpool.h"
int main(void) {
  if (bevpool_abi_version() != BEVPOOL_ABI_VERSION) return 2;
  if (bevpool_index_workspace_bytes(1000, 2000) == 0) return 3;
  /* refused before any HIP call: status and message, as documented */
  if (bevpool_sort(NULL, 1000, 2000, NULL, NULL, NULL, NULL, NULL, 0, NULL) != BEVPOOL_EINVAL)
    return 4;
  if (strlen(bevpool_last_error()) == 0) return 5;
  puts(bevpool_last_error());
  return 0;
}
"""


def test_c_caller_links_and_calls(pkg, tmp_path):
    """A plain C program (what a cgo / JNI / FFI binding compiles against)
    includes include/bevpool.h as C99, links the library directly (no torch
    in the process) and gets the documented status and message."""
    import shutil
    import subprocess

    cc = shutil.which('gcc') or shutil.which('cc')
    if cc is None:
        pytest.skip('no C compiler')
    lib = ROOT / 'bevfusion-triton_amd' / 'libbevpool_amd.so'
    src = tmp_path / 'caller.c'
    src.write_text(C_CALLER)
    exe = tmp_path / 'caller'
    subprocess.run([cc, '-std=c99', '-Wall', '-Werror', f'-I{ROOT / "include"}', str(src), '-o',
                    str(exe), str(lib), f'-Wl,-rpath,{lib.parent}'], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.strip()


def test_workspace_sizes(pkg):
    lib = pkg.library()
    small = lib.bevpool_index_workspace_bytes(1000, 100)
    big = lib.bevpool_index_workspace_bytes(2_000_000, 129600)
    assert 0 < small < big
    assert big >= 2_000_000 * 8  # ping-pong key buffer
    assert big % 256 == 0
    assert lib.bevpool_forward_scratch_bytes(129600, 80) == 129600 * 80 * 4
    assert lib.bevpool_backward_scratch_bytes(129600, 80, 2) == 129600 * 80 * 2


def test_status_codes_without_gpu(pkg):
    from bevfusion_triton_amd import _lib

    lib = pkg.library()
    meta = np.zeros(8, np.int32)
    ws = np.zeros(1 << 16, np.uint8)
    # unsupported dtype code
    st = lib.bevpool_forward(None, 7, 1, 1, 0, None, None, None, None, 1, 1, 1, 1, 1, 1, None,
                             None, 0, None)
    assert st == -1 and b'dtype' in lib.bevpool_last_error()
    # B*D*H*W out of range
    st = lib.bevpool_sort(None, 0, 0, None, None, None, meta.ctypes.data, ws.ctypes.data,
                          ws.size, None)
    assert st == -1 and b'B*D*H*W' in lib.bevpool_last_error()
    # workspace too small
    st = lib.bevpool_sort(meta.ctypes.data, 100000, 10, None, None, None, meta.ctypes.data,
                          ws.ctypes.data, 16, None)
    assert st == -3 and b'workspace' in lib.bevpool_last_error()
    # non-positive grid
    st = lib.bevpool_coord_ranks(None, 4, 0, 4, 1, 0, 1, 1, None, meta.ctypes.data,
                                 ws.ctypes.data, ws.size, None)
    assert st == -1
    # coords element size
    st = lib.bevpool_coord_ranks(None, 2, 0, 4, 1, 1, 1, 1, None, meta.ctypes.data,
                                 ws.ctypes.data, ws.size, None)
    assert st == -1 and b'coord_bytes' in lib.bevpool_last_error()
    with pytest.raises(_lib.BevPoolError, match='status -1'):
        _lib.check(lib.bevpool_forward(None, 7, 1, 1, 0, None, None, None, None, 1, 1, 1, 1, 1,
                                       1, None, None, 0, None), 'bevpool_forward')


def test_op_level_checks_mirror_reference(pkg):
    k = json.loads((GOLDEN / 'known_case.json').read_text())
    for case in k['reject']:
        feats = torch.zeros((4, 3), dtype=getattr(torch, case['feats_dtype']))
        coords = torch.zeros((4, 4), dtype=getattr(torch, case['coords_dtype']))
        with pytest.raises(TypeError):
            pkg.bev_pool(feats, coords, 1, 1, 1, 1)
    with pytest.raises(ValueError, match=r'feats must have shape \[N, C\]'):
        pkg.bev_pool(torch.zeros(4), torch.zeros(4, 4, dtype=torch.int32), 1, 1, 1, 1)
    with pytest.raises(ValueError, match=r'coords must have shape \[N, 4\]'):
        pkg.bev_pool(torch.zeros(4, 3), torch.zeros(4, 3, dtype=torch.int32), 1, 1, 1, 1)
    with pytest.raises(ValueError, match='same number of points'):
        pkg.bev_pool(torch.zeros(4, 3), torch.zeros(5, 4, dtype=torch.int32), 1, 1, 1, 1)
    with pytest.raises(ValueError, match='positive'):
        pkg.bev_pool(torch.zeros(4, 3), torch.zeros(4, 4, dtype=torch.int32), 1, 0, 1, 1)
    # 0-d integer tensors are accepted for the sizes (the vtransform passes nx[k])
    with pytest.raises(ValueError, match='positive'):
        pkg.bev_pool(torch.zeros(4, 3), torch.zeros(4, 4, dtype=torch.int32), torch.tensor(1),
                     torch.tensor(0), torch.tensor(1), torch.tensor(1))


def test_no_cpu_fallback(pkg):
    k = json.loads((GOLDEN / 'known_case.json').read_text())
    feats = torch.tensor(k['feats'])
    coords = torch.tensor(k['coords'], dtype=torch.int32)
    with pytest.raises(RuntimeError, match='no CPU fallback'):
        pkg.bev_pool(feats, coords, 1, 1, 2, 1)
    geom = torch.zeros(1, 1, 1, 1, 2, 3)
    x = torch.zeros(1, 1, 1, 1, 2, 4)
    with pytest.raises(RuntimeError, match='no CPU fallback'):
        pkg.lss_bev_pool(geom, x, *pkg.gen_dx_bx((-1, 1, 1), (-1, 1, 1), (-1, 1, 2)))


def test_binding_keeps_cpu_branch(pkg):
    """The op-level binding a maintainer adds to the reference replaces only the
    GPU branch of ``bev_pool_triton.py:219-227``: CPU tensors still reach the reference's
    CPU fallback (restated in oracle/ for this test) and give the reference's
    known answer (``tests/test_ops/test_bev_pool.py:57-84``); calling this
    package directly with CPU tensors raises the documented error."""
    from oracle import torch_fallback as ref

    def bev_pool(feats, coords, B, D, H, W):  # the binding: GPU tensors to this package
        ref.check_inputs(feats, coords, B, D, H, W)
        if feats.is_cuda:
            return pkg.bev_pool(feats, coords, B, D, H, W)
        out = ref.bev_pool_cpu(feats, coords, B, D, H, W)
        return out.permute(0, 4, 1, 2, 3).contiguous()

    k = json.loads((GOLDEN / 'known_case.json').read_text())
    feats = torch.tensor(k['feats'], requires_grad=True)
    coords = torch.tensor(k['coords'], dtype=torch.int32)
    out = bev_pool(feats, coords, k['B'], k['D'], k['H'], k['W'])
    assert out.is_contiguous() and list(out.shape) == k['expected_shape']
    assert torch.equal(out.detach(), torch.tensor(k['expected']))
    out.sum().backward()
    assert torch.equal(feats.grad, torch.ones(3, 2))
    with pytest.raises(RuntimeError, match='runs the bev_pool path on a ROCm GPU only'):
        pkg.bev_pool(feats.detach(), coords, k['B'], k['D'], k['H'], k['W'])


def test_gen_dx_bx_matches_reference_restatement(pkg):
    from oracle import torch_fallback as ref

    for bounds in [((-54.0, 54.0, 0.3), (-54.0, 54.0, 0.3), (-10.0, 10.0, 20.0)),
                   ((-51.2, 51.2, 0.4), (-51.2, 51.2, 0.4), (-10.0, 10.0, 20.0)),
                   ((-54.0, 54.0, 0.15), (-54.0, 54.0, 0.15), (-10.0, 10.0, 20.0))]:
        for a, b in zip(pkg.gen_dx_bx(*bounds), ref.gen_dx_bx(*bounds)):
            assert a.dtype == b.dtype and torch.equal(a, b)


def test_host_grid_offset_bits(pkg):
    q = json.loads((GOLDEN / 'quantize_edges.json').read_text())['grid']
    offset, dx, nx = pkg.host_grid(*pkg.gen_dx_bx(q['xbound'], q['ybound'], q['zbound']))
    assert offset.view(np.uint32).tolist() == q['offset_f32_bits']
    assert dx.view(np.uint32).tolist() == q['dx_f32_bits']
    assert nx == q['nx']


def test_transform_module_grid_cache(pkg):
    m = pkg.BevPoolTransform((-54.0, 54.0, 0.3), (-54.0, 54.0, 0.3), (-10.0, 10.0, 20.0))
    g0 = m.grid()
    assert g0[2] == [360, 360, 1]
    with torch.no_grad():
        m.dx.mul_(2.0)  # in-place change is picked up
    assert m.grid()[1][0] == np.float32(0.6)


def test_synthetic_rig_shapes(pkg):
    from bevfusion_triton_amd import synthetic

    spec = synthetic.CASES['det']
    geom = synthetic.make_geometry(spec)
    assert geom.shape == (1, 6, 118, 32, 88, 3)
    assert geom[..., 0].numel() == 1_993_728
    # cameras 1.5 m high: the nearest depth bin lies within a few metres
    assert torch.isfinite(geom).all()


def test_status_codes_new_entry_points_without_gpu(pkg):
    """Argument checks of the depth-weighted, planar and camera entry points
    return before any HIP call."""
    lib = pkg.library()
    meta = np.zeros(8, np.int32)
    rank = np.zeros(64, np.int32)
    ws = np.zeros(1 << 16, np.uint8)
    buf = np.zeros(256, np.float32)
    p = buf.ctypes.data
    # meta_report: null meta or destination
    assert lib.bevpool_meta_report(None, p, None) == -1
    assert lib.bevpool_meta_report(meta.ctypes.data, None, None) == -1
    assert b'null' in lib.bevpool_last_error()
    # forward_depth: C must be a positive multiple of 4
    st = lib.bevpool_forward_depth(p, p, 6, 0, 1, 1, None, p, p, meta.ctypes.data, 1, 1, 1, 1,
                                   1, 1, p, p, 1 << 20, None)
    assert st == -1 and b'multiple of 4' in lib.bevpool_last_error()
    # forward_depth: n_points must be a multiple of D*HW
    st = lib.bevpool_forward_depth(p, p, 8, 7, 2, 2, None, p, p, meta.ctypes.data, 1, 1, 1, 1,
                                   1, 1, p, p, 1 << 20, None)
    assert st == -1 and b'multiple of D*HW' in lib.bevpool_last_error()
    # backward_depth: C <= 256, and 2*D + C <= 1024
    st = lib.bevpool_backward_depth(p, 1, 1, 1, 300, None, 4, 1, 4, p, p, p, p, 1, 1, 1, p, p,
                                    1, 1, p, 1 << 30, None)
    assert st == -1 and b'[1, 256]' in lib.bevpool_last_error()
    st = lib.bevpool_backward_depth(p, 1, 1, 1, 80, rank.ctypes.data, 500, 500, 1, p, p, p, p, 1,
                                    1, 1, p, p, 1, 1, p, 1 << 30, None)
    assert st == -1 and b'2*D + C' in lib.bevpool_last_error()
    # planar_rows / backward_planar
    st = lib.bevpool_planar_rows(p, 1, 1, 1, 0, 4, p, None)
    assert st == -1 and b'planar shape' in lib.bevpool_last_error()
    assert lib.bevpool_planar_rows(p, 1, 1, 0, 4, 4, p, None) == 0  # empty: nothing to do
    # a launch past the 2^32 work-item grid is refused, not truncated: the
    # element-wise form (C = 6, 2^30 rows) and the tiled form (1,024 x 2^26 rows)
    st = lib.bevpool_planar_rows(p, 6 << 30, 1 << 30, 1, 6, 1 << 30, p, None)
    assert st == -1 and b'work-item grid' in lib.bevpool_last_error()
    st = lib.bevpool_planar_rows(p, 80 << 26, 1 << 26, 1024, 80, 1 << 26, p, None)
    assert st == -1 and b'work-item grid' in lib.bevpool_last_error()
    st = lib.bevpool_backward_planar(p, 1, 1, 1, 4, rank.ctypes.data, 10, p, p, 1, 1, 1, 4, p,
                                     1, 1, p, 1 << 20, None)
    assert st == -1 and b'multiple of S' in lib.bevpool_last_error()
    # quantize_cameras: sizes and required matrices
    f3 = lambda *v: (ctypes.c_float * 3)(*v)
    i3 = lambda *v: (ctypes.c_int32 * 3)(*v)
    st = lib.bevpool_quantize_cameras(p, 0, 1, 1, p, p, p, p, p, None, None, 1, 1,
                                      f3(0, 0, 0), f3(1, 1, 1), i3(4, 4, 1), rank.ctypes.data,
                                      meta.ctypes.data, ws.ctypes.data, ws.size, None)
    assert st == -1 and b'frustum/camera sizes' in lib.bevpool_last_error()
    st = lib.bevpool_quantize_cameras(p, 2, 2, 2, None, p, p, p, p, None, None, 1, 1,
                                      f3(0, 0, 0), f3(1, 1, 1), i3(4, 4, 1), rank.ctypes.data,
                                      meta.ctypes.data, ws.ctypes.data, ws.size, None)
    assert st == -1 and b'camera matrices' in lib.bevpool_last_error()


def test_legacy_ext_module_surface(pkg):
    """The reference's tests/test_ops/test_bev_pool.py:50-54 against the
    drop-in legacy module: an ``ext_module`` with both extension functions."""
    legacy_ref_mod = pkg.legacy
    assert hasattr(legacy_ref_mod, 'ext_module')
    assert hasattr(legacy_ref_mod.ext_module, 'bev_pool_forward')
    assert hasattr(legacy_ref_mod.ext_module, 'bev_pool_backward')


def test_op_and_legacy_status_codes(pkg):
    lib = pkg.library()
    ws = np.zeros(1 << 12, np.uint8)
    need = lib.bevpool_op_workspace_bytes(1000, 100, 8)
    ix = lib.bevpool_op_index_bytes(1000, 100)
    sc = lib.bevpool_op_scratch_bytes(1000, 100, 8)
    assert need == ix + sc and ix % 256 == 0 and sc % 256 == 0
    assert ix >= 1000 * 12 + 100 * 8 and sc >= 100 * 8 * 4
    st = lib.bevpool_op_forward(None, 0, 8, 8, None, 4, 4, 1000, 1, 1, 10, 10, None,
                                ws.ctypes.data, ws.size, ws.ctypes.data, ws.size, None, None)
    assert st == -3 and b'op index buffer' in lib.bevpool_last_error()
    big = np.zeros(ix, np.uint8)
    st = lib.bevpool_op_forward(None, 0, 8, 8, None, 4, 4, 1000, 1, 1, 10, 10, None,
                                big.ctypes.data, big.size, ws.ctypes.data, 256, None, None)
    assert st == -3 and b'op scratch' in lib.bevpool_last_error()
    st = lib.bevpool_op_forward(None, 0, 8, 8, None, 4, 4, 10, 1, 0, 10, 10, None,
                                ws.ctypes.data, ws.size, ws.ctypes.data, ws.size, None, None)
    assert st == -1
    st = lib.bevpool_op_backward(None, 0, 1, 1, 1, 8, 1000, 1, 1, 10, 10, None, 8, 1,
                                 ws.ctypes.data, 256, ws.ctypes.data, ws.size, None)
    assert st == -3 and b'op index buffer' in lib.bevpool_last_error()
    st = lib.bevpool_legacy_forward(None, 10, 0, None, None, None, 0, None, 1, 1, 1, 1,
                                    ws.ctypes.data, None, None)
    assert st == -1 and b'C must be positive' in lib.bevpool_last_error()
    st = lib.bevpool_runs(None, 2, 10, None, None, ws.ctypes.data, ws.ctypes.data, ws.size, None)
    assert st == -1 and b'rank_bytes' in lib.bevpool_last_error()
    st = lib.bevpool_runs(None, 8, 1 << 20, None, None, ws.ctypes.data, ws.ctypes.data, 16, None)
    assert st == -3
