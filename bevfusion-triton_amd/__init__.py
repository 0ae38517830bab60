"""bevfusion-triton_amd -- MI355X-native (gfx950) LSS camera-to-BEV pooling.

A from-scratch HIP implementation of the ``bev_pool`` hot path of
ziyangyeh/bevfusion-triton behind the reference's own Python surface:

  bev_pool(feats, coords, B, D, H, W)       ops/bev_pool/src/bev_pool_triton.py:219-227
  BevPoolFunction                           ops/bev_pool/src/bev_pool_triton.py:153-216
  gen_dx_bx / BevPoolTransform.bev_pool     models/vtransforms/base.py:19-23, 131-165
  lss_bev_pool                              the same as a function
  lss_bev_pool_depth                        the same fused with depth_lss.py:91-94's
                                            depth (x) context product
  lss_index_cameras / CameraIndex           base.py:82-126 get_geometry fused into the
                                            quantisation (cacheable for static cameras)
  legacy.bev_pool / legacy.QuickCumsumCuda  ops/bev_pool/bev_pool_legacy.py:53-108

The kernels live in ``csrc/bevpool.hip`` and are reached through the C ABI of
``include/bevpool.h`` (``libbevpool_amd.so``, loaded by ``_lib``).  There is no
CPU or Triton fallback.

The directory name is not a Python identifier; load it with
``__graft_entry__.load_package()`` (registers it as ``bevfusion_triton_amd``).
"""
from . import legacy
from ._lib import BevPoolError, LibraryNotBuilt, library
from .bev_pool import BevPoolFunction, BevPoolIndexExport, bev_pool, check_errors
from .vtransform import (BevPoolTransform, CameraIndex, LSSIndexExport, create_frustum, gen_dx_bx, host_grid, lss_bev_pool, lss_bev_pool_depth,
                         lss_index_cameras)

__all__ = [
    'BevPoolError',
    'BevPoolFunction',
    'BevPoolIndexExport',
    'BevPoolTransform',
    'CameraIndex',
    'LSSIndexExport',
    'LibraryNotBuilt',
    'bev_pool',
    'check_errors',
    'create_frustum',
    'gen_dx_bx',
    'host_grid',
    'legacy',
    'library',
    'lss_bev_pool',
    'lss_bev_pool_depth',
    'lss_index_cameras',
]
