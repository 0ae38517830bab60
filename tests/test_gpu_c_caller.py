"""The op level driven from plain C, the way a non-Python binding would call
the library: a C99 program allocates device memory with the HIP runtime,
calls bevpool_op_forward / bevpool_op_backward through include/bevpool.h
and compares the results bit for bit with the C oracle
(oracle/bevpool_seq.c, linked as test infrastructure).  No torch is loaded
in that process, so the library runs on the image's own HIP runtime."""
from __future__ import annotations

import shutil
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

PROGRAM = r"""
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <hip/hip_runtime_api.h>
#include "bevpool.h"

int64_t oracle_coord_ranks(const int64_t *coords, int64_t n, int64_t B, int64_t D, int64_t H,
                           int64_t W, int64_t *rank);
void oracle_forward(const float *x, int64_t ld, int64_t C, const int64_t *rank, int64_t n,
                    int64_t n_cells, float *out);
void oracle_backward(const uint32_t *grad_rows, int64_t C, const int64_t *rank, int64_t n,
                     uint32_t *x_grad);

#define CHECK(x) do { if (!(x)) { printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #x); return 1; } } while (0)

static uint32_t lcg = 12345u;
static uint32_t next(void) { lcg = lcg * 1664525u + 1013904223u; return lcg >> 8; }
static float frand(void) { return (float)next() / 16777216.0f * 2.0f - 1.0f; }

int main(void) {
  const int64_t N = 30000, C = 24, B = 2, D = 2, H = 30, W = 40;
  const int64_t cells = B * D * H * W;
  int32_t *coords = malloc(N * 4 * sizeof(int32_t));
  int64_t *coords64 = malloc(N * 4 * sizeof(int64_t));
  float *feats = malloc(N * C * sizeof(float));
  int64_t *rank = malloc(N * sizeof(int64_t));
  int64_t nbad_exp = 0, first_bad = -1;
  for (int64_t p = 0; p < N; ++p) {
    int32_t c[4] = {(int32_t)(next() % H), (int32_t)(next() % W), (int32_t)(next() % D),
                    (int32_t)(next() % B)};
    if (next() % 97 == 0) c[3] = (int32_t)B;  /* outside the grid */
    for (int k = 0; k < 4; ++k) { coords[p * 4 + k] = c[k]; coords64[p * 4 + k] = c[k]; }
    for (int64_t k = 0; k < C; ++k) feats[p * C + k] = frand();
  }
  nbad_exp = oracle_coord_ranks(coords64, N, B, D, H, W, rank);
  for (int64_t p = 0; p < N && first_bad < 0; ++p) if (rank[p] < 0) first_bad = p;
  CHECK(nbad_exp > 0);
  float *rows = malloc(cells * C * sizeof(float));
  oracle_forward(feats, C, C, rank, N, cells, rows);

  const size_t ix_bytes = bevpool_op_index_bytes(N, cells);
  const size_t sc_bytes = bevpool_op_scratch_bytes(N, cells, C);
  CHECK(bevpool_op_workspace_bytes(N, cells, C) == ix_bytes + sc_bytes);
  void *d_feats, *d_coords, *d_out, *d_ix, *d_sc, *d_grad, *d_xg;
  CHECK(hipMalloc(&d_feats, N * C * 4) == hipSuccess);
  CHECK(hipMalloc(&d_coords, N * 16) == hipSuccess);
  CHECK(hipMalloc(&d_out, cells * C * 4) == hipSuccess);
  CHECK(hipMalloc(&d_ix, ix_bytes) == hipSuccess);
  CHECK(hipMalloc(&d_sc, sc_bytes) == hipSuccess);
  CHECK(hipMalloc(&d_grad, cells * C * 4) == hipSuccess);
  CHECK(hipMalloc(&d_xg, N * C * 4) == hipSuccess);
  CHECK(hipMemcpy(d_feats, feats, N * C * 4, hipMemcpyHostToDevice) == hipSuccess);
  CHECK(hipMemcpy(d_coords, coords, N * 16, hipMemcpyHostToDevice) == hipSuccess);

  /* forward: (B, C, D, H, W) contiguous */
  int st = bevpool_op_forward(d_feats, BEVPOOL_F32, C, (int32_t)C, d_coords, 4, 4, N,
                              (int32_t)B, (int32_t)D, (int32_t)H, (int32_t)W, d_out, d_ix,
                              ix_bytes, d_sc, sc_bytes, NULL, NULL);
  if (st) printf("op_forward: %s\n", bevpool_last_error());
  CHECK(st == BEVPOOL_OK);
  CHECK(hipDeviceSynchronize() == hipSuccess);
  float *out = malloc(cells * C * 4);
  int32_t meta[BEVPOOL_META_LEN];
  CHECK(hipMemcpy(out, d_out, cells * C * 4, hipMemcpyDeviceToHost) == hipSuccess);
  CHECK(hipMemcpy(meta, d_ix, sizeof(meta), hipMemcpyDeviceToHost) == hipSuccess);
  CHECK(meta[BEVPOOL_META_N_KEPT] == N - nbad_exp);
  CHECK(meta[BEVPOOL_META_N_BAD] == nbad_exp);
  CHECK(meta[BEVPOOL_META_FIRST_BAD] == first_bad);
  const int64_t per_b = C * D * H * W, per_c = D * H * W;
  int64_t bad_fwd = 0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t s = 0; s < D * H * W; ++s) {
        const float got = out[b * per_b + c * per_c + s];
        const float exp = rows[(b * D * H * W + s) * C + c];
        if (memcmp(&got, &exp, 4)) ++bad_fwd;
      }
  CHECK(bad_fwd == 0);

  /* backward: x_grad[p] = grad[b, :, z, x, y], zero rows for invalid coords */
  float *grad = malloc(cells * C * 4);
  float *grad_rows = malloc(cells * C * 4);
  for (int64_t i = 0; i < cells * C; ++i) grad[i] = frand();
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t s = 0; s < D * H * W; ++s)
        grad_rows[(b * D * H * W + s) * C + c] = grad[b * per_b + c * per_c + s];
  CHECK(hipMemcpy(d_grad, grad, cells * C * 4, hipMemcpyHostToDevice) == hipSuccess);
  /* the forward's scratch is not needed any more: the backward gets a fresh
     one, filled with junk first */
  CHECK(hipFree(d_sc) == hipSuccess);
  const size_t bsc_bytes = bevpool_backward_scratch_bytes(cells, (int32_t)C, BEVPOOL_F32);
  CHECK(bsc_bytes <= sc_bytes);
  CHECK(hipMalloc(&d_sc, bsc_bytes) == hipSuccess);
  CHECK(hipMemset(d_sc, 0x5a, bsc_bytes) == hipSuccess);
  st = bevpool_op_backward(d_grad, BEVPOOL_F32, per_b, per_c, H * W, (int32_t)C, N,
                           (int32_t)B, (int32_t)D, (int32_t)H, (int32_t)W, d_xg, C, 1, d_ix,
                           ix_bytes, d_sc, bsc_bytes, NULL);
  if (st) printf("op_backward: %s\n", bevpool_last_error());
  CHECK(st == BEVPOOL_OK);
  CHECK(hipDeviceSynchronize() == hipSuccess);
  uint32_t *xg = malloc(N * C * 4), *xg_exp = malloc(N * C * 4);
  CHECK(hipMemcpy(xg, d_xg, N * C * 4, hipMemcpyDeviceToHost) == hipSuccess);
  oracle_backward((const uint32_t *)grad_rows, C, rank, N, xg_exp);
  CHECK(memcmp(xg, xg_exp, N * C * 4) == 0);

  printf("ok: %lld points, %lld invalid (first %lld), forward and backward bit-exact\n",
         (long long)N, (long long)nbad_exp, (long long)first_bad);
  return 0;
}
"""


def test_c_caller_op_level_end_to_end(tmp_path):
    cc = shutil.which('gcc') or shutil.which('cc')
    if cc is None:
        pytest.skip('no C compiler')
    lib = ROOT / 'bevfusion-triton_amd' / 'libbevpool_amd.so'
    oracle = ROOT / 'oracle' / '_build' / 'liboracle_seq.so'
    assert lib.exists() and oracle.exists(), 'build the library and the oracle first'
    src = tmp_path / 'op_level.c'
    src.write_text(PROGRAM)
    exe = tmp_path / 'op_level'
    rocm = '/opt/rocm'
    subprocess.run([cc, '-std=c99', '-O1', '-Wall', '-Werror', '-D__HIP_PLATFORM_AMD__',
                    f'-I{rocm}/include', f'-I{ROOT / "include"}', str(src), '-o', str(exe),
                    str(lib), str(oracle), f'-L{rocm}/lib', '-lamdhip64',
                    f'-Wl,-rpath,{lib.parent}:{oracle.parent}:{rocm}/lib'], check=True)
    print('running the C caller', flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.startswith('ok:')
