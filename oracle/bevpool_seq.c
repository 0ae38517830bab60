/*
 * bevpool_seq.c -- strictly sequential plain-C restatement of the LSS
 * bev_pool path.  TEST INFRASTRUCTURE ONLY: the checker for the HIP library
 * and an independent cross-check of the torch restatement in
 * oracle/torch_fallback.py.  Built with gcc -O2 -ffp-contract=off (no fast
 * math), so every float operation is one IEEE-754 fp32 operation.
 *
 * Reference files restated (paths relative to the reference repository):
 *   models/vtransforms/base.py:139-158       quantise, batch index, kept mask
 *   ops/bev_pool/src/bev_pool_triton.py:34-48 ranks, zeros + index_add_
 *   ops/bev_pool/bev_pool_legacy.py:56-61     interval starts / lengths
 *   ops/bev_pool/src/bev_pool_triton.py:102-150 backward gather
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* torch's CPU float -> int64 conversion (x86 cvttss2si semantics): truncate
 * toward zero; NaN and values outside [-2^63, 2^63) give INT64_MIN. */
static int64_t torch_long(float q) {
  if (isnan(q) || q >= 9223372036854775808.0f || q < -9223372036854775808.0f) return INT64_MIN;
  return (int64_t)q;
}

/* base.py:139-158 + bev_pool_triton.py:34-39.  rank[p] = ((b*nz + z)*nx0 + x)*nx1 + y
 * for kept points, -1 otherwise.  q = (g - offset) / dx with
 * offset = fp32(bx) - fp32(dx)/2 computed by the caller in fp32. */
void oracle_quantize_geom(const float *geom, int64_t n, int64_t points_per_batch,
                          const float offset[3], const float dx[3], const int64_t nx[3],
                          int64_t *rank) {
  for (int64_t p = 0; p < n; ++p) {
    int64_t q[3];
    for (int k = 0; k < 3; ++k) {
      float diff = geom[p * 3 + k] - offset[k];
      float qf = diff / dx[k];
      q[k] = torch_long(qf);
    }
    int kept = 1;
    for (int k = 0; k < 3; ++k) kept &= (q[k] >= 0) && (q[k] < nx[k]);
    if (kept) {
      int64_t b = p / points_per_batch;
      rank[p] = ((b * nx[2] + q[2]) * nx[0] + q[0]) * nx[1] + q[1];
    } else {
      rank[p] = -1;
    }
  }
}

/* bev_pool_triton.py:34-39 in wrapping int64 arithmetic; ranks outside
 * [0, B*D*H*W) (which make index_add_ raise) become -1 and are counted. */
int64_t oracle_coord_ranks(const int64_t *coords, int64_t n, int64_t B, int64_t D, int64_t H,
                           int64_t W, int64_t *rank) {
  int64_t bad = 0;
  const uint64_t cells = (uint64_t)(B * D * H * W);
  for (int64_t p = 0; p < n; ++p) {
    uint64_t x = (uint64_t)coords[p * 4 + 0], y = (uint64_t)coords[p * 4 + 1];
    uint64_t z = (uint64_t)coords[p * 4 + 2], b = (uint64_t)coords[p * 4 + 3];
    uint64_t r = ((b * (uint64_t)D + z) * (uint64_t)H + x) * (uint64_t)W + y;
    if (r < cells) {
      rank[p] = (int64_t)r;
    } else {
      rank[p] = -1;
      ++bad;
    }
  }
  return bad;
}

/* Stable counting sort of the kept points by rank: perm lists point indices
 * ordered by (rank, index).  Returns the number of kept points. */
int64_t oracle_stable_sort(const int64_t *rank, int64_t n, int64_t n_cells, int64_t *perm,
                           int64_t *sorted_rank) {
  int64_t *count = (int64_t *)calloc((size_t)n_cells + 1, sizeof(int64_t));
  if (!count) return -1;
  int64_t kept = 0;
  for (int64_t p = 0; p < n; ++p)
    if (rank[p] >= 0) {
      count[rank[p] + 1]++;
      kept++;
    }
  for (int64_t c = 0; c < n_cells; ++c) count[c + 1] += count[c];
  for (int64_t p = 0; p < n; ++p) {
    if (rank[p] < 0) continue;
    int64_t pos = count[rank[p]]++;
    perm[pos] = p;
    sorted_rank[pos] = rank[p];
  }
  free(count);
  return kept;
}

/* bev_pool_legacy.py:56-61: starts where r[i] != r[i-1], lengths by
 * difference, last = n - start.  Returns the number of intervals. */
int64_t oracle_intervals(const int64_t *sorted_rank, int64_t n, int32_t *starts,
                         int32_t *lengths) {
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i)
    if (i == 0 || sorted_rank[i] != sorted_rank[i - 1]) starts[m++] = (int32_t)i;
  for (int64_t j = 0; j + 1 < m; ++j) lengths[j] = starts[j + 1] - starts[j];
  if (m > 0) lengths[m - 1] = (int32_t)(n - starts[m - 1]);
  return m;
}

/* bev_pool_triton.py:42-48: out = zeros; out[rank[p]] += x[p] for p in
 * increasing order.  out is cell-major (n_cells x C); every sum starts at
 * +0.0f and each step is one fp32 addition. */
void oracle_forward(const float *x, int64_t ld, int64_t C, const int64_t *rank, int64_t n,
                    int64_t n_cells, float *out) {
  for (int64_t i = 0; i < n_cells * C; ++i) out[i] = 0.0f;
  for (int64_t p = 0; p < n; ++p) {
    int64_t r = rank[p];
    if (r < 0) continue;
    float *o = out + r * C;
    const float *v = x + p * ld;
    for (int64_t c = 0; c < C; ++c) o[c] = o[c] + v[c];
  }
}

/* Backward gather: x_grad[p] = grad_rows[rank[p]] (cell-major rows), zero row
 * for dropped points.  Raw 32-bit words, so it is a bit copy. */
void oracle_backward(const uint32_t *grad_rows, int64_t C, const int64_t *rank, int64_t n,
                     uint32_t *x_grad) {
  for (int64_t p = 0; p < n; ++p) {
    if (rank[p] < 0) {
      memset(x_grad + p * C, 0, (size_t)C * sizeof(uint32_t));
    } else {
      memcpy(x_grad + p * C, grad_rows + rank[p] * C, (size_t)C * sizeof(uint32_t));
    }
  }
}
