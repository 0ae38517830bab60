/*
 * bevpool.h -- C ABI of the MI355X (gfx950) LSS camera-to-BEV pooling library
 * (libbevpool_amd.so).
 *
 * This is the drop-in native boundary for the LSS `bev_pool` hot path of
 * ziyangyeh/bevfusion-triton.  Every entry point is plain C: raw device
 * pointers, sizes and a `hipStream_t` passed as `void *`.  No torch types
 * cross this boundary.
 *
 * Conventions shared by every call:
 *   - all work is stream-ordered on the caller's stream; nothing synchronises
 *     the device and nothing allocates device memory (the caller passes every
 *     buffer, including the scratch workspace);
 *   - the return value is a status code (BEVPOOL_OK == 0, negative on error)
 *     and bevpool_last_error() returns a thread-local message for the last
 *     failing call on the calling thread;
 *   - device-side counters live in a caller-owned `meta` array of
 *     BEVPOOL_META_LEN int32 (see BEVPOOL_META_*);
 *   - ranks are the reference's flattened (b, z, x, y) cell index
 *     ((b*D + z)*H + x)*W + y, stored as int32 (-1 marks a dropped point);
 *     the library rejects grids with B*D*H*W >= 2^31;
 *   - sorted keys are uint64 (rank << 32) | point_index, i.e. the stable
 *     argsort of the ranks expressed as a sort of unique 64-bit keys.
 *
 * The reference interfaces each call replaces are cited per declaration
 * (paths relative to the reference repository root).
 */
#ifndef BEVPOOL_AMD_H_
#define BEVPOOL_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BEVPOOL_ABI_VERSION 4

/* status codes */
#define BEVPOOL_OK 0
#define BEVPOOL_EINVAL -1  /* bad argument (shape, size, dtype, alignment)   */
#define BEVPOOL_EHIP -2    /* a HIP runtime call or kernel launch failed       */
#define BEVPOOL_ESPACE -3  /* workspace / scratch buffer too small            */

/* element types of feature / gradient tensors */
#define BEVPOOL_F32 0
#define BEVPOOL_F16 1
#define BEVPOOL_BF16 2

/* layout of the caller-owned int32 meta array (device memory) */
#define BEVPOOL_META_N_KEPT 0      /* number of kept points (sorted keys)     */
#define BEVPOOL_META_N_INTERVALS 1 /* number of occupied cells (intervals)    */
#define BEVPOOL_META_N_BAD 2       /* op-level: coords whose rank is invalid  */
#define BEVPOOL_META_FIRST_BAD 3   /* op-level: smallest invalid point index  */
#define BEVPOOL_META_LEN 8
/* a report destination: the BEVPOOL_META_LEN counters, then a done flag */
#define BEVPOOL_REPORT_LEN (BEVPOOL_META_LEN + 1)

/* ABI version of the loaded library (BEVPOOL_ABI_VERSION). */
int bevpool_abi_version(void);

/* Message describing the last failing call on this thread ("" if none). */
const char *bevpool_last_error(void);

/*
 * Bytes of scratch workspace the index stage (quantise/ranks + sort +
 * intervals) needs for n_points points and n_cells = B*D*H*W cells.
 * One workspace serves one index stage at a time on one stream.
 */
size_t bevpool_index_workspace_bytes(int64_t n_points, int64_t n_cells);

/*
 * Voxel quantisation + kept mask of LSS geometry, fused with the first pass
 * of the rank sort (its digit histogram).
 *
 * Replaces models/vtransforms/base.py:139-158 (quantise
 * ((g - (bx - dx/2)) / dx).long(), batch-index concat, in-bounds kept mask)
 * together with the rank formula of ops/bev_pool/src/bev_pool_triton.py:34-39.
 *
 *   geom        fp32 [n_points, 3] (x, y, z) in batch-major point order,
 *               row stride geom_row_stride floats, component stride 1
 *   points_per_batch  N*D*fH*fW (point p belongs to batch p / points_per_batch)
 *   offset[3]   fp32(bx) - fp32(dx)/2, computed in fp32 by the caller
 *   dx[3]       fp32 voxel size
 *   nx[3]       grid size (X -> H, Y -> W, Z -> D of the output)
 *   rank        out: int32 [n_points], -1 for dropped points
 *   meta        int32 [BEVPOOL_META_LEN], zeroed by this call
 * Must be followed by bevpool_sort on the same workspace and stream.
 */
int bevpool_quantize_geom(const float *geom, int64_t n_points, int64_t geom_row_stride,
                          int64_t points_per_batch, int32_t n_batch, const float offset[3],
                          const float dx[3], const int32_t nx[3], int32_t *rank, int32_t *meta,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * As bevpool_quantize_geom, with the geometry computed per point from the
 * camera matrices instead of read from a geometry tensor.  Replaces
 * models/vtransforms/base.py:82-126 (get_geometry) followed by :139-158.
 * fp32 arithmetic with every operation rounded separately, 3x3 products
 * summed left to right; combine = rots inv(intrins) (the reference's
 * linalg.solve, base.py:107-110) is formed in double and rounded once.
 * torch's batched matmul rounds its own way, so a point lying within
 * rounding distance of a voxel face can land in the neighbouring cell.
 *
 *   frustum      fp32 (D, fH, fW, 3) contiguous (create_frustum, base.py:67-80)
 *   rots, intrins, post_rots   fp32 [n_batch * n_cams_per_batch][3][3]
 *   trans, post_trans          fp32 [n_batch * n_cams_per_batch][3]
 *                (camera b*N + n; camera2lidar rotation / translation,
 *                intrinsics, image-augmentation rotation / translation)
 *   extra_rots   fp32 [n_batch][3][3] or NULL (identity)   base.py:114-118
 *   extra_trans  fp32 [n_batch][3] or NULL (zero)          base.py:119-123
 * all row-major and contiguous.  Point order and everything else as
 * bevpool_quantize_geom (n_points = n_batch * n_cams_per_batch * D*fH*fW).
 */
int bevpool_quantize_cameras(const float *frustum, int32_t D, int32_t fH, int32_t fW,
                             const float *rots, const float *trans, const float *intrins,
                             const float *post_rots, const float *post_trans,
                             const float *extra_rots, const float *extra_trans,
                             int32_t n_cams_per_batch, int32_t n_batch, const float offset[3],
                             const float dx[3], const int32_t nx[3], int32_t *rank,
                             int32_t *meta, void *workspace, size_t workspace_bytes,
                             void *stream);

/*
 * Op-level ranks from integer coords (columns x, y, z, b), fused with the
 * first sort pass histogram.
 *
 * Replaces ops/bev_pool/src/bev_pool_triton.py:34-39 (_flatten_ranks,
 * rank = ((b*D + z)*H + x)*W + y in int64 arithmetic).  A rank outside
 * [0, B*D*H*W) is what makes the reference CPU fallback's index_add_
 * (bev_pool_triton.py:47) raise; here such a point is excluded (rank -1),
 * counted in meta[BEVPOOL_META_N_BAD] and its index min-reduced into
 * meta[BEVPOOL_META_FIRST_BAD] so the host can raise the same error.
 *
 *   coords       int32 or int64 (coord_bytes 4 or 8) [n_points, 4],
 *                row stride coords_row_stride elements, column stride 1
 */
int bevpool_coord_ranks(const void *coords, int32_t coord_bytes, int64_t n_points,
                        int64_t coords_row_stride, int32_t B, int32_t D, int32_t H, int32_t W,
                        int32_t *rank, int32_t *meta, void *workspace, size_t workspace_bytes,
                        void *stream);

/*
 * Stream compaction of kept points + stable radix sort of their ranks
 * + dense per-cell point ranges.  Ranks of 11..20 bits take one global pass
 * by the high digit and, for the low digit, one block per group of equal
 * high digit (two above 8192 keys; 8192-key slices for groups of 1024
 * cells), which also write the group's cell ranges; other rank widths take
 * LSD passes of at most 10 bits.  All give the same keys.  The
 * index stage's histograms must come from the quantise / coord-ranks call
 * made with the same n_cells.
 *
 * Replaces the kept-point compaction of models/vtransforms/base.py:157-158
 * and the sort of ops/bev_pool/bev_pool_legacy.py:102-104, with the legacy
 * (x,y,z,b) ranks replaced by the (b,z,x,y) ranks above and the sort made
 * stable, so the permutation equals a stable argsort of the ranks.
 *
 *   rank         int32 [n_points] from bevpool_quantize_geom / bevpool_coord_ranks
 *   keys         out: uint64 [n_points]; the first meta[N_KEPT] entries are
 *                the sorted (rank << 32 | point_index) keys
 *   cell_start,
 *   cell_end     out: int32 [n_cells]; the sorted positions [start, end) of
 *                each cell's points (start == end == 0 for an empty cell)
 *   meta         meta[BEVPOOL_META_N_KEPT] is written
 */
int bevpool_sort(const int32_t *rank, int64_t n_points, int64_t n_cells, uint64_t *keys,
                 int32_t *cell_start, int32_t *cell_end, int32_t *meta, void *workspace,
                 size_t workspace_bytes, void *stream);

/*
 * Interval boundaries of the sorted ranks, compacted in rank order.
 *
 * Replaces ops/bev_pool/bev_pool_legacy.py:56-61 (boundary flags
 * r[i] != r[i-1], interval_starts = where(flags), lengths by difference with
 * the last one n - start) without the host synchronisation of torch.where.
 *
 *   starts, lengths, cells   out: int32 [n_points] (capacity); the first
 *                meta[BEVPOOL_META_N_INTERVALS] entries are written
 */
int bevpool_intervals(const uint64_t *keys, int64_t n_points, const int32_t *cell_end,
                      int32_t *starts, int32_t *lengths, int32_t *cells, int32_t *meta,
                      void *workspace, size_t workspace_bytes, void *stream);

/*
 * Copies the BEVPOOL_META_LEN counters at `meta` (device memory) to
 * dst[0 .. BEVPOOL_META_LEN) with one single-block kernel on `stream`, then
 * sets dst[BEVPOOL_META_LEN] = 1 once they are written, so that a caller
 * that cleared that flag can poll it and read the counters without a host
 * synchronisation, an event, a copy engine or a second stream.  `dst`
 * (BEVPOOL_REPORT_LEN int32) is pinned host memory (hipHostMalloc; written
 * through its device address with system-scope stores) or device memory of
 * the current device; anything else is refused with BEVPOOL_EINVAL.
 *
 * No reference counterpart: the reference raises out-of-range ranks from its
 * CPU fallback's index_add_ (ops/bev_pool/src/bev_pool_triton.py:47); this
 * lets the op-level drop-in report them asynchronously.
 */
int bevpool_meta_report(const int32_t *meta, int32_t *dst, void *stream);

/* Bytes of fp32 scratch bevpool_forward needs: n_cells * C * 4. */
size_t bevpool_forward_scratch_bytes(int64_t n_cells, int32_t C);

/*
 * Forward pooling: out[cell, c] = sum over the cell's points, in increasing
 * point order, of feats[p, c], accumulated in fp32 from +0.0, written
 * channel-first with empty cells set to zero.
 *
 * Replaces ops/bev_pool/src/bev_pool_triton.py:42-48 (index_add_ fallback),
 * :155-186 (forward of the autograd Function), the permute of :227, and the
 * Z-collapse of models/vtransforms/base.py:163 (through the output strides);
 * legacy equivalent ops/bev_pool/csrc/bev_pool_cuda.cu:20-42.
 *
 *   feats        dtype [n_points, C], row stride feats_row_stride elements,
 *                channel stride 1 (rows are indexed by the keys' point index)
 *   out          dtype; element (b, c, z, xy) at
 *                b*out_stride_b + c*out_stride_c + z*out_stride_z + xy
 *                with xy = x*W + y in [0, n_xy)
 *   scratch      >= bevpool_forward_scratch_bytes(n_cells, C) bytes
 */
int bevpool_forward(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                    int64_t n_points, const uint64_t *keys, const int32_t *cell_start,
                    const int32_t *cell_end, const int32_t *meta, int32_t n_batch, int32_t n_z,
                    int64_t n_xy, int64_t out_stride_b, int64_t out_stride_c,
                    int64_t out_stride_z, void *out, void *scratch, size_t scratch_bytes,
                    void *stream);

/* Bytes of scratch bevpool_backward needs: n_cells * C * element size. */
size_t bevpool_backward_scratch_bytes(int64_t n_cells, int32_t C, int32_t dtype);

/*
 * Backward pooling: x_grad[p, :] = grad[b, :, z, xy] of p's cell for a kept
 * point and 0 for a dropped one (rank -1).  A pure copy of the gradient's
 * bits.
 *
 * Replaces ops/bev_pool/src/bev_pool_triton.py:102-150 and :189-216 (the
 * gather backward, including the out_grad.contiguous() transpose of :192)
 * and the zero-filled gradient of the kept-mask gather of
 * models/vtransforms/base.py:157; legacy equivalent
 * ops/bev_pool/csrc/bev_pool_cuda.cu:61-84.
 *
 *   grad         dtype; element (b, c, z, xy) at
 *                b*grad_stride_b + c*grad_stride_c + z*grad_stride_z + xy
 *   x_grad       out: dtype [n_points, C], row stride x_grad_row_stride
 *   zero_dropped 1: rows of dropped points (rank -1) are written as zero (the
 *                zero-filled gradient of base.py:157's kept-mask gather);
 *                0: those rows are left untouched
 *   scratch      >= bevpool_backward_scratch_bytes(n_cells, C, dtype) bytes
 */
int bevpool_backward(const void *grad, int32_t dtype, int64_t grad_stride_b,
                     int64_t grad_stride_c, int64_t grad_stride_z, int32_t C,
                     const int32_t *rank, int64_t n_points, const int32_t *cell_start,
                     const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                     void *x_grad, int64_t x_grad_row_stride, int32_t zero_dropped,
                     void *scratch, size_t scratch_bytes, void *stream);

/*
 * Planar (channel-first) camera features.  The reference's features are the
 * view rearrange(x, '(b n) c d h w -> b n d h w c') of channel-first storage
 * (models/vtransforms/depth_lss.py:94); base.py:136 then copies them into
 * (N_all, C) rows with x.reshape.  A planar tensor (BN, C, S), S = D*fH*fW,
 * has element (bn, c, s) at bn*stride_bn + c*stride_c + s; point p = bn*S + s.
 */

/*
 * Planar (BN, C, S) fp32 -> rows [BN*S, C] fp32 (the copy of base.py:136,
 * as one transposing kernel).  Any strides; the fast form needs C, S and both
 * strides multiples of 4 and 16-byte aligned pointers.
 */
int bevpool_planar_rows(const float *src, int64_t stride_bn, int64_t stride_c, int32_t BN,
                        int32_t C, int64_t S, float *rows, void *stream);

/*
 * Backward of the pooling straight into a planar fp32 gradient:
 * x_grad[bn, c, s] = grad at the cell of point bn*S + s (0 for dropped
 * points), i.e. the gradient autograd hands the channel-first producer
 * through the rearrange view (bev_pool_triton.py:192 gather, then
 * depth_lss.py:94 and base.py:136 backwards).  Arguments as bevpool_backward
 * (fp32 grad) plus S and the x_grad strides; n_points = BN*S.
 */
int bevpool_backward_planar(const float *grad, int64_t grad_stride_b, int64_t grad_stride_c,
                            int64_t grad_stride_z, int32_t C, const int32_t *rank,
                            int64_t n_points, const int32_t *cell_start,
                            const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                            int64_t S, float *x_grad, int64_t x_stride_bn, int64_t x_stride_c,
                            void *scratch, size_t scratch_bytes, void *stream);

/*
 * Depth-weighted (fused depth x context) pooling.  The reference builds the
 * camera features as the outer product x[bn, c, d, h, w] =
 * depth[bn, d, h, w] * context[bn, c, h, w] (models/vtransforms/depth_lss.py:
 * 91-94, 638 MB at the det shape) and pools x; these calls pool
 * depth[p] * context[pix(p), :] without materialising x.  Point p of the
 * (B, N, D, fH, fW) frustum is p = (bn*D + d)*HW + hw with bn = b*N + n and
 * HW = fH*fW; its context row is pix(p) = bn*HW + hw.  Ranks, keys and cell
 * ranges come from bevpool_quantize_geom + bevpool_sort as for x.  Forward sums
 * use the same products and order as the reference (fp32 product rounded,
 * then added in point order), so they are bit-identical to pooling x.
 */

/*
 * Context (BN, C, HW) fp32, element (bn, c, hw) at bn*stride_bn + c*stride_c
 * + hw, to channel-last rows [BN*HW, C] (the layout the pooled rows are read
 * in).  Replaces the context operand of depth_lss.py:92 (x[:, D:D+C], a
 * channel-first slice of the depthnet output).  Same as bevpool_planar_rows
 * with S = HW.
 */
int bevpool_context_rows(const float *context, int64_t stride_bn, int64_t stride_c, int32_t BN,
                         int32_t C, int64_t HW, float *rows, void *stream);

/*
 * Forward of the depth-weighted pooling into the channel-first output, as
 * bevpool_forward for x = depth (x) context.  Replaces depth_lss.py:91-94 followed
 * by models/vtransforms/base.py:131-165 (bev_pool of the outer product).
 *
 *   depth         fp32 [n_points] = (BN, D, HW) contiguous
 *   context_rows  fp32 [BN*HW, C] from bevpool_context_rows, 16-byte aligned;
 *                 C a multiple of 4
 *   n_points      BN * D * HW
 *   scratch       >= bevpool_forward_scratch_bytes(n_cells, C) bytes
 */
int bevpool_forward_depth(const float *depth, const float *context_rows, int32_t C,
                          int64_t n_points, int32_t D, int64_t HW, const uint64_t *keys,
                          const int32_t *cell_start, const int32_t *cell_end,
                          const int32_t *meta, int32_t n_batch, int32_t n_z, int64_t n_xy,
                          int64_t out_stride_b, int64_t out_stride_c, int64_t out_stride_z,
                          float *out, void *scratch, size_t scratch_bytes, void *stream);

/*
 * Backward of the depth-weighted pooling: the reference's autograd through
 * the outer product (depth_lss.py:93) and the pooling, without the [n_points,
 * C] feature gradient:
 *   grad_depth[p]           = sum_c g[cell(p), c] * context[pix(p), c]
 *                             (0 for a dropped point)
 *   grad_context[bn, c, hw] = sum_d g[cell(p_d), c] * depth[p_d]
 *                             over the pixel's D points p_d (kept ones)
 * Sums are fp32 in a fixed order (over channels: 16-lane partial sums then a
 * fixed reduction tree; over depth bins: four interleaved sequential chains
 * added in order), so results are deterministic and agree with the reference
 * within fp32 rounding (the reference sums in torch's reduction order).
 *
 *   grad          fp32 BEV gradient; element (b, c, z, xy) at
 *                 b*grad_stride_b + c*grad_stride_c + z*grad_stride_z + xy
 *   C             <= 256, and 2*D + C <= 1024
 *   grad_depth    out: fp32 [n_points]
 *   grad_context  out: fp32, element (bn, c, hw) at
 *                 bn*gctx_stride_bn + c*gctx_stride_c + hw
 *   scratch       >= bevpool_backward_scratch_bytes(n_cells, C, BEVPOOL_F32)
 */
int bevpool_backward_depth(const float *grad, int64_t grad_stride_b, int64_t grad_stride_c,
                           int64_t grad_stride_z, int32_t C, const int32_t *rank,
                           int64_t n_points, int32_t D, int64_t HW, const float *depth,
                           const float *context_rows, const int32_t *cell_start,
                           const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                           float *grad_depth, float *grad_context, int64_t gctx_stride_bn,
                           int64_t gctx_stride_c, void *scratch, size_t scratch_bytes,
                           void *stream);

/*
 * One-call op level: ops/bev_pool/src/bev_pool_triton.py:219-227
 * (bev_pool(feats, coords, B, D, H, W)) as bevpool_coord_ranks ->
 * bevpool_sort -> bevpool_forward.  Two caller-owned buffers:
 *   index    >= bevpool_op_index_bytes(n_points, B*D*H*W): what the backward
 *            needs (meta counters, ranks, sorted keys, cell ranges); it
 *            starts with the BEVPOOL_META_LEN int32 meta counters
 *            (meta[BEVPOOL_META_N_BAD] = points whose rank falls outside
 *            [0, B*D*H*W): they are excluded, where the reference CPU
 *            fallback raises).  Keep it from the forward to its backward.
 *   scratch  >= bevpool_op_scratch_bytes(n_points, B*D*H*W, C): the
 *            index-stage workspace and the cell rows, needed only during
 *            the call (free or reuse it afterwards).
 * One index buffer serves one forward/backward pair at a time.
 *
 *   feats        dtype [n_points, C], row stride feats_row_stride, channel stride 1
 *   coords       int32 / int64 (coord_bytes 4 / 8) [n_points, 4] (x, y, z, b)
 *   out          dtype, contiguous (B, C, D, H, W)
 *   report       NULL, or BEVPOOL_REPORT_LEN int32 of pinned host memory
 *                (or device memory) that receives a copy of the meta
 *                counters and then the done flag report[BEVPOOL_META_LEN] = 1,
 *                written by the call's last kernel (as bevpool_meta_report,
 *                folded in: no launch of its own): a host that cleared the
 *                flag polls it and then reads the count of excluded points
 * bevpool_op_workspace_bytes is the sum of the two (the allocation-free
 * forward below keeps both in one static array).
 */
size_t bevpool_op_index_bytes(int64_t n_points, int64_t n_cells);
size_t bevpool_op_scratch_bytes(int64_t n_points, int64_t n_cells, int32_t C);
size_t bevpool_op_workspace_bytes(int64_t n_points, int64_t n_cells, int32_t C);

int bevpool_op_forward(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                       const void *coords, int32_t coord_bytes, int64_t coords_row_stride,
                       int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W, void *out,
                       void *index, size_t index_bytes, void *scratch, size_t scratch_bytes,
                       int32_t *report, void *stream);

/*
 * bevpool_op_forward without a workspace argument, for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  The workspace lives in a
 * static device array of BEVPOOL_NOALLOC_MAX_BYTES bytes inside the
 * library's code object, one copy per GPU: every GPU on which any entry
 * point of this library has run holds its 96 MiB until the process ends,
 * whether or not this entry point is used.  A call whose workspace
 * (bevpool_op_workspace_bytes) exceeds it returns BEVPOOL_ESPACE.
 *
 * The first call on a device resolves the array's device address
 * (hipGetSymbolAddress, cached per device); if no kernel of the library has
 * run on that device yet, that lookup loads the code object there, which
 * reserves the array.  Make one call (or any other library call) on each
 * device before relying on the no-allocation property.  After that a call
 * allocates nothing: no hipMalloc, no events even with timing enabled.
 * Graph capture of this entry point is not tested and not claimed.
 *
 * Every call on one GPU uses that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (concurrent streams or threads)
 * race, and the index left behind is not kept for a backward.  Points with
 * invalid coords are excluded, as in bevpool_op_forward; the count is not
 * reported.
 */
#define BEVPOOL_NOALLOC_MAX_BYTES ((size_t)96 << 20)

int bevpool_op_forward_noalloc(const void *feats, int32_t dtype, int64_t feats_row_stride,
                               int32_t C, const void *coords, int32_t coord_bytes,
                               int64_t coords_row_stride, int64_t n_points, int32_t B, int32_t D,
                               int32_t H, int32_t W, void *out, void *stream);

/*
 * Backward of bevpool_op_forward (bev_pool_triton.py:189-216): x_grad[p, :]
 * = grad at p's cell, on the index the forward left in `index`.  grad
 * element (b, c, z, xy) at b*grad_stride_b + c*grad_stride_c +
 * z*grad_stride_z + xy (xy = x*W + y contiguous); zero_dropped as
 * bevpool_backward.  scratch >= bevpool_backward_scratch_bytes(B*D*H*W, C,
 * dtype) (bevpool_op_scratch_bytes is always enough).
 */
int bevpool_op_backward(const void *grad, int32_t dtype, int64_t grad_stride_b,
                        int64_t grad_stride_c, int64_t grad_stride_z, int32_t C,
                        int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W,
                        void *x_grad, int64_t x_grad_row_stride, int32_t zero_dropped,
                        const void *index, size_t index_bytes, void *scratch,
                        size_t scratch_bytes, void *stream);

/*
 * Legacy native interface: the reference's pybind extension functions
 * bev_pool_forward / bev_pool_backward (ops/bev_pool/csrc/bev_pool_cpu.cpp:22-94,
 * kernels ops/bev_pool/csrc/bev_pool_cuda.cu:20-98), called by
 * ops/bev_pool/bev_pool_legacy.py:64-73, 85-94.  Intervals are caller-given
 * runs of rows: interval j covers rows [interval_starts[j],
 * interval_starts[j] + interval_lengths[j]) of x, and its cell is
 * geom_feats[interval_starts[j]] = (x, y, z, b).
 *
 * Forward: out (b, d, h, w, C) fp32 contiguous is zero-filled, then
 * out[cell, :] = the sum of the interval's rows, fp32 from +0.0 in row order
 * (the reference kernel's psum loop).  Backward: x_grad (n, C) fp32 is
 * zero-filled, then every row of an interval gets out_grad[cell, :]
 * (out_grad (b, d, h, w, C) contiguous).  Two intervals of one cell race as
 * in the reference.
 *
 * Differences from the reference: an interval whose rows or cell fall outside
 * the arrays is skipped and counted in meta[BEVPOOL_META_N_BAD] (meta may be
 * NULL) instead of reading/writing out of bounds; the interval count is
 * n_intervals, or, when n_intervals_dev is not NULL, min(n_intervals,
 * *n_intervals_dev) read on the device (capacity + device count, so a caller
 * chaining bevpool_runs needs no host synchronisation).  The caller passes
 * the arrays in the reference's argument order (lengths before starts in the
 * Python wrapper, starts before lengths in the kernel; here starts first).
 *   x, geom_feats, out_grad: contiguous; interval arrays int32.
 */
int bevpool_legacy_forward(const float *x, int64_t n, int32_t C, const int32_t *geom_feats,
                           const int32_t *interval_starts, const int32_t *interval_lengths,
                           int64_t n_intervals, const int32_t *n_intervals_dev, int32_t b,
                           int32_t d, int32_t h, int32_t w, float *out, int32_t *meta,
                           void *stream);

int bevpool_legacy_backward(const float *out_grad, int64_t n, int32_t C,
                            const int32_t *geom_feats, const int32_t *interval_starts,
                            const int32_t *interval_lengths, int64_t n_intervals,
                            const int32_t *n_intervals_dev, int32_t b, int32_t d, int32_t h,
                            int32_t w, float *x_grad, int32_t *meta, void *stream);

/*
 * Runs of equal values in a rank array (int32 or int64, rank_bytes 4 / 8):
 * ops/bev_pool/bev_pool_legacy.py:56-61 (start flags rank[i] != rank[i-1],
 * interval_starts = where(flags), lengths by difference, the last n - start)
 * without torch.where's host synchronisation.
 *   starts, lengths   out: int32 [n] (capacity); the first
 *                     meta[BEVPOOL_META_N_INTERVALS] entries are written
 *   meta              int32 [BEVPOOL_META_LEN], reset by this call
 *   workspace         >= bevpool_runs_workspace_bytes(n)
 */
size_t bevpool_runs_workspace_bytes(int64_t n);

int bevpool_runs(const void *ranks, int32_t rank_bytes, int64_t n, int32_t *starts,
                 int32_t *lengths, int32_t *meta, void *workspace, size_t workspace_bytes,
                 void *stream);

/*
 * Optional per-kernel timing.  When enabled, every kernel launch is bracketed
 * by HIP events on the launch stream; bevpool_timing_read() synchronises
 * those events and returns, per kernel name, the summed milliseconds and
 * launch count since the last reset.  Used by the benchmark only.
 */
int bevpool_timing_enable(int enable);
int bevpool_timing_reset(void);
/* Writes up to max_entries entries; returns the number of entries or < 0. */
int bevpool_timing_read(char *names, int name_stride, double *total_ms, int64_t *launches,
                        int max_entries);

#ifdef __cplusplus
}
#endif

#endif /* BEVPOOL_AMD_H_ */
