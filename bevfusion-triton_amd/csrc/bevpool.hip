// bevpool.hip -- gfx950 (MI355X, CDNA4) kernels and C ABI for the LSS
// camera-to-BEV pooling path of ziyangyeh/bevfusion-triton.
//
// Pipeline (all stream-ordered on the caller's stream, no host sync):
//
//   index stage
//     quantize_geom_kernel / coord_ranks_kernel  point -> int32 rank (-1 dropped)
//       / quantize_frustum_kernel                + radix pass-0 block histogram
//                                                (frustum: geometry computed from
//                                                the camera matrices in-kernel)
//     radix_scan_kernel                          per-digit exclusive scan of the
//                                                block histograms (+ zero cell ranges)
//     radix_scatter_kernel<from_rank>            stable wave-ballot ranked scatter;
//                                                pass 0 also compacts kept points
//     radix_hist_kernel                          block histograms of passes >= 1
//     cell_ranges_kernel                         dense [start, end) per cell
//     bucket_sort_kernel                         ranks of 11..20 bits: after one
//                                                global pass by the high digit,
//                                                one block per group sorts the low
//                                                digit and writes its cell ranges
//                                                (replaces the passes >= 1 and
//                                                cell_ranges_kernel)
//     count_starts_kernel + scan_counts_kernel
//       + interval_write_kernel                  compacted interval starts/lengths
//   forward
//     accum_pipe_kernel<T,..>   ranges of 256 sorted points (snapped to cell
//                               boundaries); loader waves gather 16-byte row
//                               pieces through a register ring into LDS, one
//                               summing wave keeps a sequential fp32
//                               accumulator per channel
//     accum_rows_kernel<T>      the same for rows that are not 16-byte pieces
//     rows_to_bev_kernel<T>     cell-major rows -> channel-first tile via LDS
//                               transpose; empty cells written as zero
//   backward
//     bev_to_rows_kernel<T>     channel-first grad tile -> cell-major rows
//                               (occupied cells only) via LDS transpose
//     gather_rows_kernel<V>     leading blocks read the ranks (per XCD) and the
//                               occupied rows once so the rest find them
//                               cached; then a point-order streaming copy of
//                               each point's cell row (zero rows for dropped
//                               points)
//   planar (channel-first) operands
//     planar_rows_kernel        (BN, C, S) -> channel-last rows (context, or
//                               channel-first camera features)
//     gather_planar_kernel      backward straight into a (BN, C, S) gradient
//   depth-weighted pooling (fused depth x context)
//     accum_pipe_kernel<..,true> forward sums of depth[p] * ctx[pix(p)]
//     depth_grad_kernel         grad_depth (dot products) and grad_context
//                               (depth-weighted sums along each ray)
//
// Numerics: the quantisation is IEEE fp32 subtraction followed by a correctly
// rounded fp32 division (built without fast-math, with
// -fhip-fp32-correctly-rounded-divide-sqrt and -ffp-contract=off), exactly as
// torch evaluates ((g - (bx - dx/2)) / dx) on the CPU.  Forward sums start at
// +0.0 and add the cell's points in increasing point index order, which is
// the order torch's CPU index_add_ uses, so fp32 results are bit-identical.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>
#include <type_traits>
#include <string>
#include <unordered_map>
#include <vector>

#include "bevpool.h"

namespace {

// ---------------------------------------------------------------------------
// constants
// ---------------------------------------------------------------------------
constexpr int kThreads = 256;              // threads per block, every kernel
constexpr int kWaves = kThreads / 64;      // wave64 waves per block
// Keys per thread of the sort's tile kernels (quantise / coord ranks, radix
// histogram and scatter): 8 (tiles of 2048 keys) up to kLargeSortPoints
// points, 16 (4096) above.  Larger tiles halve the [digit][tile] histogram
// that every pass writes, scans and reads: at 4 x 360 x 360 and 2 x 720 x 720
// the forward took 7 and 16 us less on MI355X; at 1 x 360 x 360, whose tiles
// fill the chip in one round, 3-5 us more.
constexpr int kItemsSmall = 8, kItemsLarge = 16;
constexpr int64_t kLargeSortPoints = int64_t(4) << 20;
inline int sort_items(int64_t n_points) {
  return n_points > kLargeSortPoints ? kItemsLarge : kItemsSmall;
}
constexpr int kMaxDigitBits = 10;
constexpr int kMaxRadix = 1 << kMaxDigitBits;
constexpr int kCellTile = 64;              // cells per transpose tile
constexpr int kTileChannels = 128;         // max channels per transpose pass

// 16- and 8-byte integer vectors.  HIP's uint4 struct blocks register
// promotion.  Float vectors are avoided on purpose: with packed fp32 ops
// disabled, hipcc 7.2 lowered a <2 x float> add of a 64-bit LDS load into two
// scalar adds that both read the low half.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#ifndef BEVPOOL_RANGE_POINTS
#define BEVPOOL_RANGE_POINTS 256
#endif
constexpr int64_t kRangePoints = BEVPOOL_RANGE_POINTS;  // nominal sorted points per forward range
#ifndef BEVPOOL_XCD_MAP
#define BEVPOOL_XCD_MAP 1
#endif
constexpr int kXcds = 8;                   // MI355X: 8 XCDs, one L2 each

// Workgroup i of a launch runs on XCD i % 8.  xcd_chunk maps it to chunk
// (i % 8) * (n / 8) + i / 8 of a grid of n workgroups (n a multiple of 8,
// padded by xcd_grid), so each XCD walks one contiguous eighth of the
// chunks and neighbouring chunks share that XCD's L2.  A bijection on [0, n).
__device__ __forceinline__ int64_t xcd_chunk(int64_t i, int64_t n) {
#if BEVPOOL_XCD_MAP
  return (i % kXcds) * (n / kXcds) + i / kXcds;
#else
  (void)n;
  return i;
#endif
}

inline unsigned xcd_grid(int64_t blocks) {
#if BEVPOOL_XCD_MAP
  return unsigned((blocks + kXcds - 1) / kXcds * kXcds);
#else
  return unsigned(blocks);
#endif
}

// Grid of a kernel that walks the tiles of the sort (at least one
// block: block 0 also resets meta).  Such kernels take tile
// xcd_chunk(blockIdx.x, gridDim.x), so the 32 tiles that share a 128-byte
// line of a digit's histogram row are written from one XCD's L2.
inline unsigned sort_grid(int64_t tiles) { return tiles > 0 ? xcd_grid(tiles) : 1u; }

// ---------------------------------------------------------------------------
// error reporting
// ---------------------------------------------------------------------------
thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// An AQL dispatch carries the grid size in work-items as 32 bits: a launch of
// more blocks * threads than that is rejected here instead of being
// truncated (which would leave part of the output unwritten).
int check_grid(int64_t blocks, int threads, const char *what) {
  if (blocks < 0 || blocks * int64_t(threads) > int64_t(UINT32_MAX))
    return fail(BEVPOOL_EINVAL, "%s: %lld blocks of %d threads exceed the 2^32 work-item grid",
                what, static_cast<long long>(blocks), threads);
  return BEVPOOL_OK;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BEVPOOL_EHIP, "%s: %s", what, hipGetErrorString(e));
  return BEVPOOL_OK;
}

// ---------------------------------------------------------------------------
// optional per-kernel timing (benchmark instrumentation)
// ---------------------------------------------------------------------------
struct TimingRecord {
  const char *name;
  hipEvent_t start, stop;
};
struct TimingTotal {
  double ms = 0.0;
  int64_t launches = 0;
};
std::mutex g_timing_mu;
bool g_timing_enabled = false;
// Set while an allocation-free entry point runs on this thread: its launches
// are never bracketed by timing events (creating one may allocate).
thread_local bool g_no_alloc_call = false;
std::vector<TimingRecord> g_timing_pending;
std::vector<hipEvent_t> g_event_pool;
std::vector<std::pair<std::string, TimingTotal>> g_timing_totals;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Brackets one kernel launch with events when timing is enabled.
struct LaunchTimer {
  const char *name;
  hipStream_t stream;
  hipEvent_t start = nullptr, stop = nullptr;
  LaunchTimer(const char *n, hipStream_t s) : name(n), stream(s) {
    if (g_no_alloc_call) return;
    std::lock_guard<std::mutex> lk(g_timing_mu);
    if (!g_timing_enabled) return;
    start = take_event();
    stop = take_event();
    if (start && stop) (void)hipEventRecord(start, stream);
  }
  ~LaunchTimer() {
    if (!start || !stop) return;
    (void)hipEventRecord(stop, stream);
    std::lock_guard<std::mutex> lk(g_timing_mu);
    g_timing_pending.push_back({name, start, stop});
  }
};

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ uint64_t lanes_below() {
  return (uint64_t(1) << lane_id()) - 1;
}

__device__ __forceinline__ int key_rank(uint64_t k) { return int(uint32_t(k >> 32)); }
__device__ __forceinline__ uint32_t key_index(uint64_t k) { return uint32_t(k); }

__device__ __forceinline__ unsigned key_digit(uint64_t k, int shift, unsigned mask) {
  return unsigned(k >> (32 + shift)) & mask;
}

// Counts the digits held by the 64 lanes of a wave into cnt with one LDS
// atomic per run of equal digits in consecutive lanes (its first lane adds
// the run length).  Sorted keys hold long runs of one digit, which a
// per-lane atomic would serialise on one LDS address.  Lanes with valid ==
// false count nothing and end any run.  All 64 lanes must be active.
__device__ __forceinline__ void count_digit_runs(int *cnt, unsigned digit, bool valid) {
  const unsigned d = valid ? digit : 0xffffffffu;
  // digit of the lane below (wave shift right by one); lane 0 gets ~d
  const unsigned below = unsigned(__builtin_amdgcn_update_dpp(int(~d), int(d), 0x138, 0xf, 0xf,
                                                              false));
  const bool head = d != below;
  const uint64_t heads = __ballot(head);
  const int lane = lane_id();
  const uint64_t after = heads & ~((uint64_t(2) << lane) - 1);  // heads above this lane
  const int next = after ? __builtin_ctzll(after) : 64;
  if (valid && head) atomicAdd(&cnt[d], next - lane);
}

// OR of v over the 64 lanes (all active), in every lane's SGPR: DPP row
// shifts, row broadcasts 15 / 31, lane 63.
__device__ __forceinline__ unsigned wave_or(unsigned v) {
  int x = int(v);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x |= __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x |= __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x |= __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x |= __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x |= __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return unsigned(__builtin_amdgcn_readlane(x, 63));
}

// The valid lanes of the wave whose digit equals this lane's (a stable
// in-wave rank is the count of them below this lane).  Only the digit bits
// that differ between valid lanes can split them: one wave OR finds those,
// and each costs a ballot and a per-lane 64-bit combine (the VALU cost of
// the rank).  Sorted and clustered keys leave most bits uniform in a wave.
// All 64 lanes must be active.
__device__ __forceinline__ uint64_t peer_mask(unsigned dg, bool valid) {
  const uint64_t vm = __ballot(valid);
  if (vm == 0) return 0;
  const unsigned d0 = unsigned(__builtin_amdgcn_readlane(int(dg), int(__builtin_ctzll(vm))));
  uint64_t peers = vm;
  for (unsigned m = wave_or(valid ? dg ^ d0 : 0u); m; m &= m - 1) {
    const bool bit = (dg >> __builtin_ctz(m)) & 1u;
    const uint64_t bal = __ballot(bit);
    peers &= bit ? bal : ~bal;
  }
  return peers;
}

// Stable rank of this lane's key among the valid lanes of its wave with the
// same digit (`below`: how many come before it) and their number (`same`).
// When every lane is valid and the digits are monotone across the lanes (as
// keys in point order often are), each digit forms one run of lanes and both
// follow from the run starts: a DPP shift, four ballots and a few bit scans.
// Otherwise from the peer mask.  Either way the same numbers.  All 64 lanes
// must be active.
__device__ __forceinline__ void digit_rank(unsigned dg, bool valid, int &below, int &same) {
  const int lane = lane_id();
  const uint64_t le = (uint64_t(2) << lane) - 1;  // lanes <= this one
  if (__ballot(valid) == ~uint64_t(0)) {
    // digit of the lane below (lane 0 keeps its own)
    const unsigned prev =
        unsigned(__builtin_amdgcn_update_dpp(int(dg), int(dg), 0x138, 0xf, 0xf, false));
    if (__ballot(dg < prev) == 0 || __ballot(dg > prev) == 0) {
      const uint64_t heads = __ballot(dg != prev) | uint64_t(1);
      const int start = 63 - __builtin_clzll(heads & le);
      const uint64_t after = heads & ~le;
      below = lane - start;
      same = (after ? __builtin_ctzll(after) : 64) - start;
      return;
    }
  }
  const uint64_t peers = peer_mask(dg, valid);
  below = __popcll(peers & (le >> 1));
  same = __popcll(peers);
}

// Exclusive scan of one int per thread across a block of kW waves (256
// threads by default).  `scratch` holds kW ints.  Every thread must call it.
template <int kW = kWaves>
__device__ int block_exclusive_scan(int v, int *scratch, int *total) {
  const int lane = lane_id(), w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    int s = scratch[i];
    before += (i < w) ? s : 0;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return before + x - v;
}

// fp32 / fp16 / bf16 element conversion.
struct F32 {
  using raw = uint32_t;
  __device__ static float load(const uint32_t *p) { return __builtin_bit_cast(float, *p); }
  __device__ static void store(uint32_t *p, float v) { *p = __builtin_bit_cast(uint32_t, v); }
  __device__ static uint32_t to_raw(float v) { return __builtin_bit_cast(uint32_t, v); }
};
struct F16 {
  using raw = uint16_t;
  __device__ static float load(const uint16_t *p) {
    return float(__builtin_bit_cast(_Float16, *p));
  }
  __device__ static void store(uint16_t *p, float v) {
    *p = __builtin_bit_cast(uint16_t, _Float16(v));
  }
  __device__ static uint16_t to_raw(float v) { return __builtin_bit_cast(uint16_t, _Float16(v)); }
  __device__ static float from_raw(uint32_t r) {
    return float(__builtin_bit_cast(_Float16, uint16_t(r)));
  }
};
struct BF16 {
  using raw = uint16_t;
  __device__ static float load(const uint16_t *p) {
    return __builtin_bit_cast(float, uint32_t(*p) << 16);
  }
  // round to nearest even; NaN -> canonical quiet NaN (torch's c10::BFloat16)
  __device__ static uint16_t to_raw(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
  }
  __device__ static void store(uint16_t *p, float v) { *p = to_raw(v); }
  __device__ static float from_raw(uint32_t r) { return __builtin_bit_cast(float, r << 16); }
};

// ---------------------------------------------------------------------------
// index stage kernels
// ---------------------------------------------------------------------------

// n / d for n < 2^31 by multiply-high and shift (Granlund & Montgomery,
// "Division by invariant integers using multiplication", 1994): with
// s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 (host side),
// q = (mulhi(n, m) + n) >> s; mulhi(n, m) <= n keeps the sum in 32 bits.
struct FastDiv {
  uint32_t d, m, s;
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return (__umulhi(n, m) + n) >> s;
  }
};

inline FastDiv make_fast_div(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
  return FastDiv{d, uint32_t(m), s};
}

// models/vtransforms/base.py:139-158: q = ((g - (bx - dx/2)) / dx).long(),
// kept iff 0 <= q_k < nx[k].  In fp32, trunc(q) in [0, n) <=> q > -1 && q < n
// (NaN fails both), which avoids converting out-of-range floats.
// Rank: ops/bev_pool/src/bev_pool_triton.py:34-39 with (D, H, W) = (nz, nx, ny).
__device__ __forceinline__ int quantize_point(float gx, float gy, float gz, int b, float o0,
                                              float o1, float o2, float d0, float d1, float d2,
                                              int n0, int n1, int n2) {
  const float q0 = (gx - o0) / d0;
  const float q1 = (gy - o1) / d1;
  const float q2 = (gz - o2) / d2;
  const bool kept = (q0 > -1.0f) & (q0 < float(n0)) & (q1 > -1.0f) & (q1 < float(n1)) &
                    (q2 > -1.0f) & (q2 < float(n2));
  if (!kept) return -1;
  const int x = int(q0), y = int(q1), z = int(q2);
  return ((b * n2 + z) * n0 + x) * n1 + y;
}

// Each thread handles groups of 4 consecutive points (group g of the block:
// points base + 4 * (g * kThreads + tid) + 0..3); with kVec (row stride 3
// floats, 16-byte aligned base) a group is three 16-byte loads and one
// 16-byte rank store.  All groups' loads are issued before any is used.
template <bool kVec, int kIt>
__global__ __launch_bounds__(kThreads) void quantize_geom_kernel(
    const float *__restrict__ geom, int64_t n_points, int64_t gstride, FastDiv ppb, float o0,
    float o1, float o2, float d0, float d1, float d2, int n0, int n1, int n2,
    int32_t *__restrict__ rank, int32_t *__restrict__ hist, int nblocks, int shift, int bits,
    int32_t *__restrict__ meta) {
  constexpr int kGroups = kIt / 4;
  __shared__ int cnt[kMaxRadix];
  if (blockIdx.x == 0 && threadIdx.x < BEVPOOL_META_LEN)  // nothing else touches meta here
    meta[threadIdx.x] = threadIdx.x == BEVPOOL_META_FIRST_BAD ? 0x7fffffff : 0;
  const int tile = int(xcd_chunk(blockIdx.x, gridDim.x));
  if (tile >= nblocks) return;  // grid padding, or the one block of an empty launch
  const int R = 1 << bits;
  const unsigned mask = unsigned(R - 1);
  for (int d = threadIdx.x; d < R; d += kThreads) cnt[d] = 0;
  const uint32_t base = uint32_t(tile) * (kThreads * kIt);  // n_points < 2^31
  const uint32_t n = uint32_t(n_points);
  // raw fp32 bits: lanes of a 16-byte load are never bit cast to float
  // while still in vector form (hipcc 7.2 folded such casts of lanes y/z/w
  // into lane x)
  uint32_t g[kGroups][12];
  const uint32_t *gb = reinterpret_cast<const uint32_t *>(geom);
#pragma unroll
  for (int k = 0; k < kGroups; ++k) {
    const uint32_t p0 = base + 4u * (uint32_t(k) * kThreads + threadIdx.x);
    if (kVec) {
      // groups past the last whole one read that one (in bounds, n >= 4);
      // a partial group is reloaded point by point below
      const uint32_t last = (n - 4) & ~3u;
      const uint32_t q0 = p0 + 3 < n ? p0 : last;
      const u32x4 *src = reinterpret_cast<const u32x4 *>(gb + int64_t(q0) * 3);
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const u32x4 v = src[j];
        g[k][4 * j + 0] = v.x;
        g[k][4 * j + 1] = v.y;
        g[k][4 * j + 2] = v.z;
        g[k][4 * j + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t p = p0 + u < n ? p0 + u : n - 1;
        const uint32_t *gp = gb + int64_t(p) * gstride;
        g[k][3 * u + 0] = gp[0];
        g[k][3 * u + 1] = gp[1];
        g[k][3 * u + 2] = gp[2];
      }
    }
  }
  __syncthreads();  // cnt zeroed
#pragma unroll
  for (int k = 0; k < kGroups; ++k) {
    const uint32_t p0 = base + 4u * (uint32_t(k) * kThreads + threadIdx.x);
    if (kVec && p0 < n && p0 + 3 >= n) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        if (p0 + u < n) {
          const uint32_t *gp = gb + int64_t(p0 + u) * 3;
          g[k][3 * u + 0] = gp[0];
          g[k][3 * u + 1] = gp[1];
          g[k][3 * u + 2] = gp[2];
        }
      }
    }
    int r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      r[u] = quantize_point(__builtin_bit_cast(float, g[k][3 * u]),
                            __builtin_bit_cast(float, g[k][3 * u + 1]),
                            __builtin_bit_cast(float, g[k][3 * u + 2]), int(ppb.div(p0 + u)),
                            o0, o1, o2, d0, d1, d2, n0, n1, n2);
      count_digit_runs(cnt, (unsigned(r[u]) >> shift) & mask, r[u] >= 0 && p0 + u < n);
    }
    if (kVec && p0 + 3 < n) {
      u32x4 w;
      w.x = uint32_t(r[0]);
      w.y = uint32_t(r[1]);
      w.z = uint32_t(r[2]);
      w.w = uint32_t(r[3]);
      *reinterpret_cast<u32x4 *>(rank + p0) = w;
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (p0 + u < n) rank[p0 + u] = r[u];
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += kThreads) hist[int64_t(d) * nblocks + tile] = cnt[d];
}

// ---- geometry from camera matrices, fused with the quantisation -----------
//
// models/vtransforms/base.py:82-126 (get_geometry) per point, in fp32 with
// every product and sum rounded separately (no contraction), each 3x3
// product summed left to right:
//   a = frustum[d, h, w] - post_trans          (base.py:95)
//   b = post_rots^T a                           (:96-98)
//   c = (b0 b2, b1 b2, b2)                      (:100-106)
//   g = combine c + camera2lidar_trans          (:107-112)
//   g = extra_rots g + extra_trans              (:114-123, when given)
// then quantize_point as for a geometry tensor.  combine = rots inv(intrins)
// (the reference's linalg.solve) is formed in double from the adjugate of
// intrins and rounded to fp32 once.  Per camera the kernel works from a
// 24-float table: post_rots^T (9, row-major), post_trans (3), combine (9),
// camera2lidar_trans (3); per batch a 12-float table: extra_rots (9),
// extra_trans (3).
constexpr int kCamFloats = 24;
constexpr int kBatchFloats = 12;
constexpr int kCamSlots = 16;  // cameras a block stages in LDS

struct CameraMats {  // fp32, row-major, contiguous per camera / batch
  const float *rots, *trans, *intrins, *post_rots, *post_trans;  // [B*N][9|3]
  const float *extra_rots, *extra_trans;                         // [B][9|3] or null
  int n_per_batch;                                               // N
  __device__ __forceinline__ bool has_extra() const { return extra_rots || extra_trans; }
};

// One camera's inputs, all loaded before any is used (one round trip).
struct CamIn {
  float pr[9], pt[3], k[9], r[9], tr[3];
};

__device__ __forceinline__ void load_camera(const CameraMats &m, uint32_t cam, CamIn &c) {
  const int64_t o9 = int64_t(cam) * 9, o3 = int64_t(cam) * 3;
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    c.pr[i] = m.post_rots[o9 + i];
    c.k[i] = m.intrins[o9 + i];
    c.r[i] = m.rots[o9 + i];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    c.pt[i] = m.post_trans[o3 + i];
    c.tr[i] = m.trans[o3 + i];
  }
}

__device__ void build_camera_table(const CamIn &c, float *__restrict__ t) {
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) t[3 * i + j] = c.pr[3 * j + i];  // post_rots^T
  for (int i = 0; i < 3; ++i) t[9 + i] = c.pt[i];
  double k[9];
  for (int i = 0; i < 9; ++i) k[i] = double(c.k[i]);
  const double c00 = k[4] * k[8] - k[5] * k[7], c01 = k[5] * k[6] - k[3] * k[8];
  const double c02 = k[3] * k[7] - k[4] * k[6];
  const double det = k[0] * c00 + k[1] * c01 + k[2] * c02;
  double inv[9] = {c00, k[2] * k[7] - k[1] * k[8], k[1] * k[5] - k[2] * k[4],
                   c01, k[0] * k[8] - k[2] * k[6], k[2] * k[3] - k[0] * k[5],
                   c02, k[1] * k[6] - k[0] * k[7], k[0] * k[4] - k[1] * k[3]};
  for (int i = 0; i < 9; ++i) inv[i] /= det;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      double v = 0.0;
      for (int q = 0; q < 3; ++q) v += double(c.r[3 * i + q]) * inv[3 * q + j];
      t[12 + 3 * i + j] = float(v);
    }
  for (int i = 0; i < 3; ++i) t[21 + i] = c.tr[i];
}

__device__ void camera_table(const CameraMats &m, uint32_t cam, float *__restrict__ t) {
  CamIn c;
  load_camera(m, cam, c);
  build_camera_table(c, t);
}

// The lidar-augmentation table of batch b (identity when absent), with one
// branch per pointer so that its loads are issued together.
__device__ __forceinline__ void batch_table(const CameraMats &m, uint32_t b,
                                            float *__restrict__ t) {
  if (m.extra_rots) {
#pragma unroll
    for (int i = 0; i < 9; ++i) t[i] = m.extra_rots[int64_t(b) * 9 + i];
  } else {
#pragma unroll
    for (int i = 0; i < 9; ++i) t[i] = i % 4 == 0 ? 1.0f : 0.0f;
  }
  if (m.extra_trans) {
#pragma unroll
    for (int i = 0; i < 3; ++i) t[9 + i] = m.extra_trans[int64_t(b) * 3 + i];
  } else {
#pragma unroll
    for (int i = 0; i < 3; ++i) t[9 + i] = 0.0f;
  }
}

__device__ __forceinline__ void frustum_point(const float *__restrict__ c,
                                              const float *__restrict__ e, float fx, float fy,
                                              float fz, float &gx, float &gy, float &gz) {
  const float a0 = fx - c[9], a1 = fy - c[10], a2 = fz - c[11];
  const float b0 = (c[0] * a0 + c[1] * a1) + c[2] * a2;
  const float b1 = (c[3] * a0 + c[4] * a1) + c[5] * a2;
  const float b2 = (c[6] * a0 + c[7] * a1) + c[8] * a2;
  const float c0 = b0 * b2, c1 = b1 * b2;
  gx = ((c[12] * c0 + c[13] * c1) + c[14] * b2) + c[21];
  gy = ((c[15] * c0 + c[16] * c1) + c[17] * b2) + c[22];
  gz = ((c[18] * c0 + c[19] * c1) + c[20] * b2) + c[23];
  if (e) {
    const float h0 = ((e[0] * gx + e[1] * gy) + e[2] * gz) + e[9];
    const float h1 = ((e[3] * gx + e[4] * gy) + e[5] * gz) + e[10];
    const float h2 = ((e[6] * gx + e[7] * gy) + e[8] * gz) + e[11];
    gx = h0;
    gy = h1;
    gz = h2;
  }
}

// Point p = cam * DHW + f (cam = b*N + n, f = (d*fH + h)*fW + w); frustum
// fp32 (D, fH, fW, 3) contiguous.  A block takes kThreads * kIt consecutive points
// (as quantize_geom_kernel, so the pass-0 histograms line up); its first
// threads build the tables of the cameras it spans in LDS.  A block spanning
// more than kCamSlots cameras (frustums under ~140 points) builds each
// point's table in registers instead.
template <int kIt>
__global__ __launch_bounds__(kThreads) void quantize_frustum_kernel(
    const float *__restrict__ frustum, int64_t n_points, FastDiv dhw, FastDiv npb, CameraMats cm,
    float o0,
    float o1, float o2, float d0, float d1, float d2, int n0, int n1, int n2,
    int32_t *__restrict__ rank, int32_t *__restrict__ hist, int nblocks, int shift, int bits,
    int32_t *__restrict__ meta) {
  __shared__ int cnt[kMaxRadix];
  __shared__ float lcam[kCamSlots][kCamFloats];
  __shared__ float lbat[kCamSlots][kBatchFloats];
  if (blockIdx.x == 0 && threadIdx.x < BEVPOOL_META_LEN)
    meta[threadIdx.x] = threadIdx.x == BEVPOOL_META_FIRST_BAD ? 0x7fffffff : 0;
  const int tile = int(xcd_chunk(blockIdx.x, gridDim.x));
  if (tile >= nblocks) return;
  const int R = 1 << bits;
  const unsigned mask = unsigned(R - 1);
  for (int d = threadIdx.x; d < R; d += kThreads) cnt[d] = 0;
  const uint32_t n = uint32_t(n_points);
  const uint32_t base = uint32_t(tile) * (kThreads * kIt);
  const uint32_t last = (base + (kThreads * kIt) < n ? base + (kThreads * kIt) : n) - 1;
  const uint32_t cam_lo = dhw.div(base), cam_hi = dhw.div(last);
  const bool staged = cam_hi - cam_lo < uint32_t(kCamSlots);
  const bool extra = cm.has_extra();
  // all frustum loads first (points past n reload point n - 1), issued
  // before the camera tables are built so that their latencies overlap
  float fx[kIt], fy[kIt], fz[kIt];
  uint32_t camv[kIt];
  if (staged) {
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const uint32_t p = base + uint32_t(k) * kThreads + threadIdx.x;
      const uint32_t pc = p < n ? p : n - 1;
      const uint32_t cam = dhw.div(pc), f = pc - cam * dhw.d;
      camv[k] = cam;
      fx[k] = frustum[int64_t(f) * 3];
      fy[k] = frustum[int64_t(f) * 3 + 1];
      fz[k] = frustum[int64_t(f) * 3 + 2];
    }
  }
  if (staged && threadIdx.x <= cam_hi - cam_lo) {
    // the camera's and its batch's inputs loaded together, then the tables
    const uint32_t cam = cam_lo + threadIdx.x;
    CamIn c;
    load_camera(cm, cam, c);
    float e[kBatchFloats];
    if (extra) batch_table(cm, npb.div(cam), e);
    build_camera_table(c, lcam[threadIdx.x]);
    if (extra)
#pragma unroll
      for (int i = 0; i < kBatchFloats; ++i) lbat[threadIdx.x][i] = e[i];
  }
  __syncthreads();
  if (staged) {
    // then the products; digit counts by runs (every lane active)
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const uint32_t p = base + uint32_t(k) * kThreads + threadIdx.x;
      const uint32_t c = camv[k] - cam_lo;
      float gx, gy, gz;
      frustum_point(lcam[c], extra ? lbat[c] : nullptr, fx[k], fy[k], fz[k], gx, gy, gz);
      const int r = quantize_point(gx, gy, gz, int(npb.div(camv[k])), o0, o1, o2, d0, d1, d2, n0,
                                   n1, n2);
      count_digit_runs(cnt, (unsigned(r) >> shift) & mask, p < n && r >= 0);
      if (p < n) rank[p] = r;
    }
  } else {
    // more cameras than LDS slots: each point's tables in registers
    for (int k = 0; k < kIt; ++k) {
      const uint32_t p = base + uint32_t(k) * kThreads + threadIdx.x;
      int r = -1;
      if (p < n) {
        const uint32_t cam = dhw.div(p), f = p - cam * dhw.d;
        const float *fr = frustum + int64_t(f) * 3;
        float gx, gy, gz;
        float ct[kCamFloats], bt[kBatchFloats];
        camera_table(cm, cam, ct);
        if (extra) batch_table(cm, npb.div(cam), bt);
        frustum_point(ct, extra ? bt : nullptr, fr[0], fr[1], fr[2], gx, gy, gz);
        r = quantize_point(gx, gy, gz, int(npb.div(cam)), o0, o1, o2, d0, d1, d2, n0, n1, n2);
        if (r >= 0) atomicAdd(&cnt[(unsigned(r) >> shift) & mask], 1);
        rank[p] = r;
      }
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += kThreads) hist[int64_t(d) * nblocks + tile] = cnt[d];
}

// ops/bev_pool/src/bev_pool_triton.py:34-39 in int64 (wrapping) arithmetic.
// Invalid ranks are counted into meta with atomics (meta initialised by an
// earlier launch) or, with kTileBad, per tile into tile_bad[tile] (count) and
// tile_bad[nblocks + tile] (smallest point index, INT32_MAX if none), which
// the first scatter reduces into meta -- so the op level needs no separate
// launch to initialise meta.
template <typename TC, int kIt, bool kTileBad>
__global__ __launch_bounds__(kThreads) void coord_ranks_kernel(
    const TC *__restrict__ coords, int64_t n_points, int64_t cstride, int64_t B, int64_t D,
    int64_t H, int64_t W, int32_t *__restrict__ rank, int32_t *__restrict__ meta,
    int32_t *__restrict__ hist, int nblocks, int shift, int bits,
    int32_t *__restrict__ tile_bad) {
  __shared__ int cnt[kMaxRadix];
  __shared__ int s_bad[2];
  const int R = 1 << bits;
  const unsigned mask = unsigned(R - 1);
  const int tile = int(xcd_chunk(blockIdx.x, gridDim.x));
  if (tile >= nblocks) return;  // grid padding
  for (int d = threadIdx.x; d < R; d += kThreads) cnt[d] = 0;
  if (kTileBad && threadIdx.x == 0) {
    s_bad[0] = 0;
    s_bad[1] = INT32_MAX;
  }
  __syncthreads();
  const int64_t base = int64_t(tile) * (kThreads * kIt);
  const uint64_t cells = uint64_t(B * D * H * W);
  // the coordinates of kBatch points per thread are loaded before any is
  // used (clamped to the last point, so the loads need no branch); the
  // digits are counted one atomic per run of equal digits
  constexpr int kBatch = sizeof(TC) == 4 ? 8 : 4;  // 32 VGPRs of coordinates
  static_assert(kIt % kBatch == 0, "whole batches per thread");
  for (int k0 = 0; k0 < kIt; k0 += kBatch) {
    TC cv[kBatch][4];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t p = base + int64_t(k0 + u) * kThreads + threadIdx.x;
      const TC *c = coords + (p < n_points ? p : n_points - 1) * cstride;
#pragma unroll
      for (int j = 0; j < 4; ++j) cv[u][j] = c[j];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t p = base + int64_t(k0 + u) * kThreads + threadIdx.x;
      const uint64_t x = uint64_t(int64_t(cv[u][0])), y = uint64_t(int64_t(cv[u][1]));
      const uint64_t z = uint64_t(int64_t(cv[u][2])), b = uint64_t(int64_t(cv[u][3]));
      const uint64_t r64 = ((b * uint64_t(D) + z) * uint64_t(H) + x) * uint64_t(W) + y;
      const bool ok = p < n_points && r64 < cells;  // unsigned: negative ranks fail too
      const int r = ok ? int(r64) : -1;
      count_digit_runs(cnt, (unsigned(r) >> shift) & mask, ok);  // every lane takes part
      if (p < n_points) {
        if (!ok) {
          if (kTileBad) {
            atomicAdd(&s_bad[0], 1);
            atomicMin(&s_bad[1], int(p));
          } else {
            atomicAdd(&meta[BEVPOOL_META_N_BAD], 1);
            atomicMin(&meta[BEVPOOL_META_FIRST_BAD], int(p));
          }
        }
        rank[p] = r;
      }
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += kThreads) hist[int64_t(d) * nblocks + tile] = cnt[d];
  if (kTileBad && threadIdx.x == 0) {
    tile_bad[tile] = s_bad[0];
    tile_bad[nblocks + tile] = s_bad[1];
  }
}

__global__ void init_meta_kernel(int32_t *meta) {
  if (threadIdx.x < BEVPOOL_META_LEN)
    meta[threadIdx.x] = threadIdx.x == BEVPOOL_META_FIRST_BAD ? 0x7fffffff : 0;
}


// One block per digit: exclusive scan over the blocks of hist[d][*] in place,
// totals[d] = row sum.  Optionally zeroes the dense cell ranges (grid-stride).
__global__ __launch_bounds__(kThreads) void radix_scan_kernel(
    int32_t *__restrict__ hist, int nblocks, int32_t *__restrict__ totals,
    int32_t *__restrict__ cstart, int32_t *__restrict__ cend, int64_t zero_cells) {
  __shared__ int scratch[kWaves];
  int32_t *row = hist + int64_t(blockIdx.x) * nblocks;
  int carry = 0;
  for (int t0 = 0; t0 < nblocks; t0 += kThreads * 4) {
    int v[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = t0 + threadIdx.x * 4 + i;
      v[i] = j < nblocks ? row[j] : 0;
      s += v[i];
    }
    int tot;
    int ex = block_exclusive_scan(s, scratch, &tot) + carry;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = t0 + threadIdx.x * 4 + i;
      if (j < nblocks) row[j] = ex;
      ex += v[i];
    }
    carry += tot;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
  for (int64_t c = int64_t(blockIdx.x) * kThreads + threadIdx.x; c < zero_cells;
       c += int64_t(gridDim.x) * kThreads) {
    cstart[c] = 0;
    cend[c] = 0;
  }
}

// Block histogram of one digit over the sorted keys of the previous pass.
template <int kIt>
__global__ __launch_bounds__(kThreads) void radix_hist_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    int32_t *__restrict__ hist, int nblocks, int shift, int bits) {
  __shared__ int cnt[kMaxRadix];
  const int R = 1 << bits;
  const unsigned mask = unsigned(R - 1);
  const int tile = int(xcd_chunk(blockIdx.x, gridDim.x));
  if (tile >= nblocks) return;  // grid padding
  for (int d = threadIdx.x; d < R; d += kThreads) cnt[d] = 0;
  __syncthreads();
  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t base = int64_t(tile) * (kThreads * kIt);
  // all loads first (in bounds: past n they read key 0), then the counts
  uint64_t key[kIt];
#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    const int64_t e = base + int64_t(k) * kThreads + threadIdx.x;
    key[k] = keys[e < n ? e : 0];
  }
#pragma unroll
  for (int k = 0; k < kIt; ++k)
    count_digit_runs(cnt, key_digit(key[k], shift, mask),
                     base + int64_t(k) * kThreads + threadIdx.x < n);
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += kThreads) hist[int64_t(d) * nblocks + tile] = cnt[d];
}

// Stable scatter of one LSD radix pass.  Wave w of block b owns the 64 * kIt
// consecutive keys [(b*4 + w) * 64 * kIt, +64 * kIt) and walks them 64 at a
// time in order; a key's destination is
//   (keys of smaller digits overall) + (same digit in earlier blocks)
//   + (same digit in earlier waves of this block) + (same digit earlier in
//   this wave),
// the last term from a ballot-built peer mask, so equal digits keep their
// input order.  Pass 0 (kFromRank) reads int32 ranks in point order, skips
// dropped points (compaction) and builds the (rank << 32 | point) keys.
template <bool kFromRank, int kIt>
__global__ __launch_bounds__(kThreads) void radix_scatter_kernel(
    const int32_t *__restrict__ rank_in, const uint64_t *__restrict__ keys_in,
    int64_t n_points, int32_t *__restrict__ meta, uint64_t *__restrict__ keys_out,
    const int32_t *__restrict__ hist, const int32_t *__restrict__ totals, int nblocks,
    int shift, int bits, const int32_t *__restrict__ tile_bad, int32_t *__restrict__ gstart) {
  __shared__ int s_base[kMaxRadix];
  __shared__ int s_cnt[kWaves * kMaxRadix];
  __shared__ int s_scan[kWaves];
  const int R = 1 << bits;
  const unsigned mask = unsigned(R - 1);
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int64_t n = kFromRank ? n_points : int64_t(meta[BEVPOOL_META_N_KEPT]);
  // XCD-contiguous tiles: a digit's runs from neighbouring tiles are adjacent
  // in the output, so writing them from one XCD lets its L2 merge them into
  // whole lines
  const int tile = int(xcd_chunk(blockIdx.x, gridDim.x));
  const int64_t blk0 = int64_t(tile) * (kThreads * kIt);
  if (tile >= nblocks || blk0 >= n) return;  // whole block leaves before any barrier

  // this wave's keys, in order (loads issued first so that their latency
  // overlaps the digit-base computation below)
  uint64_t key[kIt];
  bool valid[kIt];
  const int64_t wbase = blk0 + int64_t(w) * (64 * kIt);
#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    const int64_t e = wbase + k * 64 + lane;
    if (kFromRank) {
      const int r = rank_in[e < n ? e : n - 1];
      valid[k] = e < n && r >= 0;
      key[k] = (uint64_t(uint32_t(r)) << 32) | uint64_t(uint32_t(e));
    } else {
      valid[k] = e < n;
      key[k] = keys_in[e < n ? e : n - 1];
    }
  }

  // digit bases: exclusive scan of the digit totals + this block's prefix
  // (both loaded before the scan, so their latencies overlap); tile 0's bases
  // are the digit starts, kept in gstart for the per-group sort
  constexpr int kPer = kMaxRadix / kThreads;  // digits per thread (4)
  int loc[kPer], pre[kPer], tsum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = tid * kPer + i;
    loc[i] = d < R ? totals[d] : 0;
    pre[i] = d < R ? hist[int64_t(d) * nblocks + tile] : 0;
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) tsum += loc[i];
  for (int d = tid; d < kWaves * R; d += kThreads) s_cnt[d] = 0;
  int total;
  int ex = block_exclusive_scan(tsum, s_scan, &total);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = tid * kPer + i;
    if (d < R) {
      s_base[d] = ex + pre[i];
      if (gstart && tile == 0) gstart[d] = ex;
    }
    ex += loc[i];
  }
  if (kFromRank && tile == 0) {
    if (tile_bad) {
      // ranks from coord_ranks_kernel<..., true>: meta was never initialised;
      // write all of it (kept count, the reduced invalid-rank counters, zeros)
      int nbad = 0, first = INT32_MAX;
      for (int t = tid; t < nblocks; t += kThreads) {
        nbad += tile_bad[t];
        first = min(first, tile_bad[nblocks + t]);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        nbad += __shfl_xor(nbad, o, 64);
        first = min(first, __shfl_xor(first, o, 64));
      }
      __shared__ int s_red[2 * kWaves];
      if (lane == 0) {
        s_red[w] = nbad;
        s_red[kWaves + w] = first;
      }
      __syncthreads();
      if (tid < BEVPOOL_META_LEN) {
        int v = 0;
        if (tid == BEVPOOL_META_N_KEPT) {
          v = total;
        } else if (tid == BEVPOOL_META_N_BAD) {
#pragma unroll
          for (int i = 0; i < kWaves; ++i) v += s_red[i];
        } else if (tid == BEVPOOL_META_FIRST_BAD) {
          v = INT32_MAX;
#pragma unroll
          for (int i = 0; i < kWaves; ++i) v = min(v, s_red[kWaves + i]);
        }
        meta[tid] = v;
      }
    } else if (tid == 0) {
      meta[BEVPOOL_META_N_KEPT] = total;
    }
  }
  __syncthreads();

  // per-wave digit counts
  int *cnt = s_cnt + w * R;
#pragma unroll
  for (int k = 0; k < kIt; ++k) count_digit_runs(cnt, key_digit(key[k], shift, mask), valid[k]);
  __syncthreads();
  for (int d = tid; d < R; d += kThreads) {
    int run = s_base[d];
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const int c = s_cnt[ww * R + d];
      s_cnt[ww * R + d] = run;
      run += c;
    }
  }
  __syncthreads();

#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    const unsigned dg = key_digit(key[k], shift, mask);
    int below, same;
    digit_rank(dg, valid[k], below, same);
    if (valid[k]) {
      const int pos = cnt[dg] + below;
      keys_out[pos] = key[k];
      if (below == 0) cnt[dg] = pos + same;
    }
  }
}

// Second half of the sort when the ranks need 11..20 bits.  One global pass
// (radix_scatter_kernel<true> by the high digit rank >> lbits) has grouped
// the kept keys by high digit, each group in point order.  The keys of group
// b are sorted stably by the low lbits bits, so the keys end sorted by rank
// with ties in point order, as two LSD passes would leave them, and the dense
// [start, end) of the group's 2^lbits cells is written (0, 0 when empty),
// which replaces cell_ranges_kernel and the zeroing of the cell ranges.
// A group of gn keys is cut into P = min(parts_max, ceil(gn / part_keys))
// consecutive parts, one block each, so that a large group (the cells near
// the cameras) is not ranked by one block alone.  The block of part p first
// counts the digits of the group's other keys (those before its part apart),
// then walks its own part as one block walks a whole group:
// Wave w of kBucketWaves owns the w-th slice of the part (a multiple of 64
// keys) and walks it 64 keys at a time, in order, twice: the first walk
// counts its digits, the second puts each key at
//   (group start) + (smaller digits in the group) + (same digit in earlier
//   parts) + (same digit in earlier waves) + (same digit earlier in this
//   wave),
// the last term from a ballot-built peer mask as in radix_scatter_kernel.
// No block waits for another.  Block i takes part parts_max - 1 - i / n of
// group i % n (n groups): the blocks of the later parts, of which only the
// large groups' do any work, come first, so that those start at once.  The
// block of part 0 writes the cell ranges.  Keys are loaded kBucketBatch
// sub-batches (of 64) at a time; a wave whose slice fits in one batch keeps
// it in registers for the second walk.  Otherwise the second walk drains
// each batch's loads before its first key store: vmcnt counts loads and
// stores together, so a wait for a load issued after a store would also wait
// for the store.  Dynamic LDS: (kBucketWaves + 2) * 2^lbits ints (16 waves,
// up to 512 digits: at most 36 KB per block).  Groups of 1024 cells take the
// sliced form below instead.
template <int kBucketWaves>
__global__ __launch_bounds__(64 * kBucketWaves, 8) void bucket_sort_kernel(
    const uint64_t *__restrict__ keys_in, const int32_t *__restrict__ totals,
    const int32_t *__restrict__ gstart, int n_buckets, int64_t n_cells,
    uint64_t *__restrict__ keys_out, int32_t *__restrict__ cstart, int32_t *__restrict__ cend,
    int lbits, int parts_max, int part_keys) {
  constexpr int kBucketThreads = 64 * kBucketWaves;
  // sub-batches per load batch: 12 keeps the 16-wave kernel within 64 VGPRs
  // (56; two blocks per CU) and a wave's part of any group up to 12,288 keys
  // in registers between its two walks (16 spills)
  constexpr int kBucketBatch = 12;
  extern __shared__ int s_cnt[];  // [kBucketWaves][R] own part, then [R] other parts, [R] before
  __shared__ int s_scan[kBucketWaves];
  const int bkt = int(blockIdx.x) % n_buckets;
  const int part = parts_max - 1 - int(blockIdx.x) / n_buckets;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int R = 1 << lbits;
  const unsigned mask = unsigned(R - 1);

  // group start (keys of smaller high digits, from the global pass) and size
  const int gs = gstart[bkt];
  const int gn = totals[bkt];
  const int np = gn > part_keys ? (gn + part_keys - 1) / part_keys : 1;
  const int P = np < parts_max ? np : parts_max;
  if (part >= P) return;
  // this part: [ps, pe), a multiple of 64 keys but the last
  const int L = ((gn + P - 1) / P + 63) & ~63;
  const int64_t ge = int64_t(gs) + gn;
  const int ps = int(gs + int64_t(part) * L < ge ? gs + int64_t(part) * L : ge);
  const int pe = int(gs + int64_t(part + 1) * L < ge ? gs + int64_t(part + 1) * L : ge);
  int *s_out = s_cnt + kBucketWaves * R;  // digits of the group's other parts
  int *s_before = s_out + R;              // digits of the parts before this one
  for (int d = tid; d < (kBucketWaves + 2) * R; d += kBucketThreads) s_cnt[d] = 0;
  const int64_t q = (int64_t(pe - ps) + kBucketThreads - 1) / kBucketThreads * 64;  // keys per wave
  const int wb = int(ps + w * q < pe ? ps + w * q : pe);
  const int we = int(ps + (w + 1) * q < pe ? ps + (w + 1) * q : pe);
  __syncthreads();

  uint64_t key[kBucketBatch];
  if (P > 1) {
    // the other parts' keys: [gs, ps) (counted as before this part too) and
    // [pe, ge), each range cut into wave slices
#pragma unroll 1
    for (int r = 0; r < 2; ++r) {
      const int a = r == 0 ? gs : pe, e = r == 0 ? ps : int(ge);
      const int64_t qo = (int64_t(e - a) + kBucketThreads - 1) / kBucketThreads * 64;
      const int ob = int(a + w * qo < e ? a + w * qo : e);
      const int oe = int(a + (w + 1) * qo < e ? a + (w + 1) * qo : e);
      for (int e0 = ob; e0 < oe; e0 += 64 * kBucketBatch) {
#pragma unroll
        for (int j = 0; j < kBucketBatch; ++j) {
          const int i = e0 + 64 * j + lane;
          if (e0 + 64 * j < oe) key[j] = keys_in[i < oe ? i : ob];
        }
#pragma unroll
        for (int j = 0; j < kBucketBatch; ++j)
          if (e0 + 64 * j < oe) {
            const unsigned dg = key_digit(key[j], 0, mask);
            const bool valid = e0 + 64 * j + lane < oe;
            count_digit_runs(s_out, dg, valid);
            if (r == 0) count_digit_runs(s_before, dg, valid);
          }
      }
    }
  }

  int *cnt = s_cnt + w * R;
  const bool resident = we - wb <= 64 * kBucketBatch;  // wave-uniform
  for (int e0 = wb; e0 < we; e0 += 64 * kBucketBatch) {
    // sub-batches past the slice end are skipped (wave-uniform tests)
#pragma unroll
    for (int j = 0; j < kBucketBatch; ++j) {
      const int e = e0 + 64 * j + lane;
      if (e0 + 64 * j < we) key[j] = keys_in[e < we ? e : wb];
    }
#pragma unroll
    for (int j = 0; j < kBucketBatch; ++j)
      if (e0 + 64 * j < we)
        count_digit_runs(cnt, key_digit(key[j], 0, mask), e0 + 64 * j + lane < we);
  }
  __syncthreads();

  // digit starts within the group (digits kPer * tid + i), the cells'
  // ranges (part 0), per-wave bases of this part
  constexpr int kPer = kMaxRadix / kBucketThreads;  // digits per thread (1 or 2)
  int tot[kPer], tsum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = kPer * tid + i;
    tot[i] = 0;
    if (d < R) {
#pragma unroll
      for (int ww = 0; ww < kBucketWaves; ++ww) tot[i] += s_cnt[ww * R + d];
      tot[i] += s_out[d];
    }
    tsum += tot[i];
  }
  int gtotal;
  int ex = gs + block_exclusive_scan<kBucketWaves>(tsum, s_scan, &gtotal);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = kPer * tid + i;
    if (d < R) {
      const int64_t cell = int64_t(bkt) * R + d;
      if (part == 0 && cell < n_cells) {
        cstart[cell] = tot[i] ? ex : 0;
        cend[cell] = tot[i] ? ex + tot[i] : 0;
      }
      int run = ex + s_before[d];
#pragma unroll
      for (int ww = 0; ww < kBucketWaves; ++ww) {
        const int c = s_cnt[ww * R + d];
        s_cnt[ww * R + d] = run;
        run += c;
      }
    }
    ex += tot[i];
  }
  __syncthreads();

  for (int e0 = wb; e0 < we; e0 += 64 * kBucketBatch) {
    if (!resident) {
#pragma unroll
      for (int j = 0; j < kBucketBatch; ++j) {
        const int e = e0 + 64 * j + lane;
        if (e0 + 64 * j < we) key[j] = keys_in[e < we ? e : wb];
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the batch is in registers
    }
#pragma unroll
    for (int j = 0; j < kBucketBatch; ++j) {
      if (e0 + 64 * j >= we) break;
      const bool valid = e0 + 64 * j + lane < we;
      const unsigned dg = key_digit(key[j], 0, mask);
      int below, same;
      digit_rank(dg, valid, below, same);
      if (valid) {
        const int pos = cnt[dg] + below;
        keys_out[pos] = key[j];
        if (below == 0) cnt[dg] = pos + same;
      }
    }
  }
}

// Sliced form of the second half of the sort (same result as
// bucket_sort_kernel).  Each group of equal high digit, in point order after
// the global pass, is cut into slices of kSliceKeys consecutive keys, so that
// a large group (the cells near the cameras: up to ~65 K keys at 2 x 720 x
// 720) is spread over several blocks instead of being walked by one:
//   bucket_count_kernel   one block per slice: the slice's low-digit counts;
//   bucket_scan_kernel    one block per group: each slice's first sorted
//                         position per digit (in place of its counts) and
//                         the group's dense cell ranges;
//   bucket_place_kernel   one block per slice: each key to its position
//                         (the ranking of bucket_sort_kernel within a slice).
// Slices are numbered group by group; a block finds its slice from the group
// sizes (exclusive scans over the <= 1024 groups), so no kernel waits on
// another block.
constexpr int kSliceKeys = 8192;
// Groups of 2^kSlicedBits cells take the sliced form.  Smaller groups (at
// most ~35 K keys measured) take bucket_sort_kernel, whose one launch is
// faster there (MI355X: 21.6 against 41 us at 1 x 360 x 360, 51 against 74
// at 4 x 360 x 360; sorting one-slice groups in their place block and
// counting only the others still lost: 30.5 and 63 us); at 2^10 cells per
// group the sliced form takes 103 against 148 us (2 x 720 x 720).
constexpr int kSlicedBits = 10;
constexpr int kSliceWaves = 8;  // 8 waves x 2^10 per-wave digit counts: 32 KB of LDS

template <int kW>
struct SliceShape {
  static constexpr int kT = 64 * kW;
  static constexpr int kBatch = kSliceKeys / kT;  // 64-key sub-batches per wave
  static_assert(kBatch * kT == kSliceKeys && kBatch <= 16, "slice shape");
};

__host__ __device__ inline int slices_of(int keys) {
  return (keys + kSliceKeys - 1) / kSliceKeys;
}

// This block's slice: group g, slice id (== blockIdx.x; slices are numbered
// group by group), sorted positions [first, end).  False (for the whole
// block) past the last slice.  (Dealing the slices to the XCDs in 8
// contiguous ranges, so that a group's interleaved writes share one L2, was
// measured slower on MI355X.)
struct SliceLoc {
  int g, id, first, end;
};

template <int kW>
__device__ bool find_slice(const int32_t *__restrict__ totals, int n_groups, SliceLoc *loc) {
  constexpr int kT = 64 * kW;
  constexpr int kG = (kMaxRadix + kT - 1) / kT;  // groups per thread
  __shared__ int s_scan[kW];
  __shared__ int s_loc[4];
  const int tid = threadIdx.x;
  int gn[kG], tk = 0, ts = 0;
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    const int g = tid * kG + i;
    gn[i] = g < n_groups ? totals[g] : 0;
    tk += gn[i];
    ts += slices_of(gn[i]);
  }
  if (tid == 0) s_loc[0] = -1;  // ordered before the writes below by the scans' barriers
  int unused, n_slices;
  int kb = block_exclusive_scan<kW>(tk, s_scan, &unused);
  int sb = block_exclusive_scan<kW>(ts, s_scan, &n_slices);
  const int b = int(blockIdx.x);
  if (b >= n_slices) return false;  // block-uniform
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    const int ns = slices_of(gn[i]);
    if (b >= sb && b < sb + ns) {
      const int first = kb + (b - sb) * kSliceKeys;
      s_loc[0] = tid * kG + i;
      s_loc[1] = b;
      s_loc[2] = first;
      s_loc[3] = gn[i] - (b - sb) * kSliceKeys < kSliceKeys ? kb + gn[i] : first + kSliceKeys;
    }
    sb += ns;
    kb += gn[i];
  }
  __syncthreads();
  loc->g = s_loc[0];
  loc->id = s_loc[1];
  loc->first = s_loc[2];
  loc->end = s_loc[3];
  return true;
}

// The keys of this wave's part of the slice (kBatch sub-batches of 64; past
// the slice end they read its first key).
template <int kW>
__device__ __forceinline__ void load_slice_keys(const uint64_t *__restrict__ keys_in,
                                                const SliceLoc &L, int w, int lane,
                                                uint64_t (&key)[SliceShape<kW>::kBatch]) {
  constexpr int kB = SliceShape<kW>::kBatch;
  const int wb = L.first + w * 64 * kB;
#pragma unroll
  for (int j = 0; j < kB; ++j) {
    const int e = wb + 64 * j + lane;
    key[j] = keys_in[e < L.end ? e : L.first];
  }
}

template <int kW>
__global__ __launch_bounds__(64 * kW) void bucket_count_kernel(
    const uint64_t *__restrict__ keys_in, const int32_t *__restrict__ totals, int n_groups,
    int lbits, int32_t *__restrict__ slice_cnt) {
  constexpr int kT = SliceShape<kW>::kT, kB = SliceShape<kW>::kBatch;
  extern __shared__ int s_cnt[];  // [R]
  SliceLoc L;
  if (!find_slice<kW>(totals, n_groups, &L)) return;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int R = 1 << lbits;
  const unsigned mask = unsigned(R - 1);
  uint64_t key[kB];
  load_slice_keys<kW>(keys_in, L, w, lane, key);
  for (int d = tid; d < R; d += kT) s_cnt[d] = 0;
  __syncthreads();
  const int wb = L.first + w * 64 * kB;
#pragma unroll
  for (int j = 0; j < kB; ++j)
    if (wb + 64 * j < L.end)  // wave-uniform
      count_digit_runs(s_cnt, key_digit(key[j], 0, mask), wb + 64 * j + lane < L.end);
  __syncthreads();
  int32_t *out = slice_cnt + int64_t(L.id) * R;
  for (int d = tid; d < R; d += kT) out[d] = s_cnt[d];
}

__global__ __launch_bounds__(kThreads) void bucket_scan_kernel(
    const int32_t *__restrict__ totals, int n_groups, int64_t n_cells, int lbits,
    int32_t *__restrict__ slice_cnt, int32_t *__restrict__ cstart, int32_t *__restrict__ cend) {
  __shared__ int s_scan[kWaves];
  const int g = int(blockIdx.x);
  if (g >= n_groups) return;
  const int tid = threadIdx.x;
  const int R = 1 << lbits;
  // group start and first slice: sums over the groups before g
  int pk = 0, ps = 0;
  for (int d = tid; d < g; d += kThreads) {
    const int t = totals[d];
    pk += t;
    ps += slices_of(t);
  }
  int gs, sb;
  block_exclusive_scan(pk, s_scan, &gs);
  block_exclusive_scan(ps, s_scan, &sb);
  const int ns = slices_of(totals[g]);
  int32_t *sc = slice_cnt + int64_t(sb) * R;
  // thread t owns digits 4t .. 4t+3 (R is a multiple of 4, >= 32): the
  // group's totals per digit, then the digit starts
  constexpr int kU = 8;  // slices whose counts are loaded together
  const int d0 = 4 * tid;
  const bool mine = d0 < R;
  u32x4 tot = {0u, 0u, 0u, 0u};
  if (mine) {
    for (int k0 = 0; k0 < ns; k0 += kU) {
      u32x4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u)
        v[u] = k0 + u < ns ? *reinterpret_cast<const u32x4 *>(sc + int64_t(k0 + u) * R + d0)
                           : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int u = 0; u < kU; ++u) tot += v[u];
    }
  }
  int unused;
  int ex = gs + block_exclusive_scan(int(tot.x + tot.y + tot.z + tot.w), s_scan, &unused);
  if (!mine) return;
  // first sorted position of each of the four digits in slice 0
  u32x4 run;
  run.x = uint32_t(ex);
  run.y = run.x + tot.x;
  run.z = run.y + tot.y;
  run.w = run.z + tot.z;
  const int64_t cell0 = int64_t(g) * R + d0;
  const uint32_t t4[4] = {tot.x, tot.y, tot.z, tot.w};
  const uint32_t r4[4] = {run.x, run.y, run.z, run.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (cell0 + i < n_cells) {
      cstart[cell0 + i] = t4[i] ? int(r4[i]) : 0;
      cend[cell0 + i] = t4[i] ? int(r4[i] + t4[i]) : 0;
    }
  }
  for (int k0 = 0; k0 < ns; k0 += kU) {
    u32x4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      v[u] = k0 + u < ns ? *reinterpret_cast<const u32x4 *>(sc + int64_t(k0 + u) * R + d0)
                         : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (k0 + u < ns) *reinterpret_cast<u32x4 *>(sc + int64_t(k0 + u) * R + d0) = run;
      run += v[u];
    }
  }
}

template <int kW>
__global__ __launch_bounds__(64 * kW) void bucket_place_kernel(
    const uint64_t *__restrict__ keys_in, const int32_t *__restrict__ totals, int n_groups,
    int lbits, const int32_t *__restrict__ slice_cnt, uint64_t *__restrict__ keys_out) {
  constexpr int kT = SliceShape<kW>::kT, kB = SliceShape<kW>::kBatch;
  extern __shared__ int s_cnt[];  // [kW][R]
  SliceLoc L;
  if (!find_slice<kW>(totals, n_groups, &L)) return;
  const int tid = threadIdx.x, lane = lane_id(), w = tid >> 6;
  const int R = 1 << lbits;
  const unsigned mask = unsigned(R - 1);
  uint64_t key[kB];
  load_slice_keys<kW>(keys_in, L, w, lane, key);
  for (int d = tid; d < kW * R; d += kT) s_cnt[d] = 0;
  __syncthreads();
  int *cnt = s_cnt + w * R;
  const int wb = L.first + w * 64 * kB;
#pragma unroll
  for (int j = 0; j < kB; ++j)
    if (wb + 64 * j < L.end)
      count_digit_runs(cnt, key_digit(key[j], 0, mask), wb + 64 * j + lane < L.end);
  __syncthreads();
  // per-wave bases: the slice's first position of the digit + earlier waves
  const int32_t *base = slice_cnt + int64_t(L.id) * R;
  for (int d = tid; d < R; d += kT) {
    int run = base[d];
#pragma unroll
    for (int ww = 0; ww < kW; ++ww) {
      const int c = s_cnt[ww * R + d];
      s_cnt[ww * R + d] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kB; ++j) {
    if (wb + 64 * j >= L.end) break;
    const bool valid = wb + 64 * j + lane < L.end;
    const unsigned dg = key_digit(key[j], 0, mask);
    int below, same;
    digit_rank(dg, valid, below, same);
    if (valid) {
      const int pos = cnt[dg] + below;
      keys_out[pos] = key[j];
      if (below == 0) cnt[dg] = pos + same;
    }
  }
}

// bev_pool_legacy.py:56-61 boundary flags on the sorted ranks: writes the
// dense [start, end) of every occupied cell.  Thread t handles sorted
// positions 4t .. 4t+3 (two 16-byte loads when kVec: keys 16-byte aligned).
template <bool kVec>
__global__ __launch_bounds__(kThreads) void cell_ranges_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    int32_t *__restrict__ cstart, int32_t *__restrict__ cend) {
  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t i0 = (int64_t(blockIdx.x) * kThreads + threadIdx.x) * 4;
  if (i0 >= n) return;
  const uint32_t *kw = reinterpret_cast<const uint32_t *>(keys);  // rank = odd words
  int r[6];  // ranks of positions i0-1 .. i0+4 (-1 outside [0, n))
  r[0] = i0 > 0 ? int(kw[2 * (i0 - 1) + 1]) : -1;
  if (kVec && i0 + 3 < n) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(kw + 2 * i0);
    const u32x4 b = *reinterpret_cast<const u32x4 *>(kw + 2 * i0 + 4);
    r[1] = int(a.y);
    r[2] = int(a.w);
    r[3] = int(b.y);
    r[4] = int(b.w);
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) r[1 + u] = i0 + u < n ? int(kw[2 * (i0 + u) + 1]) : -1;
  }
  r[5] = i0 + 4 < n ? int(kw[2 * (i0 + 4) + 1]) : -1;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = i0 + u;
    if (i < n) {
      if (r[u] != r[u + 1]) cstart[r[u + 1]] = int(i);
      if (r[u + 2] != r[u + 1]) cend[r[u + 1]] = int(i + 1);
    }
  }
}

// Interval starts (r[i] != r[i-1]) per block of 256 sorted keys: wave ballot
// + popcount, summed over the block's waves.
__global__ __launch_bounds__(kThreads) void count_starts_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    int32_t *__restrict__ bcount) {
  __shared__ int s_w[kWaves];
  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  bool is_start = false;
  if (i < n) is_start = (i == 0) || key_rank(keys[i - 1]) != key_rank(keys[i]);
  const uint64_t b = __ballot(is_start);
  if (lane_id() == 0) s_w[threadIdx.x >> 6] = __popcll(b);
  __syncthreads();
  if (threadIdx.x == 0) {
    int s = 0;
    for (int j = 0; j < kWaves; ++j) s += s_w[j];
    bcount[blockIdx.x] = s;
  }
}

// Single-block exclusive scan of counts[0..n) in place; *total_out = sum.
__global__ __launch_bounds__(kThreads) void scan_counts_kernel(int32_t *__restrict__ counts,
                                                               int64_t n,
                                                               int32_t *__restrict__ total_out) {
  __shared__ int scratch[kWaves];
  int carry = 0;
  for (int64_t t0 = 0; t0 < n; t0 += kThreads * 4) {
    int v[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t j = t0 + threadIdx.x * 4 + i;
      v[i] = j < n ? counts[j] : 0;
      s += v[i];
    }
    int tot;
    int ex = block_exclusive_scan(s, scratch, &tot) + carry;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t j = t0 + threadIdx.x * 4 + i;
      if (j < n) counts[j] = ex;
      ex += v[i];
    }
    carry += tot;
  }
  if (threadIdx.x == 0) *total_out = carry;
}

// Compacted interval j (the j-th start in sorted order): starts[j], lengths[j]
// (= end - start, the legacy "difference of starts"), cells[j] = rank.
__global__ __launch_bounds__(kThreads) void interval_write_kernel(
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    const int32_t *__restrict__ cend, const int32_t *__restrict__ boff,
    int32_t *__restrict__ starts, int32_t *__restrict__ lengths, int32_t *__restrict__ cells) {
  __shared__ int s_w[kWaves];
  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int w = threadIdx.x >> 6;
  bool is_start = false;
  int r = 0;
  if (i < n) {
    r = key_rank(keys[i]);
    is_start = (i == 0) || key_rank(keys[i - 1]) != r;
  }
  const uint64_t b = __ballot(is_start);
  if (lane_id() == 0) s_w[w] = __popcll(b);
  __syncthreads();
  if (is_start) {
    int off = boff[blockIdx.x] + __popcll(b & lanes_below());
    for (int j = 0; j < w; ++j) off += s_w[j];
    starts[off] = int(i);
    lengths[off] = cend[r] - int(i);
    cells[off] = r;
  }
}

// ---------------------------------------------------------------------------
// forward kernels
// ---------------------------------------------------------------------------

// First sorted position >= i that starts a cell (n if none).
__device__ __forceinline__ int64_t snap_to_cell(int64_t i, int64_t n,
                                                const uint64_t *__restrict__ keys,
                                                const int32_t *__restrict__ cend) {
  if (i <= 0) return 0;
  if (i >= n) return n;
  const int r = key_rank(keys[i]);
  if (key_rank(keys[i - 1]) != r) return i;
  return cend[r];
}

// Block b owns the sorted positions [snap(b*P), snap((b+1)*P)): whole cells
// only, so every cell's sum is one sequential chain.  Rows (feats[point]) of
// R sorted points at a time are gathered into LDS by all threads; thread c
// then adds column c of the R rows in order into its fp32 accumulator and
// stores it to acc[cell*C + c] when the cell ends.
template <typename T>
__global__ __launch_bounds__(kThreads) void accum_rows_kernel(
    const typename T::raw *__restrict__ x, int64_t ld, int C, int CB, int R,
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    const int32_t *__restrict__ cend, float *__restrict__ acc, int64_t P) {
  extern __shared__ float smem[];
  float *buf = smem;                         // R * CB floats
  int *rk = reinterpret_cast<int *>(smem + R * CB);  // R + 1 ints
  const int tid = threadIdx.x;
  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t r0 = int64_t(blockIdx.x) * P;
  if (r0 >= n) return;
  const int64_t s = snap_to_cell(r0, n, keys, cend);
  const int64_t e = snap_to_cell(r0 + P < n ? r0 + P : n, n, keys, cend);
  if (s >= e) return;
  using raw = typename T::raw;
  for (int c0 = 0; c0 < C; c0 += CB) {
    const int cb = C - c0 < CB ? C - c0 : CB;
    float a = 0.0f;
    for (int64_t base = s; base < e; base += R) {
      const int rows = int(e - base < R ? e - base : R);
      __syncthreads();
      for (int j = tid; j <= rows; j += kThreads)
        rk[j] = (base + j < e) ? key_rank(keys[base + j]) : -1;
      for (int slot = tid; slot < rows * cb; slot += kThreads) {
        const int j = slot / cb, c = slot - j * cb;
        const int64_t idx = key_index(keys[base + j]);
        buf[slot] = T::load(reinterpret_cast<const raw *>(x) + idx * ld + c0 + c);
      }
      __syncthreads();
      if (tid < cb) {
        for (int j = 0; j < rows; ++j) {
          a += buf[j * cb + tid];
          const int r = rk[j];
          if (rk[j + 1] != r) {
            acc[int64_t(r) * C + c0 + tid] = a;
            a = 0.0f;
          }
        }
      }
    }
  }
}

// ---- software-pipelined forward accumulation (16-byte rows) ---------------
//
// Same ownership as accum_rows_kernel (block b owns the sorted positions
// [snap(b*P), snap((b+1)*P)), whole cells only), restructured so memory
// latency is hidden inside the block.  Roles:
//   * loader waves (1..4, 256 threads) gather the rows of each stage of
//     kStageRows sorted points with 16-byte loads (loader slot i of thread t
//     covers row (t + 256 i) / rowq, 16-byte column (t + 256 i) % rowq) into
//     a ring of kDepth register stages, and move the oldest arrived stage to
//     LDS once per step;
//   * wave 0 sums the stage in LDS, one channel per lane (channels l + 64 j),
//     each lane adding its column in row order into one fp32 accumulator; a
//     cell's sum is stored to acc when the next cell starts (start flags from
//     a ballot over the stage's ranks) or the range ends, so a cell spanning
//     stages keeps one sequential chain.
// Step k: wave 0 sums stage k from LDS buffer k&1 while the loaders issue the
// rows of stage k+kDepth and the point indices of stage k+2*kDepth, then store
// stage k+1 (issued kDepth-1 steps earlier) into buffer (k+1)&1; one barrier.
// The loaders issue loads only and always fetch a stage's indices kDepth steps
// before its rows, so every wait they need (indices of stage k+kDepth, rows of
// stage k+1) leaves all younger row loads in flight (vmcnt retires in issue
// order).  The summing wave issues no loads, so its stores never hold up a
// wait.  Loads of stages past the range end are pointed at the range's first
// row (a single line) so the code stays straight-line.
#ifndef BEVPOOL_STAGE_ROWS
#define BEVPOOL_STAGE_ROWS 32
#endif
#ifndef BEVPOOL_DEPTH
#define BEVPOOL_DEPTH 2
#endif
constexpr int kStageRows = BEVPOOL_STAGE_ROWS;  // sorted points per stage
constexpr int kDepth = BEVPOOL_DEPTH;           // row stages in flight per loader thread
#ifndef BEVPOOL_SUMMERS
#define BEVPOOL_SUMMERS 1
#endif
#ifndef BEVPOOL_LOADER_WAVES
#define BEVPOOL_LOADER_WAVES 2
#endif
constexpr int kSummers = BEVPOOL_SUMMERS;       // summing waves (waves 0..kSummers-1)
constexpr int kLoaders = 64 * BEVPOOL_LOADER_WAVES;  // loader threads (the other waves)
constexpr int kPipeThreads = 64 * kSummers + kLoaders;
// Only 32-row stages are built and tested.  A 64-row variant built with
// -DBEVPOOL_STAGE_ROWS=64 failed one camera-index parity case on MI355X and
// passed it on the next run, without a cause found; 16-row stages were only
// ever timed.  Other values are therefore refused at compile time.
static_assert(kStageRows == 32, "only 32-row accumulation stages are supported");

// native 16-byte vector (register-promotable, unlike the HIP uint4 wrapper)

// Where the accumulation's rows come from and how they are loaded:
//   kRowsPlain   feature rows, ordinary loads;
//   kRowsStream  feature rows, non-temporal loads: the rows are read once,
//                and keeping them out of the caches keeps the index (ranks,
//                keys) and the cell rows there for the transposes and the
//                backward gather.  Measured on MI355X at 1 x 360 x 360
//                (638 MB of feature rows): forward -3.5 us, backward -5 us per
//                step.  With 2.6-5.1 GB of rows (4 x 360 x 360, 2 x 720 x 720)
//                the accumulation itself got 4-6% slower and nothing else
//                faster, so inputs of more than kStreamRowBytes of rows keep
//                ordinary loads.
//   kRowsDepth   depth-weighted context rows (DepthRows), ordinary loads:
//                a context row is read for every depth bin.
constexpr int kRowsPlain = 0, kRowsDepth = 1, kRowsStream = 2;
constexpr int64_t kStreamRowBytes = int64_t(1) << 30;

struct PipeRange {
  int64_t s, e;  // sorted positions [s, e)
  int rowq;      // 16-byte slots per row of this channel block
  __device__ __forceinline__ int rows(int k) const {
    const int64_t b = s + int64_t(k) * kStageRows;
    return b >= e ? 0 : int(e - b < kStageRows ? e - b : kStageRows);
  }
};

// Register ring of one loader thread.
template <int kSlots>
struct LoaderRing {
  u32x4 d[kDepth][kSlots];       // gathered 16-byte pieces of a stage
  uint32_t idx[kDepth][kSlots];  // point indices of a later stage
  int rk[kDepth];                // rank of row (lt % kStageRows) of a stage
  uint32_t dpi[kDepth];          // depth-weighted rows: point index of that row
  float dp[kDepth];              //   and its depth weight
  int srow[kSlots];              // row of slot i within a stage (unclamped)
  int sq[kSlots];                // 16-byte column of slot i
};

// Rows of the depth-weighted forward (fused depth x context pooling): the row
// of point p = (bn*D + d)*HW + hw is context row pix = bn*HW + hw, weighted by
// depth[p] (the reference materialises depth[p] * context[pix, c],
// models/vtransforms/depth_lss.py:91-94).
struct DepthRows {
  const float *depth;  // (BN, D, HW) contiguous: depth[p]
  FastDiv hw, nd;      // HW and D
  // p = (bn*D + d)*HW + hw -> bn*HW + hw, with e = p / HW = bn*D + d
  __device__ __forceinline__ uint32_t pix(uint32_t p) const {
    const uint32_t e = hw.div(p);
    return nd.div(e) * hw.d + (p - e * hw.d);
  }
};

// Point indices of stage k into ring slot j.  Slots past the stage's rows
// repeat its last row; a stage past the range end reads the range's first row.
template <int kSlots, int j, int kRows>
__device__ __forceinline__ void ring_index(LoaderRing<kSlots> &R, int lt,
                                           const uint32_t *__restrict__ kw, const PipeRange &pr,
                                           int k) {
  constexpr bool kMul = kRows == kRowsDepth;
  const int rows = pr.rows(k);
  const int64_t base = pr.s + int64_t(k) * kStageRows;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const int r = R.srow[i] < rows - 1 ? R.srow[i] : rows - 1;
    R.idx[j][i] = kw[2 * (rows > 0 ? base + r : pr.s)];  // low word: point index
  }
  if constexpr (kMul) {
    int64_t p = base + (lt & (kStageRows - 1));
    p = base >= pr.e ? pr.s : (p < pr.e ? p : pr.e - 1);
    R.dpi[j] = kw[2 * p];
  }
}

// Rows of stage k into ring slot j (its indices are in R.idx[j]), plus the rank
// of row lt % kStageRows.
template <int kSlots, int j, int kRows>
__device__ __forceinline__ void ring_rows(LoaderRing<kSlots> &R, int lt,
                                          const uint32_t *__restrict__ kw,
                                          const char *__restrict__ xb, int64_t ld_bytes,
                                          int col_bytes, const PipeRange &pr, int k,
                                          const DepthRows &dr) {
  constexpr bool kMul = kRows == kRowsDepth;
  const bool live = pr.rows(k) > 0;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const int q = live ? R.sq[i] : 0;
    const uint32_t row = kMul ? dr.pix(R.idx[j][i]) : R.idx[j][i];
    const u32x4 *src =
        reinterpret_cast<const u32x4 *>(xb + int64_t(row) * ld_bytes + col_bytes + q * 16);
    if constexpr (kRows == kRowsStream)
      R.d[j][i] = __builtin_nontemporal_load(src);
    else
      R.d[j][i] = *src;
  }
  const int64_t b = pr.s + int64_t(k) * kStageRows;
  int64_t p = b + (lt & (kStageRows - 1));
  p = b >= pr.e ? pr.s : (p < pr.e ? p : pr.e - 1);
  R.rk[j] = kw[2 * p + 1];  // high word: rank
  if constexpr (kMul) R.dp[j] = dr.depth[R.dpi[j]];
}

// Ring slot j (stage k) into an LDS buffer.
template <int kSlots, int j, int kRows>
__device__ __forceinline__ void ring_store(const LoaderRing<kSlots> &R, int lt,
                                           const PipeRange &pr, int k, u32x4 *__restrict__ lbuf,
                                           int *__restrict__ lrk) {
  constexpr bool kMul = kRows == kRowsDepth;
  const int rows = pr.rows(k);
  const int n = rows * pr.rowq;
  if constexpr (kMul) {
    // slot i of this thread holds a piece of row srow[i]; lane r of every
    // loader wave holds the depth weight of row r (ring_index / ring_rows):
    // all lanes shuffle it in before any store is masked off, then scale the
    // piece (one fp32 product per element, as the reference's product)
    u32x4 v[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int r = R.srow[i] < kStageRows - 1 ? R.srow[i] : kStageRows - 1;
      const float w = __shfl(R.dp[j], r, 64);
      // __uint_as_float takes the element by value: hipcc 7.2's
      // __builtin_bit_cast of a vector element (v.y) reads element 0
      const float x0 = __uint_as_float(R.d[j][i].x) * w;
      const float x1 = __uint_as_float(R.d[j][i].y) * w;
      const float x2 = __uint_as_float(R.d[j][i].z) * w;
      const float x3 = __uint_as_float(R.d[j][i].w) * w;
      v[i] = u32x4{__float_as_uint(x0), __float_as_uint(x1), __float_as_uint(x2),
                   __float_as_uint(x3)};
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int slot = lt + kLoaders * i;
      if (slot < n) lbuf[slot] = v[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int slot = lt + kLoaders * i;
      if (slot < n) lbuf[slot] = R.d[j][i];
    }
  }
  if (lt < kStageRows) lrk[lt] = R.rk[j];
}

// One loader step k with ring slot r = k % kDepth (a template constant).
template <int kSlots, int r, int kRows>
__device__ __forceinline__ void loader_step(LoaderRing<kSlots> &R, int lt,
                                            const uint32_t *__restrict__ kw,
                                            const char *__restrict__ xb, int64_t ld_bytes,
                                            int col_bytes, const PipeRange &pr, int k, int nst,
                                            u32x4 *__restrict__ buf0, u32x4 *__restrict__ buf1,
                                            int *__restrict__ rk0s, int *__restrict__ rk1s,
                                            const DepthRows &dr) {
  ring_rows<kSlots, r, kRows>(R, lt, kw, xb, ld_bytes, col_bytes, pr, k + kDepth, dr);
  ring_index<kSlots, r, kRows>(R, lt, kw, pr, k + 2 * kDepth);
  if (k + 1 < nst) {
    if ((k + 1) & 1)
      ring_store<kSlots, (r + 1) % kDepth, kRows>(R, lt, pr, k + 1, buf1, rk1s);
    else
      ring_store<kSlots, (r + 1) % kDepth, kRows>(R, lt, pr, k + 1, buf0, rk0s);
  }
  __syncthreads();
}

// Sequential per-channel sums of one stage by one summing wave: lane l owns
// channels c0 + l + 64 i (i < kCPL, c0 the wave's first channel).  Rows are
// read from LDS 16 at a time before they are added (one LDS latency per 16
// dependent adds).  A 16-row chunk without a cell start is 16 straight adds;
// a chunk with exactly one start at row b jumps (16-way switch) to
// straight-line code for that b: add rows [0, b), store the finished cell,
// restart from +0.0, add rows [b, 16); other chunks go row by row.
// A finished cell row is stored in the output's element type: fp32 for fp32
// input; for 16-bit input the fp32 sum rounded once (T::to_raw), the value
// the output gets, so the transpose that follows moves half the bytes.
// With 16-bit input a lane owns channel pairs instead (pair l + 64 i =
// channels 2(l + 64 i), +1): one 4-byte LDS read per row and one packed
// 4-byte store per finished cell; kCPL then counts pairs per lane.
template <typename T, int kCPL>
struct RowSum {
  using TO = typename std::conditional<sizeof(typename T::raw) == 2, typename T::raw, float>::type;
  static constexpr bool kPair = sizeof(typename T::raw) == 2;
  static constexpr int kA = kPair ? 2 * kCPL : kCPL;  // fp32 accumulators per lane
  float a[kA];
  int cur = -1;    // rank of the current cell
  int carry = -1;  // rank of the previous stage's last row

  __device__ __forceinline__ void flush(int nch, TO *__restrict__ out, int64_t row_elems) {
    if (cur >= 0) {
      TO *o = out + int64_t(cur) * row_elems;
      const int lane = lane_id();
      if constexpr (kPair) {
        uint32_t *o32 = reinterpret_cast<uint32_t *>(o);  // row and channel offsets even
#pragma unroll
        for (int i = 0; i < kCPL; ++i)
          if (2 * (lane + 64 * i) < nch)
            o32[lane + 64 * i] =
                uint32_t(T::to_raw(a[2 * i])) | (uint32_t(T::to_raw(a[2 * i + 1])) << 16);
      } else {
#pragma unroll
        for (int i = 0; i < kCPL; ++i)
          if (lane + 64 * i < nch) o[lane + 64 * i] = a[i];
      }
    }
  }

  template <int kB, int kStart>
  __device__ __forceinline__ void split_chunk(const float (&v)[kB][kA], int rkl, int j0, int nch,
                                              TO *__restrict__ out, int64_t row_elems) {
#pragma unroll
    for (int u = 0; u < kStart; ++u)
#pragma unroll
      for (int i = 0; i < kA; ++i) a[i] += v[u][i];
    flush(nch, out, row_elems);
#pragma unroll
    for (int i = 0; i < kA; ++i) a[i] = 0.0f;
    cur = __builtin_amdgcn_readlane(rkl, j0 + kStart);
#pragma unroll
    for (int u = kStart; u < kB; ++u)
#pragma unroll
      for (int i = 0; i < kA; ++i) a[i] += v[u][i];
  }

  // lb: the stage's rows in LDS (row stride cb elements), col: this lane's
  // columns; nch: channels of this wave (stores of lanes past nch are skipped).
  __device__ __forceinline__ void add_stage(const typename T::raw *__restrict__ lb,
                                            const int *__restrict__ lrk, int rows, int cb,
                                            const int (&col)[kCPL], int nch,
                                            TO *__restrict__ out, int64_t row_elems) {
    const int lane = lane_id();
    const int rkl = lane < rows ? lrk[lane] : -1;
    int prev = __shfl_up(rkl, 1, 64);
    if (lane == 0) prev = carry;
    const uint64_t starts = __ballot(lane < rows && rkl != prev);
    if (rows > 0) carry = __builtin_amdgcn_readlane(rkl, rows - 1);
    constexpr int kB = kStageRows < 16 ? kStageRows : 16;
    for (int j0 = 0; j0 < rows; j0 += kB) {
      float v[kB][kA];
      if constexpr (kPair) {  // col[i]: pair index; cb even
        const uint32_t *lb32 = reinterpret_cast<const uint32_t *>(lb);
#pragma unroll
        for (int u = 0; u < kB; ++u)
#pragma unroll
          for (int i = 0; i < kCPL; ++i) {
            const uint32_t w = lb32[(j0 + u) * (cb >> 1) + col[i]];
            v[u][2 * i] = T::from_raw(w & 0xffffu);
            v[u][2 * i + 1] = T::from_raw(w >> 16);
          }
      } else {
#pragma unroll
        for (int u = 0; u < kB; ++u)
#pragma unroll
          for (int i = 0; i < kCPL; ++i) v[u][i] = T::load(lb + (j0 + u) * cb + col[i]);
      }
      const uint32_t chunk = uint32_t(starts >> j0) & uint32_t((uint64_t(1) << kB) - 1);
      const bool full = j0 + kB <= rows;
      if (full && chunk == 0) {
#pragma unroll
        for (int u = 0; u < kB; ++u)
#pragma unroll
          for (int i = 0; i < kA; ++i) a[i] += v[u][i];
      } else if (full && (chunk & (chunk - 1)) == 0) {
        switch (__builtin_ctz(chunk)) {
#define BEVPOOL_SPLIT(B)                                                                       \
  case B:                                                                                     \
    if constexpr ((B) < kB) split_chunk<kB, ((B) < kB ? (B) : 0)>(v, rkl, j0, nch, out, row_elems); \
    break;
          BEVPOOL_SPLIT(0) BEVPOOL_SPLIT(1) BEVPOOL_SPLIT(2) BEVPOOL_SPLIT(3)
          BEVPOOL_SPLIT(4) BEVPOOL_SPLIT(5) BEVPOOL_SPLIT(6) BEVPOOL_SPLIT(7)
          BEVPOOL_SPLIT(8) BEVPOOL_SPLIT(9) BEVPOOL_SPLIT(10) BEVPOOL_SPLIT(11)
          BEVPOOL_SPLIT(12) BEVPOOL_SPLIT(13) BEVPOOL_SPLIT(14) BEVPOOL_SPLIT(15)
#undef BEVPOOL_SPLIT
          default:
            break;
        }
      } else {
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const int j = j0 + u;
          if (j < rows) {
            if ((chunk >> u) & 1) {
              flush(nch, out, row_elems);
#pragma unroll
              for (int i = 0; i < kA; ++i) a[i] = 0.0f;
              cur = __builtin_amdgcn_readlane(rkl, j);
            }
#pragma unroll
            for (int i = 0; i < kA; ++i) a[i] += v[u][i];
          }
        }
      }
    }
  }
};

// kMul: depth-weighted rows (DepthRows): xb holds the context rows and row
// p's values are depth[p] * ctx[pix(p)].
template <typename T, int kSlots, int kCPL, int kRows>
__global__ __launch_bounds__(kPipeThreads) void accum_pipe_kernel(
    const char *__restrict__ xb, int64_t ld_bytes, int C, int CB,
    const uint64_t *__restrict__ keys, const int32_t *__restrict__ meta,
    const int32_t *__restrict__ cend, float *__restrict__ acc, int64_t P, DepthRows dr) {
  using raw = typename T::raw;
  extern __shared__ u32x4 smem4[];
  const int rowq_max = CB * int(sizeof(raw)) / 16;
  u32x4 *buf0 = smem4;
  u32x4 *buf1 = smem4 + kStageRows * rowq_max;
  int *rk0s = reinterpret_cast<int *>(smem4 + 2 * kStageRows * rowq_max);
  int *rk1s = rk0s + kStageRows;
  const uint32_t *kw = reinterpret_cast<const uint32_t *>(keys);

  const int64_t n = meta[BEVPOOL_META_N_KEPT];
  const int64_t r0 = int64_t(blockIdx.x) * P;
  if (r0 >= n) return;
  PipeRange pr;
  pr.s = snap_to_cell(r0, n, keys, cend);
  pr.e = snap_to_cell(r0 + P < n ? r0 + P : n, n, keys, cend);
  if (pr.s >= pr.e) return;
  const int nst = int((pr.e - pr.s + kStageRows - 1) / kStageRows);
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const bool summer = wave < kSummers;
  const int lt = int(threadIdx.x) - 64 * kSummers;  // loader thread index (loader waves only)

  for (int c0 = 0; c0 < C; c0 += CB) {
    const int cb = C - c0 < CB ? C - c0 : CB;
    pr.rowq = cb * int(sizeof(raw)) / 16;
    if (summer) {
      // summing wave `wave` owns channels [wch, wch + nch) of the block
      // (an even count with 16-bit input, whose lanes take channel pairs)
      constexpr bool kPair = RowSum<T, kCPL>::kPair;
      int cps = (cb + kSummers - 1) / kSummers;
      if (kPair) cps += cps & 1;
      const int wch = wave * cps;
      const int nch = cb - wch < cps ? (cb - wch > 0 ? cb - wch : 0) : cps;
      int col[kCPL];
#pragma unroll
      for (int i = 0; i < kCPL; ++i) {
        const int c = lane_id() + 64 * i;
        if (kPair) {  // pair index within the stage row
          const int np = nch >> 1;
          const int pc = (wch >> 1) + (c < np ? c : (np > 0 ? np - 1 : 0));
          col[i] = pc < (cb >> 1) ? pc : (cb >> 1) - 1;
        } else {
          const int cc = wch + (c < nch ? c : (nch > 0 ? nch - 1 : 0));
          col[i] = cc < cb ? cc : cb - 1;  // idle lanes read a valid column
        }
      }
      using TO = typename RowSum<T, kCPL>::TO;  // 16-bit rows for 16-bit input
      TO *out = reinterpret_cast<TO *>(acc) + c0 + wch;
      RowSum<T, kCPL> st;
      __syncthreads();  // stage 0 is in buffer 0
      for (int k = 0; k < nst; k += kDepth) {  // barriers match the loaders'
#pragma unroll
        for (int r = 0; r < kDepth; ++r) {
          const int kk = k + r;
          st.add_stage(reinterpret_cast<const raw *>((kk & 1) ? buf1 : buf0),
                       (kk & 1) ? rk1s : rk0s, pr.rows(kk), cb, col, nch, out, C);
          __syncthreads();
        }
      }
      st.flush(nch, out, C);
    } else {
      const int col_bytes = c0 * int(sizeof(raw));
      LoaderRing<kSlots> R;
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const int slot = lt + kLoaders * i;
        R.srow[i] = slot / pr.rowq;
        R.sq[i] = slot - R.srow[i] * pr.rowq;
      }
      // prologue: indices of stages 0..D-1, rows of 0..D-1 each followed by the
      // indices of stage j+D; then stage 0 into LDS
#define BEVPOOL_RING_PRO(J)                                                                    \
  if constexpr ((J) < kDepth) ring_index<kSlots, (J), kRows>(R, lt, kw, pr, (J));
      BEVPOOL_RING_PRO(0) BEVPOOL_RING_PRO(1) BEVPOOL_RING_PRO(2) BEVPOOL_RING_PRO(3)
      BEVPOOL_RING_PRO(4) BEVPOOL_RING_PRO(5) BEVPOOL_RING_PRO(6) BEVPOOL_RING_PRO(7)
#undef BEVPOOL_RING_PRO
#define BEVPOOL_RING_PRO(J)                                                                    \
  if constexpr ((J) < kDepth) {                                                               \
    ring_rows<kSlots, (J), kRows>(R, lt, kw, xb, ld_bytes, col_bytes, pr, (J), dr);            \
    ring_index<kSlots, (J), kRows>(R, lt, kw, pr, (J) + kDepth);                               \
  }
      BEVPOOL_RING_PRO(0) BEVPOOL_RING_PRO(1) BEVPOOL_RING_PRO(2) BEVPOOL_RING_PRO(3)
      BEVPOOL_RING_PRO(4) BEVPOOL_RING_PRO(5) BEVPOOL_RING_PRO(6) BEVPOOL_RING_PRO(7)
#undef BEVPOOL_RING_PRO
      ring_store<kSlots, 0, kRows>(R, lt, pr, 0, buf0, rk0s);
      __syncthreads();
      for (int k = 0; k < nst; k += kDepth) {
#define BEVPOOL_RING_STEP(J)                                                                   \
  if constexpr ((J) < kDepth)                                                                 \
    loader_step<kSlots, (J), kRows>(R, lt, kw, xb, ld_bytes, col_bytes, pr, k + (J), nst, buf0, \
                                   buf1, rk0s, rk1s, dr);
        BEVPOOL_RING_STEP(0) BEVPOOL_RING_STEP(1) BEVPOOL_RING_STEP(2) BEVPOOL_RING_STEP(3)
        BEVPOOL_RING_STEP(4) BEVPOOL_RING_STEP(5) BEVPOOL_RING_STEP(6) BEVPOOL_RING_STEP(7)
#undef BEVPOOL_RING_STEP
      }
    }
  }
}

// ---------------------------------------------------------------------------
// transposes between cell-major rows and the channel-first BEV
// ---------------------------------------------------------------------------
// A tile is 64 consecutive cells (ranks); rows are staged in LDS as
// [cell][channel] with a pitch of CT + 1 elements, CT = channels per pass.
// On the channel-first side each thread moves 4 consecutive cells of one
// channel: one 16-byte (fp32) or 8-byte (16-bit) access when kVecBev (n_xy,
// the b/z/c strides and the base are multiples of 4 elements, so 4 cells
// starting at a multiple of 4 share a (b, z) plane and are contiguous), else
// one access per cell.  On the row side kVecRow moves 16-byte pieces of a row
// (C * element size a multiple of 16).

// Offset of cell `cell` (< 2^31) in a channel-first (b, c, z, xy) tensor
// without the channel term.
__device__ __forceinline__ int64_t cell_offset(uint32_t cell, uint32_t n_z, uint32_t n_xy,
                                               int64_t sb, int64_t sz) {
  const uint32_t per_b = n_z * n_xy;
  const uint32_t b = cell / per_b, rem = cell - b * per_b;
  const uint32_t z = rem / n_xy, xy = rem - z * n_xy;
  return int64_t(b) * sb + int64_t(z) * sz + int64_t(xy);
}

// Per-tile cell table in LDS: occupied flag and channel-first offset (-1 past
// the last cell).  Returns whether any cell of the tile is occupied.
__device__ __forceinline__ bool load_tile_cells(int64_t cell0, int64_t n_cells,
                                                const int32_t *__restrict__ cstart,
                                                const int32_t *__restrict__ cend, int n_z,
                                                int64_t n_xy, int64_t sb, int64_t sz, int *occ,
                                                int64_t *off) {
  const int tid = threadIdx.x;
  int mine = 0;
  if (tid < kCellTile) {
    const int64_t cell = cell0 + tid;
    if (cell < n_cells) {
      mine = cend[cell] > cstart[cell] ? 1 : 0;
      off[tid] = cell_offset(uint32_t(cell), uint32_t(n_z), uint32_t(n_xy), sb, sz);
    } else {
      off[tid] = -1;
    }
    occ[tid] = mine;
  }
  return __syncthreads_or(mine) != 0;
}

// acc rows (cell-major fp32, written for occupied cells only) -> out
// (channel-first, dtype T); empty cells are written as 0.  The tile holds the
// raw fp32 bits, and a staged 16-byte piece is never converted lane by lane
// to float (hipcc 7.2 with packed fp32 ops disabled folded bit casts of lanes
// y/z/w of such a vector into lane x).  With kVecRow each wave first reads
// the tile's 64 cell ends as a ballot mask, then loads every row piece of the
// occupied cells up front (kTileSlots per thread, clamped in-bounds
// addresses), so a block pays two memory latencies before its stores and
// reads no row of an empty cell (measured on MI355X: 53 -> 43 us at B = 4,
// 360 x 360, unchanged at B = 1).  Occupancy: cell_end != 0 (cell ranges are
// zeroed before the sort writes the occupied ones).
constexpr int kTileSlots = kCellTile * (kTileChannels / 4) / kThreads;  // 8
// bev_to_rows on grids of at least this many cells reads the occupancy of a
// thread's 4 cells before its gradient loads (one more memory latency per
// block, no loads for 4 empty cells); smaller grids issue every load up
// front.  Measured on MI355X: 3-10% faster from 518,400 cells (B = 4 at
// 360 x 360) up, slower at 129,600.  The same per-thread scheme for
// rows_to_bev was slower (it uses the wave-wide mask above instead).
constexpr int64_t kOccFirstCells = 200000;

// Optional copy of the meta counters into memory the host reads (pinned host
// memory through its device address), made by a kernel that runs anyway.
// One thread writes the counters as system-scope stores and then sets the
// done flag dst[BEVPOOL_META_LEN] with a system-scope release store, so a
// host that sees the flag sees the counters (the release orders the
// thread's earlier stores before the flag; no event is involved).
struct MetaReport {
  const int32_t *meta = nullptr;
  int32_t *dst = nullptr;
};

__device__ __forceinline__ void store_meta_report(const int32_t *__restrict__ meta,
                                                  int32_t *__restrict__ dst) {
  if (threadIdx.x == 0) {
    int32_t v[BEVPOOL_META_LEN];
#pragma unroll
    for (int i = 0; i < BEVPOOL_META_LEN; ++i) v[i] = meta[i];
#pragma unroll
    for (int i = 0; i < BEVPOOL_META_LEN; ++i)
      __hip_atomic_store(dst + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(dst + BEVPOOL_META_LEN, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

__device__ __forceinline__ void write_meta_report(const MetaReport &rep) {
  if (rep.dst && blockIdx.x == 0) store_meta_report(rep.meta, rep.dst);
}

// bevpool_meta_report: the counters and the done flag, one block of 64 (its
// first thread does the work).
__global__ void meta_report_kernel(const int32_t *__restrict__ meta, int32_t *__restrict__ dst) {
  store_meta_report(meta, dst);
}

// kRaw16: the cell rows already hold the output's 16-bit values (the
// pipelined accumulation stores them rounded once), moved without conversion;
// otherwise they are fp32 sums converted on the way out.
template <typename T, bool kVecRow, bool kVecBev, bool kRaw16 = false>
__global__ __launch_bounds__(kThreads) void rows_to_bev_kernel(
    const float *__restrict__ acc, int C, int CT, const int32_t *__restrict__ cstart,
    const int32_t *__restrict__ cend, int64_t n_cells, int n_z, int64_t n_xy, int64_t sb,
    int64_t sc, int64_t sz, typename T::raw *__restrict__ out, MetaReport report) {
  using raw = typename T::raw;
  static_assert(!kRaw16 || sizeof(raw) == 2, "16-bit rows for 16-bit output only");
  write_meta_report(report);
  extern __shared__ uint32_t tile_bits[];  // kCellTile * (CT + 1)
  __shared__ int occ[kCellTile];
  __shared__ int64_t off[kCellTile];
  (void)cstart;
  const int tid = threadIdx.x;
  const int64_t cell0 = int64_t(blockIdx.x) * kCellTile;
  const uint32_t *accb = reinterpret_cast<const uint32_t *>(acc);
  const int pitch = CT + 1;
  // occupancy of the tile's 64 cells as a mask in every wave (lane j loads
  // cell j's end), so that only occupied cells' rows are loaded: one more
  // dependent load, and no row bytes for empty cells (most cells of the
  // sparser grids); wave 0's mask also gives each cell's own flag, so the
  // ends are loaded once
  uint64_t occm = 0;
  if (kVecRow) {
    const int64_t cj = cell0 + lane_id();
    occm = __ballot(cj < n_cells && cend[cj] != 0);
  }
  int occ_mine = 0;
  int64_t off_mine = -1;
  if (tid < kCellTile && cell0 + tid < n_cells) {
    occ_mine = kVecRow ? int((occm >> tid) & 1u) : (cend[cell0 + tid] != 0 ? 1 : 0);
    off_mine = cell_offset(uint32_t(cell0 + tid), uint32_t(n_z), uint32_t(n_xy), sb, sz);
  }
  if (!kVecRow) {
    if (tid < kCellTile) {
      occ[tid] = occ_mine;
      off[tid] = off_mine;
    }
    __syncthreads();
  }
  const uint16_t *acch = reinterpret_cast<const uint16_t *>(acc);
  for (int c0 = 0; c0 < C; c0 += CT) {
    const int cb = C - c0 < CT ? C - c0 : CT;
    if (kVecRow) {
      constexpr uint32_t kPer = kRaw16 ? 8 : 4;  // channels per 16-byte piece
      const uint32_t q = uint32_t(cb) / kPer;    // 16-byte pieces per row
      const uint32_t n_items = kCellTile * q;
      u32x4 v[kTileSlots];
#pragma unroll
      for (int it = 0; it < kTileSlots; ++it) {
        const uint32_t i = tid + it * kThreads;
        uint32_t t = i / q, k = i - t * q;
        if (i >= n_items || cell0 + t >= n_cells) t = k = 0;
        const void *src = kRaw16
                              ? static_cast<const void *>(acch + (cell0 + t) * C + c0 + kPer * k)
                              : static_cast<const void *>(accb + (cell0 + t) * C + c0 + kPer * k);
        v[it] = ((occm >> t) & 1) ? *reinterpret_cast<const u32x4 *>(src)
                                  : u32x4{0u, 0u, 0u, 0u};
      }
      if (c0 == 0 && tid < kCellTile) {
        occ[tid] = occ_mine;
        off[tid] = off_mine;
      }
#pragma unroll
      for (int it = 0; it < kTileSlots; ++it) {
        const uint32_t i = tid + it * kThreads;
        if (i < n_items) {
          const uint32_t t = i / q, k = i - t * q;
          uint32_t *d = tile_bits + t * pitch + kPer * k;
          if constexpr (kRaw16) {  // 8 values, low half first
            d[0] = v[it].x & 0xffffu;
            d[1] = v[it].x >> 16;
            d[2] = v[it].y & 0xffffu;
            d[3] = v[it].y >> 16;
            d[4] = v[it].z & 0xffffu;
            d[5] = v[it].z >> 16;
            d[6] = v[it].w & 0xffffu;
            d[7] = v[it].w >> 16;
          } else {
            d[0] = v[it].x;
            d[1] = v[it].y;
            d[2] = v[it].z;
            d[3] = v[it].w;
          }
        }
      }
    } else {
      for (uint32_t i = tid; i < uint32_t(kCellTile * cb); i += kThreads) {
        const uint32_t t = i / uint32_t(cb), c = i - t * uint32_t(cb);
        if (occ[t])
          tile_bits[t * pitch + c] = kRaw16 ? uint32_t(acch[(cell0 + t) * C + c0 + c])
                                            : accb[(cell0 + t) * C + c0 + c];
      }
    }
    __syncthreads();
    for (int i = tid; i < cb * (kCellTile / 4); i += kThreads) {
      const int c = i >> 4, j = (i & 15) * 4;
      raw r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t b = occ[j + u] ? tile_bits[(j + u) * pitch + c] : 0u;
        if constexpr (kRaw16)
          r[u] = raw(b);
        else
          r[u] = T::to_raw(__builtin_bit_cast(float, b));
      }
      if (kVecBev) {
        if (off[j] < 0) continue;
        raw *dst = out + off[j] + int64_t(c0 + c) * sc;
        if constexpr (sizeof(raw) == 4) {
          u32x4 w;
          w.x = r[0];
          w.y = r[1];
          w.z = r[2];
          w.w = r[3];
          __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(dst));
        } else {
          u32x2 w;
          w.x = uint32_t(r[0]) | (uint32_t(r[1]) << 16);
          w.y = uint32_t(r[2]) | (uint32_t(r[3]) << 16);
          __builtin_nontemporal_store(w, reinterpret_cast<u32x2 *>(dst));
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (off[j + u] >= 0) out[off[j + u] + int64_t(c0 + c) * sc] = r[u];
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// backward kernels
// ---------------------------------------------------------------------------

// grad (channel-first, any b/c/z strides, xy contiguous) -> cell-major rows of
// the occupied cells (raw bits copied).  With kVecBev each thread always
// handles the same 4 cells (j = 4 * (tid % 16)) of channels tid / 16 + 16 it;
// all its tile loads are issued up front (clamped in-bounds addresses,
// empty cells included) together with the occupancy loads, or, with
// occ_first, after reading its 4 cells' occupancy (none when all 4 are
// empty).
template <typename TR, bool kVecRow, bool kVecBev>
__global__ __launch_bounds__(kThreads) void bev_to_rows_kernel(
    const TR *__restrict__ grad, int C, int CT, const int32_t *__restrict__ cstart,
    const int32_t *__restrict__ cend, int64_t n_cells, int n_z, int64_t n_xy, int64_t sb,
    int64_t sc, int64_t sz, bool occ_first, TR *__restrict__ rows) {
  extern __shared__ u32x4 smem_b2r[];
  TR *tile = reinterpret_cast<TR *>(smem_b2r);  // kCellTile * (CT + 1)
  __shared__ int occ[kCellTile];
  __shared__ int64_t off[kCellTile];
  const int tid = threadIdx.x;
  const int64_t cell0 = int64_t(blockIdx.x) * kCellTile;
  const int pitch = CT + 1;
  constexpr int kPer = 16 / int(sizeof(TR));  // elements per 16-byte row piece
  if (kVecBev) {
    (void)cstart;
    const int j = (tid & 15) * 4;
    const bool live = cell0 + j < n_cells;  // then all 4 cells are (n_cells % 4 == 0)
    const int64_t offj =
        cell_offset(uint32_t(live ? cell0 + j : cell0), uint32_t(n_z), uint32_t(n_xy), sb, sz);
    // sparse grids: the 4 cells' occupancy first, no gradient loads when all are empty
    bool need = true;
    if (occ_first) {
      need = false;
      if (live)
#pragma unroll
        for (int u = 0; u < 4; ++u) need |= cend[cell0 + j + u] != 0;
    }
    for (int c0 = 0; c0 < C; c0 += CT) {
      const int cb = C - c0 < CT ? C - c0 : CT;
      using V = typename std::conditional<sizeof(TR) == 4, u32x4, u32x2>::type;
      V v[kTileSlots];
#pragma unroll
      for (int it = 0; it < kTileSlots; ++it) {
        int c = (tid >> 4) + 16 * it;
        c = c < cb ? c : 0;
        v[it] = need ? *reinterpret_cast<const V *>(grad + offj + int64_t(c0 + c) * sc) : V{};
      }
      // the cells' occupancy, loaded after the gradient loads so that one
      // round trip brings both
      if (c0 == 0 && tid < kCellTile)
        occ[tid] = cell0 + tid < n_cells && cend[cell0 + tid] != 0 ? 1 : 0;
#pragma unroll
      for (int it = 0; it < kTileSlots; ++it) {
        const int c = (tid >> 4) + 16 * it;
        if (c < cb) {
          TR e[4];
          if constexpr (sizeof(TR) == 4) {
            e[0] = v[it].x;
            e[1] = v[it].y;
            e[2] = v[it].z;
            e[3] = v[it].w;
          } else {
            e[0] = TR(v[it].x);
            e[1] = TR(v[it].x >> 16);
            e[2] = TR(v[it].y);
            e[3] = TR(v[it].y >> 16);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) tile[(j + u) * pitch + c] = e[u];
        }
      }
      __syncthreads();
      if (kVecRow) {
        const uint32_t q = uint32_t(cb) / kPer;  // 16-byte pieces per row
        for (uint32_t i = tid; i < kCellTile * q; i += kThreads) {
          const uint32_t t = i / q, k = i - t * q;
          if (!occ[t]) continue;
          const TR *srow = tile + t * pitch + kPer * k;
          u32x4 w;
          if constexpr (sizeof(TR) == 4) {
            w.x = srow[0];
            w.y = srow[1];
            w.z = srow[2];
            w.w = srow[3];
          } else {
            w.x = uint32_t(srow[0]) | (uint32_t(srow[1]) << 16);
            w.y = uint32_t(srow[2]) | (uint32_t(srow[3]) << 16);
            w.z = uint32_t(srow[4]) | (uint32_t(srow[5]) << 16);
            w.w = uint32_t(srow[6]) | (uint32_t(srow[7]) << 16);
          }
          *reinterpret_cast<u32x4 *>(rows + (cell0 + t) * C + c0 + kPer * k) = w;
        }
      } else {
        for (uint32_t i = tid; i < uint32_t(kCellTile * cb); i += kThreads) {
          const uint32_t t = i / uint32_t(cb), c = i - t * uint32_t(cb);
          if (occ[t]) rows[(cell0 + t) * C + c0 + c] = tile[t * pitch + c];
        }
      }
      __syncthreads();
    }
    return;
  }
  // general strides: per-cell loads after the occupancy test
  if (!load_tile_cells(cell0, n_cells, cstart, cend, n_z, n_xy, sb, sz, occ, off)) return;
  for (int c0 = 0; c0 < C; c0 += CT) {
    const int cb = C - c0 < CT ? C - c0 : CT;
    for (int i = tid; i < cb * (kCellTile / 4); i += kThreads) {
      const int c = i >> 4, j = (i & 15) * 4;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        tile[(j + u) * pitch + c] = occ[j + u] ? grad[off[j + u] + int64_t(c0 + c) * sc] : TR(0);
    }
    __syncthreads();
    if (kVecRow) {
      const uint32_t q = uint32_t(cb) / kPer;
      for (uint32_t i = tid; i < kCellTile * q; i += kThreads) {
        const uint32_t t = i / q, k = i - t * q;
        if (!occ[t]) continue;
        const TR *srow = tile + t * pitch + kPer * k;
        u32x4 w;
        if constexpr (sizeof(TR) == 4) {
          w.x = srow[0];
          w.y = srow[1];
          w.z = srow[2];
          w.w = srow[3];
        } else {
          w.x = uint32_t(srow[0]) | (uint32_t(srow[1]) << 16);
          w.y = uint32_t(srow[2]) | (uint32_t(srow[3]) << 16);
          w.z = uint32_t(srow[4]) | (uint32_t(srow[5]) << 16);
          w.w = uint32_t(srow[6]) | (uint32_t(srow[7]) << 16);
        }
        *reinterpret_cast<u32x4 *>(rows + (cell0 + t) * C + c0 + kPer * k) = w;
      }
    } else {
      for (uint32_t i = tid; i < uint32_t(kCellTile * cb); i += kThreads) {
        const uint32_t t = i / uint32_t(cb), c = i - t * uint32_t(cb);
        if (occ[t]) rows[(cell0 + t) * C + c0 + c] = tile[t * pitch + c];
      }
    }
    __syncthreads();
  }
}

// Cache warm-up for gather_rows_kernel (its leading blocks).  Each gather piece is a dependent
// chain rank -> row -> store; with the rank array and the gradient rows
// fetched from HBM while the gather's write stream saturates it, the chains
// take about twice as long (measured 92 us vs 155-185 us at the det shape).
// Rows written by bev_to_rows_kernel are not reliably kept by the caches, rows
// that were read are, so this kernel reads both once:
//   * blocks [0, 8 * per_xcd): block wb runs on XCD wb % 8 and reads a share
//     of the ranks that XCD's gather blocks will need (the gather walks
//     XCD-contiguous eighths of its pieces, xcd_span pieces each), so they are
//     in that XCD's L2;
//   * the other blocks read the rows of the occupied cells of kWarmCells
//     consecutive cells each (16-byte pieces).
// Nothing is written: the only store is guarded by `never`, a launch argument
// that is always 0, which keeps the loads from being optimised away.
#ifndef BEVPOOL_WARM_CELLS
#define BEVPOOL_WARM_CELLS 512
#endif
constexpr int kWarmCells = BEVPOOL_WARM_CELLS;  // cells per row-warming block
constexpr int kWarmBatch = 8;                   // loads in flight per thread

struct GatherWarm {
  const u32x4 *rank16;   // rank array as 16-byte pieces (null: skip)
  int64_t n16;           // whole pieces in the array
  int64_t xcd_span;      // gather pieces (vectors of xg) per XCD
  int vpr;               // gather pieces per point
  int per_xcd;           // rank blocks per XCD
  const u32x4 *rows16;   // gradient rows as 16-byte pieces (null: skip)
  int rowq;              // 16-byte pieces per row
};

// Warm-up work of block wb (< warm_blocks(w, tiles)); returns nothing, reads only.
__device__ __forceinline__ void gather_warm_block(const GatherWarm &w, int wb, int64_t n_points,
                                                  const int32_t *__restrict__ cstart,
                                                  const int32_t *__restrict__ cend,
                                                  int64_t n_cells, int never,
                                                  uint32_t *__restrict__ sink) {
  __shared__ int occ[kWarmCells];
  const int rank_blocks = w.rank16 ? kXcds * w.per_xcd : 0;
  uint32_t m = 0;
  if (wb < rank_blocks) {
    const int x = wb % kXcds, j = wb / kXcds;
    // points [p0, p1) are gathered by XCD x; their ranks are pieces [q0, q1)
    const int64_t p0 = int64_t(x) * w.xcd_span / w.vpr;
    int64_t p1 = (int64_t(x + 1) * w.xcd_span + w.vpr - 1) / w.vpr;
    p1 = p1 < n_points ? p1 : n_points;
    const int64_t q0 = p0 / 4;
    int64_t q1 = (p1 + 3) / 4;
    q1 = q1 < w.n16 ? q1 : w.n16;
    const int64_t share = (q1 - q0 + w.per_xcd - 1) / w.per_xcd;
    const int64_t b0 = q0 + int64_t(j) * share;
    int64_t b1 = b0 + share;
    b1 = b1 < q1 ? b1 : q1;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kThreads) {
      const u32x4 v = w.rank16[i];
      m ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  } else if (w.rows16) {
    // kWarmCells consecutive cells per block: occupancy, then the occupied
    // rows' pieces, kWarmBatch loads in flight per thread
    const int64_t cell0 = int64_t(wb - rank_blocks) * kWarmCells;
    for (int t = threadIdx.x; t < kWarmCells; t += kThreads) {
      const int64_t cell = cell0 + t;
      occ[t] = (cell < n_cells && cend[cell] > cstart[cell]) ? 1 : 0;
    }
    __syncthreads();
    const uint32_t q = uint32_t(w.rowq);
    const uint32_t n = kWarmCells * q;
    for (uint32_t i0 = threadIdx.x; i0 < n; i0 += kThreads * kWarmBatch) {
      u32x4 v[kWarmBatch];
#pragma unroll
      for (int b = 0; b < kWarmBatch; ++b) {
        const uint32_t i = i0 + uint32_t(b) * kThreads < n ? i0 + uint32_t(b) * kThreads : n - 1;
        const uint32_t t = i / q, k = i - t * q;
        v[b] = occ[t] ? w.rows16[(cell0 + t) * q + k] : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int b = 0; b < kWarmBatch; ++b) m ^= v[b].x ^ v[b].y ^ v[b].z ^ v[b].w;
    }
  }
  if (never) sink[threadIdx.x] = m;
}

// x_grad[p, :] = rows[rank[p], :] (kept) or 0 (dropped); point order, so the
// writes stream.  V is a 16-byte vector when rows allow it, else one element.
// Each thread copies kGatherPer vectors spaced kThreads apart (coalesced),
// blocks walk XCD-contiguous chunks (an XCD's points map to a compact set of
// cells, whose rows then stay in its L2), and the destination is written
// with non-temporal stores (it is not read again here, and keeping it out of
// L2 leaves room for the gradient rows).  Each piece is a dependent chain
// rank -> row -> store, so the leading warm_blocks blocks first pull the ranks
// and the rows into the caches (gather_warm_block).  kNarrow: indices fit in 32
// bits.
#ifndef BEVPOOL_GATHER_PER
#define BEVPOOL_GATHER_PER 1
#endif
#ifndef BEVPOOL_GATHER_NT
#define BEVPOOL_GATHER_NT 1
#endif
constexpr int kGatherPer = BEVPOOL_GATHER_PER;

template <typename V, bool kNarrow>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const V *__restrict__ rows, int vpr, const int32_t *__restrict__ rank, int64_t n_points,
    V *__restrict__ xg, int64_t xg_ld, int warm_blocks, GatherWarm w,
    const int32_t *__restrict__ cstart, const int32_t *__restrict__ cend, int64_t n_cells,
    int never, int zero_dropped) {
  // the first warm_blocks blocks (a multiple of 8, so XCD parity is kept)
  // only pull ranks and rows into the caches ahead of the others
  if (int(blockIdx.x) < warm_blocks) {
    gather_warm_block(w, int(blockIdx.x), n_points, cstart, cend, n_cells, never,
                      reinterpret_cast<uint32_t *>(xg));
    return;
  }
  const int64_t total = n_points * vpr;
  const int64_t gb = int64_t(blockIdx.x) - warm_blocks;
  const int64_t base =
      xcd_chunk(gb, int64_t(gridDim.x) - warm_blocks) * (kThreads * kGatherPer) + threadIdx.x;
#pragma unroll
  for (int j = 0; j < kGatherPer; ++j) {
    const int64_t i = base + j * kThreads;
    if (i < total) {
      int64_t p;
      int q;
      if (kNarrow) {
        const uint32_t ui = uint32_t(i), up = ui / uint32_t(vpr);
        p = up;
        q = int(ui - up * uint32_t(vpr));
      } else {
        p = i / vpr;
        q = int(i - p * vpr);
      }
      const int r = rank[p];
      V v = V{};
      if (r >= 0) v = rows[int64_t(r) * vpr + q];
      else if (!zero_dropped) continue;  // the caller keeps dropped rows as they are
#if BEVPOOL_GATHER_NT
      __builtin_nontemporal_store(v, xg + p * xg_ld + q);
#else
      xg[p * xg_ld + q] = v;
#endif
    }
  }
}

// ---------------------------------------------------------------------------
// legacy native interface (caller-provided intervals)
// ---------------------------------------------------------------------------

// Zero bytes [0, n16 * 16) as 16-byte vectors plus a 4-byte tail (n4 words
// from `tail`), grid-stride.  A kernel rather than a memset so that a graph
// capture records no memset node.
__global__ __launch_bounds__(kThreads) void zero_fill_kernel(u32x4 *__restrict__ p, int64_t n16,
                                                             uint32_t *__restrict__ tail,
                                                             int64_t n4) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n16; i += stride)
    p[i] = u32x4{0u, 0u, 0u, 0u};
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride) tail[i] = 0u;
}

// Validates interval j and returns its cell ((b*D + z)*H + x)*W + y from the
// coordinates of its first row, geom[s] = (x, y, z, b) (the cell of
// ops/bev_pool/csrc/bev_pool_cuda.cu:33-35), or -1 when its rows [s, s+len)
// or its cell lie outside the arrays (the reference reads and writes out of
// bounds there).
__device__ __forceinline__ int64_t legacy_cell(const int32_t *__restrict__ geom, int64_t n,
                                               int64_t s, int64_t len, int nb, int nd, int nh,
                                               int nw) {
  if (s < 0 || len < 0 || s >= n || s + len > n) return -1;
  const int gx = geom[4 * s], gy = geom[4 * s + 1], gz = geom[4 * s + 2], gb = geom[4 * s + 3];
  if (gx < 0 || gx >= nh || gy < 0 || gy >= nw || gz < 0 || gz >= nd || gb < 0 || gb >= nb)
    return -1;
  return ((int64_t(gb) * nd + gz) * nh + gx) * nw + gy;
}

// Interval count: the caller's host count, or min(capacity, device count).
__device__ __forceinline__ int64_t legacy_count(int64_t cap, const int32_t *__restrict__ dev) {
  if (!dev) return cap;
  const int64_t c = *dev;
  return c < cap ? (c > 0 ? c : 0) : cap;
}

// ops/bev_pool/csrc/bev_pool_cuda.cu:20-42: interval j sums rows [s, s + len)
// of x (n, C) -- fp32 from +0.0, rows in order -- and stores the sum to
// out[cell, :] (channels last).  One wave per interval; lane l owns channels
// c0 + l + 64 i, so each row is read as one coalesced run; rows are loaded
// kLegacyBatch at a time before they are added.  Invalid intervals are
// skipped and counted in meta[BEVPOOL_META_N_BAD] (meta may be null).
constexpr int kLegacyBatch = 8;

template <int kCPL>
__global__ __launch_bounds__(kThreads) void legacy_forward_kernel(
    const float *__restrict__ x, int64_t n, int C, const int32_t *__restrict__ geom,
    const int32_t *__restrict__ starts, const int32_t *__restrict__ lengths, int64_t cap,
    const int32_t *__restrict__ count_dev, int nb, int nd, int nh, int nw,
    float *__restrict__ out, int32_t *__restrict__ meta) {
  const int64_t n_int = legacy_count(cap, count_dev);
  const int lane = lane_id();
  const int64_t nwaves = (int64_t(gridDim.x) * kThreads) >> 6;
  for (int64_t j = (int64_t(blockIdx.x) * kThreads + threadIdx.x) >> 6; j < n_int; j += nwaves) {
    const int64_t s = starts[j], len = lengths[j];
    const int64_t cell = legacy_cell(geom, n, s, len, nb, nd, nh, nw);
    if (cell < 0) {
      if (meta && lane == 0) atomicAdd(meta + BEVPOOL_META_N_BAD, 1);
      continue;
    }
    for (int c0 = 0; c0 < C; c0 += 64 * kCPL) {
      int col[kCPL];
      float acc[kCPL];
#pragma unroll
      for (int i = 0; i < kCPL; ++i) {
        const int c = c0 + lane + 64 * i;
        col[i] = c < C ? c : C - 1;  // lanes past C read a valid column, store nothing
        acc[i] = 0.0f;
      }
      for (int64_t r0 = 0; r0 < len; r0 += kLegacyBatch) {
        float v[kLegacyBatch][kCPL];
#pragma unroll
        for (int u = 0; u < kLegacyBatch; ++u) {
          const int64_t r = s + (r0 + u < len ? r0 + u : 0);
#pragma unroll
          for (int i = 0; i < kCPL; ++i) v[u][i] = x[r * C + col[i]];
        }
#pragma unroll
        for (int u = 0; u < kLegacyBatch; ++u)
          if (r0 + u < len)
#pragma unroll
            for (int i = 0; i < kCPL; ++i) acc[i] += v[u][i];
      }
#pragma unroll
      for (int i = 0; i < kCPL; ++i)
        if (c0 + lane + 64 * i < C) out[cell * C + c0 + lane + 64 * i] = acc[i];
    }
  }
}

// ops/bev_pool/csrc/bev_pool_cuda.cu:61-84: every row of interval j gets the
// gradient row of its cell, x_grad[r, :] = g[cell, :] (g channels last).  One
// wave per interval, lanes over channels as in the forward.
template <int kCPL>
__global__ __launch_bounds__(kThreads) void legacy_backward_kernel(
    const float *__restrict__ g, int64_t n, int C, const int32_t *__restrict__ geom,
    const int32_t *__restrict__ starts, const int32_t *__restrict__ lengths, int64_t cap,
    const int32_t *__restrict__ count_dev, int nb, int nd, int nh, int nw,
    float *__restrict__ xg, int32_t *__restrict__ meta) {
  const int64_t n_int = legacy_count(cap, count_dev);
  const int lane = lane_id();
  const int64_t nwaves = (int64_t(gridDim.x) * kThreads) >> 6;
  for (int64_t j = (int64_t(blockIdx.x) * kThreads + threadIdx.x) >> 6; j < n_int; j += nwaves) {
    const int64_t s = starts[j], len = lengths[j];
    const int64_t cell = legacy_cell(geom, n, s, len, nb, nd, nh, nw);
    if (cell < 0) {
      if (meta && lane == 0) atomicAdd(meta + BEVPOOL_META_N_BAD, 1);
      continue;
    }
    for (int c0 = 0; c0 < C; c0 += 64 * kCPL) {
      float v[kCPL];
#pragma unroll
      for (int i = 0; i < kCPL; ++i) {
        const int c = c0 + lane + 64 * i;
        v[i] = g[cell * C + (c < C ? c : C - 1)];
      }
      for (int64_t r = s; r < s + len; ++r)
#pragma unroll
        for (int i = 0; i < kCPL; ++i)
          if (c0 + lane + 64 * i < C) xg[r * C + c0 + lane + 64 * i] = v[i];
    }
  }
}

// Run boundaries of a rank array (ops/bev_pool/bev_pool_legacy.py:56-61:
// flag[0] = 1, flag[i] = rank[i] != rank[i-1]).  Per block of 256 positions:
// the number of run starts.
template <typename TR>
__global__ __launch_bounds__(kThreads) void run_count_kernel(const TR *__restrict__ ranks,
                                                             int64_t n,
                                                             int32_t *__restrict__ bcount) {
  __shared__ int s_w[kWaves];
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const bool is_start = i < n && (i == 0 || ranks[i] != ranks[i - 1]);
  const uint64_t b = __ballot(is_start);
  if (lane_id() == 0) s_w[threadIdx.x >> 6] = __popcll(b);
  __syncthreads();
  if (threadIdx.x == 0) {
    int s = 0;
    for (int j = 0; j < kWaves; ++j) s += s_w[j];
    bcount[blockIdx.x] = s;
  }
}

// Run starts in order, at the block offsets scanned from run_count_kernel.
template <typename TR>
__global__ __launch_bounds__(kThreads) void run_write_kernel(const TR *__restrict__ ranks,
                                                             int64_t n,
                                                             const int32_t *__restrict__ boff,
                                                             int32_t *__restrict__ starts) {
  __shared__ int s_w[kWaves];
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int w = threadIdx.x >> 6;
  const bool is_start = i < n && (i == 0 || ranks[i] != ranks[i - 1]);
  const uint64_t b = __ballot(is_start);
  if (lane_id() == 0) s_w[w] = __popcll(b);
  __syncthreads();
  if (is_start) {
    int off = boff[blockIdx.x] + __popcll(b & lanes_below());
    for (int j = 0; j < w; ++j) off += s_w[j];
    starts[off] = int(i);
  }
}

// lengths[j] = starts[j + 1] - starts[j], the last one n - starts[j]
// (bev_pool_legacy.py:58-61), for the count(meta) runs.
__global__ __launch_bounds__(kThreads) void run_length_kernel(const int32_t *__restrict__ starts,
                                                              int64_t n,
                                                              const int32_t *__restrict__ count,
                                                              int32_t *__restrict__ lengths) {
  const int64_t m = *count;
  const int64_t j = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (j < m) lengths[j] = int((j + 1 < m ? int64_t(starts[j + 1]) : n) - starts[j]);
}

// ---------------------------------------------------------------------------
// depth-weighted (fused depth x context) pooling helpers
// ---------------------------------------------------------------------------

// ---- planar (channel-first) <-> rows ---------------------------------------
//
// A planar tensor (BN, C, S) has element (bn, c, s) at bn*sbn + c*sc + s (s
// contiguous): the depth-net context (S = fH*fW) and channel-first camera
// features (S = D*fH*fW, the storage behind the reference's rearrange view,
// depth_lss.py:94).  Point p = bn*S + s.

// planar -> rows (BN*S, C), fp32.  Tiled form (C <= 128, C, S, sbn, sc
// multiples of 4, 16-byte aligned bases): planar_tile_kernel.  Vector form
// (wider rows): a block covers 256 consecutive s of one bn; thread
// (wave w, lane l) owns points s0 + [0, 4) and walks the channels in 4x4
// blocks c0 + [0, 4) (c0 = 4 (l >> 4) + 16 i): four 16-byte loads along s (16
// lanes of a channel read 256 contiguous bytes), a register transpose, four
// 16-byte row stores (4 lanes write 64 contiguous bytes of a row; the wave
// completes its 64 rows within one pass over the channels).  Non-temporal
// stores: the rows are read back by a random gather, not from cache.  No LDS,
// no barrier.  Scalar form: one element per thread.
#ifndef BEVPOOL_PLANAR_NT
#define BEVPOOL_PLANAR_NT 1
#endif

__device__ __forceinline__ void store16(u32x4 *p, u32x4 v) {
#if BEVPOOL_PLANAR_NT
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// Tiled planar -> rows: a block moves kPlanarTile consecutive s of one bn,
// all C channels, through an LDS tile [s][C + 1] (<= 66 KB at C = 128).  Each
// group of kPlanarTile / 4 lanes loads kPlanarTile * 4 contiguous bytes of one
// channel (kPer 16-byte loads per thread, all issued before the tile is
// written); after one barrier the block writes its rows as one contiguous run
// of kPlanarTile * C floats, 16 bytes per thread, consecutive threads at
// consecutive addresses (non-temporal).  Measured at det (1.28 GB): 64-point
// tiles 248 us against 288 us for the register transpose, whose row stores
// scatter 16-byte pieces over 16 rows; 128-point tiles (512-byte runs per
// channel) a further -6 us on the channel-first forward.
#ifndef BEVPOOL_PLANAR_TS
#define BEVPOOL_PLANAR_TS 128
#endif
constexpr int kPlanarTile = BEVPOOL_PLANAR_TS;  // points per tile (64 or 128)
template <int kPer>
__global__ __launch_bounds__(kThreads) void planar_tile_kernel(
    const float *__restrict__ src, int C, int64_t S, int64_t tiles_s, int64_t sbn, int64_t sc,
    float *__restrict__ rows) {
  constexpr int kQ = kPlanarTile / 4;  // 16-byte pieces per channel of a tile
  extern __shared__ float tile[];  // [kPlanarTile][C + 1]
  const int pitch = C + 1, tid = threadIdx.x;
  const int64_t bn = int64_t(blockIdx.x) / tiles_s;
  const int64_t s0 = (int64_t(blockIdx.x) - bn * tiles_s) * kPlanarTile;
  const int np = S - s0 < kPlanarTile ? int(S - s0) : kPlanarTile;  // a multiple of 4
  const float *in = src + bn * sbn + s0;
  const int npc = C * kQ;  // 16-byte pieces on the channel side
  u32x4 v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    // piece e: channel e / 16, points 4 (e % 16) + [0, 4); pieces past the
    // tile reload an in-bounds one and are not written
    const int e = tid + kThreads * i;
    const int c = e / kQ, pq = e % kQ;
    const int cc = c < C ? c : C - 1, pp = 4 * pq < np ? pq : 0;
    v[i] = *reinterpret_cast<const u32x4 *>(in + int64_t(cc) * sc + 4 * pp);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + kThreads * i;
    const int c = e / kQ, pq = e % kQ;
    if (e < npc && 4 * pq < np) {
      float *t = tile + (4 * pq) * pitch + c;
      t[0] = __uint_as_float(v[i].x);
      t[pitch] = __uint_as_float(v[i].y);
      t[2 * pitch] = __uint_as_float(v[i].z);
      t[3 * pitch] = __uint_as_float(v[i].w);
    }
  }
  __syncthreads();
  const int q = C >> 2, nrp = np * q;
  u32x4 *out = reinterpret_cast<u32x4 *>(rows + (bn * S + s0) * C);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = tid + kThreads * i;  // row e / q, 16-byte column e % q
    if (e < nrp) {
      const int p = e / q, j = e - p * q;
      const float *t = tile + p * pitch + 4 * j;
      store16(out + e, u32x4{__float_as_uint(t[0]), __float_as_uint(t[1]), __float_as_uint(t[2]),
                             __float_as_uint(t[3])});
    }
  }
}

template <bool kVec, int kIt>
__global__ __launch_bounds__(kThreads) void planar_rows_kernel(
    const float *__restrict__ src, int C, int64_t S, int64_t tiles_s, int64_t n_rows,
    int64_t sbn, int64_t sc, float *__restrict__ rows) {
  if constexpr (kVec) {
    const int64_t bn = int64_t(blockIdx.x) / tiles_s;
    const int64_t ts = int64_t(blockIdx.x) - bn * tiles_s;
    const int lane = lane_id(), w = threadIdx.x >> 6;
    const int64_t s0 = ts * 256 + w * 64 + (lane & 15) * 4;
    if (s0 >= S) return;
    const float *in = src + bn * sbn + s0;
    u32x4 *out = reinterpret_cast<u32x4 *>(rows + (bn * S + s0) * C);
    const int q = C / 4;  // 16-byte pieces per row
    // all channels of these rows, 16 at a time (kIt passes with every load
    // issued before the first store), so each row is completed by this wave
    // within a few instructions
    for (int cb = (lane >> 4) * 4; cb < C; cb += 16 * kIt) {
      u32x4 a[kIt][4];
#pragma unroll
      for (int i = 0; i < kIt; ++i) {
        const int c0 = cb + 16 * i < C ? cb + 16 * i : cb;  // past C: reload (not stored)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          a[i][k] = *reinterpret_cast<const u32x4 *>(in + int64_t(c0 + k) * sc);
      }
#pragma unroll
      for (int i = 0; i < kIt; ++i) {
        if (cb + 16 * i < C) {
          u32x4 *o = out + (cb + 16 * i) / 4;
          store16(o, u32x4{a[i][0].x, a[i][1].x, a[i][2].x, a[i][3].x});
          store16(o + q, u32x4{a[i][0].y, a[i][1].y, a[i][2].y, a[i][3].y});
          store16(o + 2 * q, u32x4{a[i][0].z, a[i][1].z, a[i][2].z, a[i][3].z});
          store16(o + 3 * q, u32x4{a[i][0].w, a[i][1].w, a[i][2].w, a[i][3].w});
        }
      }
    }
  } else {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n_rows * C) return;
    const int64_t r = i / C;
    const int c = int(i - r * C);
    const int64_t bn = r / S, sp = r - bn * S;
    rows[i] = src[bn * sbn + int64_t(c) * sc + sp];
  }
}

// Backward of the op-level pooling into a planar gradient:
// x_grad[bn, c, s] = g[rank[bn*S + s], c] (0 for dropped points), g the
// cell-major rows of bev_to_rows_kernel.  Vector form (C, S, sbn, sc multiples
// of 4, 16-byte aligned x_grad): a thread takes 4 consecutive points and walks
// the channels 4 at a time: four 16-byte row loads (cache-resident rows), a
// register transpose, four 16-byte stores along s (a wave writes 1 KB
// contiguous per channel, non-temporal).  Blocks map XCD-contiguously.
template <bool kVec, int kIt>
__global__ __launch_bounds__(kThreads) void gather_planar_kernel(
    const float *__restrict__ g, int C, const int32_t *__restrict__ rank, int64_t n_points,
    int64_t S, int64_t sbn, int64_t sc, float *__restrict__ x_grad) {
  if constexpr (kVec) {
    const int64_t groups = n_points / 4;  // S % 4 == 0: a group never spans two bn
    const int64_t gi = xcd_chunk(blockIdx.x, gridDim.x) * kThreads + threadIdx.x;
    if (gi >= groups) return;
    const int64_t p0 = gi * 4;
    const u32x4 rk = *reinterpret_cast<const u32x4 *>(rank + p0);
    const int r0 = int(rk.x), r1 = int(rk.y), r2 = int(rk.z), r3 = int(rk.w);
    const u32x4 *g0 = reinterpret_cast<const u32x4 *>(g + int64_t(r0 >= 0 ? r0 : 0) * C);
    const u32x4 *g1 = reinterpret_cast<const u32x4 *>(g + int64_t(r1 >= 0 ? r1 : 0) * C);
    const u32x4 *g2 = reinterpret_cast<const u32x4 *>(g + int64_t(r2 >= 0 ? r2 : 0) * C);
    const u32x4 *g3 = reinterpret_cast<const u32x4 *>(g + int64_t(r3 >= 0 ? r3 : 0) * C);
    const uint32_t m0 = r0 >= 0 ? 0xFFFFFFFFu : 0u, m1 = r1 >= 0 ? 0xFFFFFFFFu : 0u;
    const uint32_t m2 = r2 >= 0 ? 0xFFFFFFFFu : 0u, m3 = r3 >= 0 ? 0xFFFFFFFFu : 0u;
    const int64_t bn = p0 / S, sp = p0 - bn * S;
    float *out = x_grad + bn * sbn + sp;
    const int nq = C / 4;
    for (int qb = 0; qb < nq; qb += kIt) {
      u32x4 a[kIt][4];
#pragma unroll
      for (int i = 0; i < kIt; ++i) {  // every row piece of kIt groups, then the stores
        const int q = qb + i < nq ? qb + i : qb;
        a[i][0] = g0[q] & m0;
        a[i][1] = g1[q] & m1;
        a[i][2] = g2[q] & m2;
        a[i][3] = g3[q] & m3;
      }
#pragma unroll
      for (int i = 0; i < kIt; ++i) {
        if (qb + i < nq) {
          float *o = out + int64_t(4 * (qb + i)) * sc;
          __builtin_nontemporal_store(u32x4{a[i][0].x, a[i][1].x, a[i][2].x, a[i][3].x},
                                      reinterpret_cast<u32x4 *>(o));
          __builtin_nontemporal_store(u32x4{a[i][0].y, a[i][1].y, a[i][2].y, a[i][3].y},
                                      reinterpret_cast<u32x4 *>(o + sc));
          __builtin_nontemporal_store(u32x4{a[i][0].z, a[i][1].z, a[i][2].z, a[i][3].z},
                                      reinterpret_cast<u32x4 *>(o + 2 * sc));
          __builtin_nontemporal_store(u32x4{a[i][0].w, a[i][1].w, a[i][2].w, a[i][3].w},
                                      reinterpret_cast<u32x4 *>(o + 3 * sc));
        }
      }
    }
  } else {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n_points * C) return;
    const int c = int(i / n_points);
    const int64_t p = i - int64_t(c) * n_points;
    const int r = rank[p];
    const int64_t bn = p / S, sp = p - bn * S;
    x_grad[bn * sbn + int64_t(c) * sc + sp] = r >= 0 ? g[int64_t(r) * C + c] : 0.0f;
  }
}

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15) in a fixed order:
// xor 1, xor 2 (quad permutes), then the half-row and row mirrors.  Each
// step adds two equal-order partial sums, so every lane of the row ends with
// the same value.
__device__ __forceinline__ float row_sum16(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x140, 0xF, 0xF, false));
  return v;
}

constexpr int kDgPix = 16;  // pixels per depth_grad block (4 per wave)

// Backward of out[cell] = sum_{p in cell} depth[p] * ctx[pix(p)] (the
// reference's autograd through depth_lss.py:91-94 and the pooling):
//   grad_depth[p]        = sum_c g[rank[p], c] * ctx[pix(p), c]  (0 if dropped)
//   grad_ctx[bn, c, hw]  = sum_d g[rank[p_d], c] * depth[p_d]
// with p_d = (bn*D + d)*HW + hw.
// A block takes kDgPix consecutive pixels.  Their ranks and depths are staged
// in LDS ([d][pixel], read coalesced over the pixels); each wave then takes
// kDgPix/4 pixels one after another, its four 16-lane rows taking the depth
// bins d = 4 i + row, lane j of a row the channels j + 16 k (k < kK).  Per bin
// a row gathers its cell's gradient row, reduces the dot product with
// row_sum16 and adds depth * row to its context sums; the four rows' context
// sums are combined in row order at the end of the pixel.  The dot products
// replace the ranks in LDS and, like the context sums, are written out
// coalesced.  g: cell-major fp32 rows of the occupied cells; ctx:
// channel-last rows (planar_rows_kernel).  Blocks map XCD-contiguously, so
// the cells of neighbouring pixels' rays meet in one L2.
template <int kK, int kU>
__global__ __launch_bounds__(kThreads) void depth_grad_kernel(
    const float *__restrict__ g, int C, const int32_t *__restrict__ rank,
    const float *__restrict__ depth, const float *__restrict__ ctx, int D, int64_t HW,
    int64_t n_pix, uint32_t *__restrict__ grad_depth, float *__restrict__ grad_ctx,
    int64_t gsbn, int64_t gsc) {
  extern __shared__ int dg_smem[];
  int *lr = dg_smem;                                             // [D][kDgPix]
  float *ldp = reinterpret_cast<float *>(dg_smem + D * kDgPix);  // [D][kDgPix]
  float *lgc = ldp + D * kDgPix;                                 // [C][kDgPix]
  const int tid = threadIdx.x;
  const int64_t pix0 = xcd_chunk(blockIdx.x, gridDim.x) * kDgPix;
  if (pix0 >= n_pix) return;  // XCD padding blocks
  const int npx = n_pix - pix0 < kDgPix ? int(n_pix - pix0) : kDgPix;
  for (int i = tid; i < D * kDgPix; i += kThreads) {
    const int d = i / kDgPix, t = i - d * kDgPix;
    int r = -1;
    float dv = 0.0f;
    if (t < npx) {
      const int64_t pix = pix0 + t;
      const int64_t bn = pix / HW, hw = pix - bn * HW;
      const int64_t p = (bn * D + d) * HW + hw;
      r = rank[p];
      dv = depth[p];
    }
    lr[i] = r;
    ldp[i] = dv;
  }
  __syncthreads();
  const int lane = lane_id();
  const int row = lane >> 4, j = lane & 15;
  const int wave = tid >> 6;
  int col[kK];
  bool cv[kK];
#pragma unroll
  for (int k = 0; k < kK; ++k) {
    const int c = j + 16 * k;
    cv[k] = c < C;
    col[k] = cv[k] ? c : C - 1;
  }
  const int nrow = (D + 3) >> 2;  // bins per row
  constexpr int kPerWave = kDgPix / kWaves;
  for (int q = 0; q < kPerWave; ++q) {
    const int t = wave * kPerWave + q;
    if (t >= npx) break;  // wave-uniform
    const int64_t pix = pix0 + t;
    float xc[kK], gc[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      const float v = ctx[pix * C + col[k]];
      xc[k] = cv[k] ? v : 0.0f;
      gc[k] = 0.0f;
    }
    for (int i0 = 0; i0 < nrow; i0 += kU) {
      int rr[kU];
      float dp[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int d = 4 * (i0 + u) + row;
        const int dc = d < D ? d : D - 1;
        const int r = lr[dc * kDgPix + t];
        const float w = ldp[dc * kDgPix + t];
        rr[u] = d < D ? r : -1;
        dp[u] = d < D ? w : 0.0f;
      }
      // every load is issued (clamped rows/columns) and masked by a bitwise
      // AND afterwards: a select would let the compiler sink each load into
      // a branch of its own and wait for it there
      const uint32_t *gb = reinterpret_cast<const uint32_t *>(g);
      float gv[kU][kK];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t base = int64_t(rr[u] >= 0 ? rr[u] : 0) * C;
#pragma unroll
        for (int k = 0; k < kK; ++k) {
          const uint32_t m = (rr[u] >= 0 && cv[k]) ? 0xFFFFFFFFu : 0u;
          gv[u][k] = __builtin_bit_cast(float, gb[base + col[k]] & m);
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < kK; ++k) part += gv[u][k] * xc[k];
        const float dot = row_sum16(part);
        const int d = 4 * (i0 + u) + row;
        if (j == 0 && d < D) lr[d * kDgPix + t] = __builtin_bit_cast(int, rr[u] >= 0 ? dot : 0.0f);
#pragma unroll
        for (int k = 0; k < kK; ++k) gc[k] += gv[u][k] * dp[u];
      }
    }
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      const float s0 = __shfl(gc[k], j, 64);
      const float s1 = __shfl(gc[k], j + 16, 64);
      const float s2 = __shfl(gc[k], j + 32, 64);
      const float s3 = __shfl(gc[k], j + 48, 64);
      const float tot = ((s0 + s1) + s2) + s3;
      if (row == 0 && cv[k]) lgc[(j + 16 * k) * kDgPix + t] = tot;
    }
  }
  __syncthreads();
  for (int i = tid; i < D * kDgPix; i += kThreads) {
    const int d = i / kDgPix, t = i - d * kDgPix;
    if (t < npx) {
      const int64_t pix = pix0 + t;
      const int64_t bn = pix / HW, hw = pix - bn * HW;
      grad_depth[(bn * D + d) * HW + hw] = uint32_t(lr[i]);
    }
  }
  for (int i = tid; i < C * kDgPix; i += kThreads) {
    const int c = i / kDgPix, t = i - c * kDgPix;
    if (t < npx) {
      const int64_t pix = pix0 + t;
      const int64_t bn = pix / HW, hw = pix - bn * HW;
      grad_ctx[bn * gsbn + int64_t(c) * gsc + hw] = lgc[i];
    }
  }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// LSD passes of at most kMaxDigitBits bits each; or, for ranks of 11..20
// bits (local_bits > 0), one global pass by the high digit (shift[0] =
// local_bits) and bucket_sort_kernel for the low local_bits bits.
#ifndef BEVPOOL_BUCKET_SORT
#define BEVPOOL_BUCKET_SORT 1
#endif
// Per-group sort: a group of more than kBucketPartKeys keys is ranked by up to
// kBucketParts blocks.  Each part's block also counts the rest of its group,
// so more parts cost more counting: at 1 x 360 x 360 the per-group sort took
// 21.6 us with one block per group, 19.0 with 2 parts above 8192 keys, 20.0
// with 4, 20.7 with 4 above 6144 keys and 22.6 with 4 above 4096 (MI355X).
#ifndef BEVPOOL_BUCKET_PARTS
#define BEVPOOL_BUCKET_PARTS 2
#endif
#ifndef BEVPOOL_BUCKET_PART_KEYS
#define BEVPOOL_BUCKET_PART_KEYS 8192
#endif
constexpr int kBucketParts = BEVPOOL_BUCKET_PARTS;
constexpr int kBucketPartKeys = BEVPOOL_BUCKET_PART_KEYS;
struct DigitPlan {
  int passes = 1;
  int bits[4] = {1, 0, 0, 0};
  int shift[4] = {0, 0, 0, 0};
  int local_bits = 0;
};

DigitPlan plan_digits(int64_t n_cells) {
  int total_bits = 0;
  for (uint64_t v = uint64_t(n_cells > 1 ? n_cells - 1 : 0); v; v >>= 1) ++total_bits;
  if (total_bits < 1) total_bits = 1;
  DigitPlan p;
  if (BEVPOOL_BUCKET_SORT && total_bits > kMaxDigitBits && total_bits <= 2 * kMaxDigitBits) {
    p.bits[0] = (total_bits + 1) / 2;  // high digit: global pass
    // Narrower groups shorten the per-group sort, whose largest group sets
    // its length; tile histograms of up to 2^9 digits cost the global pass
    // no more than 2^8, 2^10 cost it ~5 us at 1 x 360 x 360 (MI355X).  So a
    // 16-bit rank space takes 9 + 7 bits (256 x 256: per-group sort 25.0 ->
    // 16.9 us), while 17 bits keep 9 + 8.
    if (total_bits - p.bits[0] > 7 && p.bits[0] < 9)
      p.bits[0] = total_bits - 7 < 9 ? total_bits - 7 : 9;
    p.local_bits = total_bits - p.bits[0];
    p.shift[0] = p.local_bits;
    return p;
  }
  p.passes = int((total_bits + kMaxDigitBits - 1) / kMaxDigitBits);
  const int per = (total_bits + p.passes - 1) / p.passes;
  int shift = 0;
  for (int i = 0; i < p.passes; ++i) {
    p.shift[i] = shift;
    p.bits[i] = total_bits - shift < per ? total_bits - shift : per;
    shift += p.bits[i];
  }
  return p;
}

struct IndexLayout {
  size_t keys_tmp, hist, totals, gstart, bcount, tile_bad, slices, total;
  int64_t sort_blocks, cell_blocks;
  int items;  // keys per thread of the tile kernels (sort_items)
};

// Slices of the sliced bucket sort (an upper bound: every group may end in a
// partial slice) and the bytes of their low-digit counts.
int64_t slice_bound(int64_t n_points, int64_t n_cells, int lbits) {
  return ceil_div(n_cells, int64_t(1) << lbits) + ceil_div(n_points, int64_t(kSliceKeys));
}

size_t slice_count_bytes(int64_t n_points, int64_t n_cells) {
  const DigitPlan plan = plan_digits(n_cells);
  if (plan.local_bits < kSlicedBits) return 0;
  return size_t(slice_bound(n_points, n_cells, plan.local_bits)) << plan.local_bits << 2;
}

// Index-stage workspace.  The slice counts at the end depend on n_cells; a
// caller that only uses the other regions may pass n_cells = 1.
IndexLayout index_layout(int64_t n_points, int64_t n_cells) {
  IndexLayout L;
  L.items = sort_items(n_points);
  L.sort_blocks = ceil_div(n_points, int64_t(kThreads) * L.items);
  L.cell_blocks = ceil_div(n_points, kThreads);
  size_t o = 0;
  L.keys_tmp = o;
  o = align256(o + size_t(n_points) * sizeof(uint64_t));
  L.hist = o;
  o = align256(o + size_t(kMaxRadix) * size_t(L.sort_blocks) * sizeof(int32_t));
  L.totals = o;
  o = align256(o + size_t(kMaxRadix) * sizeof(int32_t));
  L.gstart = o;  // start of each group of the global pass (per-group sort)
  o = align256(o + size_t(kMaxRadix) * sizeof(int32_t));
  L.bcount = o;
  o = align256(o + size_t(L.cell_blocks) * sizeof(int32_t));
  L.tile_bad = o;  // op level: invalid-rank count and first index per tile
  o = align256(o + size_t(2) * size_t(L.sort_blocks) * sizeof(int32_t));
  L.slices = o;
  o = align256(o + slice_count_bytes(n_points, n_cells));
  L.total = o;
  return L;
}

template <typename P>
P *at(void *base, size_t off) {
  return reinterpret_cast<P *>(static_cast<char *>(base) + off);
}

int check_index_args(int64_t n_points, int64_t n_cells, const void *rank, const void *meta,
                     void *ws, size_t ws_bytes) {
  if (n_points < 0 || n_points > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_points=%lld out of range [0, 2^31)", (long long)n_points);
  if (n_cells < 1 || n_cells > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "B*D*H*W=%lld out of range [1, 2^31)", (long long)n_cells);
  if (!meta || !ws) return fail(BEVPOOL_EINVAL, "null meta or workspace");
  if (n_points > 0 && !rank) return fail(BEVPOOL_EINVAL, "null rank");
  const size_t need = index_layout(n_points, n_cells).total;
  if (ws_bytes < need)
    return fail(BEVPOOL_ESPACE, "index workspace %zu bytes < required %zu", ws_bytes, need);
  return BEVPOOL_OK;
}

size_t dtype_size(int32_t dtype) { return dtype == BEVPOOL_F32 ? 4 : 2; }

// 4 consecutive cells of one channel of a channel-first tensor form one
// aligned 4-element vector when n_xy and the b/c/z strides are multiples of
// 4 and the base is aligned to 4 elements (tiles start at multiples of 64).
bool bev_vec_ok(const void *base, size_t es, int64_t n_xy, int64_t sb, int64_t sc,
                int64_t sz) {
  return n_xy % 4 == 0 && sb % 4 == 0 && sc % 4 == 0 && sz % 4 == 0 &&
         reinterpret_cast<uintptr_t>(base) % (4 * es) == 0;
}

template <typename T, int kCPL>
int launch_accum_pipe_t(int slots, unsigned grid, size_t smem, hipStream_t s, const char *x,
                        int64_t ld_bytes, int C, int CB, const uint64_t *keys,
                        const int32_t *meta, const int32_t *cend, float *acc,
                        const DepthRows &dr, bool stream_rows) {
#define BEVPOOL_PIPE_CASE(K)                                                                   \
  case K:                                                                                      \
    if constexpr (std::is_same<T, F32>::value) { /* depth-weighted rows are fp32 only */       \
      if (dr.depth) {                                                                          \
        hipLaunchKernelGGL((accum_pipe_kernel<T, K, kCPL, kRowsDepth>), dim3(grid),            \
                           dim3(kPipeThreads), smem, s, x, ld_bytes, C, CB, keys, meta, cend,  \
                           acc, kRangePoints, dr);                                            \
        break;                                                                                 \
      }                                                                                        \
    }                                                                                          \
    if (stream_rows)                                                                           \
      hipLaunchKernelGGL((accum_pipe_kernel<T, K, kCPL, kRowsStream>), dim3(grid),             \
                         dim3(kPipeThreads), smem, s, x, ld_bytes, C, CB, keys, meta, cend,    \
                         acc, kRangePoints, dr);                                              \
    else                                                                                       \
      hipLaunchKernelGGL((accum_pipe_kernel<T, K, kCPL, kRowsPlain>), dim3(grid),              \
                         dim3(kPipeThreads), smem, s, x, ld_bytes, C, CB, keys, meta, cend,    \
                         acc, kRangePoints, dr);                                              \
    break;
  switch (slots) {
    BEVPOOL_PIPE_CASE(1)
    BEVPOOL_PIPE_CASE(2)
    BEVPOOL_PIPE_CASE(3)
    BEVPOOL_PIPE_CASE(4)
    BEVPOOL_PIPE_CASE(5)
    BEVPOOL_PIPE_CASE(6)
    BEVPOOL_PIPE_CASE(7)
    BEVPOOL_PIPE_CASE(8)
    default:
      return fail(BEVPOOL_EINVAL, "internal: %d slots per thread", slots);
  }
#undef BEVPOOL_PIPE_CASE
  return check_launch("accum_pipe");
}

// Channels per summing lane for a block of CB channels split over kSummers
// waves: 1 (<= 64 per wave), 2 (<= 128) or 4 (<= 256).
int pipe_cpl(int CB) {
  const int cps = (CB + kSummers - 1) / kSummers;
  return cps <= 64 ? 1 : (cps <= 128 ? 2 : 4);
}

int launch_accum_pipe(int32_t dtype, int slots, unsigned grid, size_t smem, hipStream_t s,
                      const char *x, int64_t ld_bytes, int C, int CB, const uint64_t *keys,
                      const int32_t *meta, const int32_t *cend, float *acc,
                      const DepthRows &dr, bool stream_rows) {
  // summing-lane slots: channels for fp32, channel pairs for 16-bit rows
  const int cpl = dtype == BEVPOOL_F32 ? pipe_cpl(CB) : pipe_cpl((CB + 1) / 2);
#define BEVPOOL_PIPE_ARGS                                                                      \
  slots, grid, smem, s, x, ld_bytes, C, CB, keys, meta, cend, acc, dr, stream_rows
#define BEVPOOL_PIPE_DTYPE(T)                                                                  \
  return cpl == 1   ? launch_accum_pipe_t<T, 1>(BEVPOOL_PIPE_ARGS)                            \
         : cpl == 2 ? launch_accum_pipe_t<T, 2>(BEVPOOL_PIPE_ARGS)                            \
                    : launch_accum_pipe_t<T, 4>(BEVPOOL_PIPE_ARGS);
  switch (dtype) {
    case BEVPOOL_F32:
      BEVPOOL_PIPE_DTYPE(F32)
    case BEVPOOL_F16:
      BEVPOOL_PIPE_DTYPE(F16)
    default:
      BEVPOOL_PIPE_DTYPE(BF16)
  }
#undef BEVPOOL_PIPE_DTYPE
#undef BEVPOOL_PIPE_ARGS
}

// Pipelined forward accumulation (16-byte rows) into cell-major fp32 rows.
int launch_forward_pipe(int32_t dtype, const char *x, int64_t ld_bytes, int C, int64_t n_points,
                        const uint64_t *keys, const int32_t *meta, const int32_t *cend,
                        float *acc, const DepthRows &dr, hipStream_t s) {
  const size_t es = dtype_size(dtype);
  // plain block order: ranges that run at the same time then read rows from
  // one window of the feature tensor (an XCD-contiguous order measured slower)
  const unsigned grid = unsigned(ceil_div(n_points, kRangePoints));
  // channel block of at most 384 bytes per row: <= 6 16-byte slots per thread per
  // stage and two stages + ranks in <= 24.3 KB of LDS
  const int CBmax = int(384 / es);
  const int CB = C < CBmax ? C : CBmax;
  const int rowq = int(size_t(CB) * es / 16);
  const int slots = (kStageRows * rowq + kLoaders - 1) / kLoaders;
  const size_t smem = size_t(2) * kStageRows * rowq * 16 + size_t(2) * kStageRows * sizeof(int);
  if (smem > 65536) return fail(BEVPOOL_EINVAL, "internal: %zu bytes of LDS", smem);
  // rows of every point (an upper bound of the kept rows read)
  const bool stream_rows = !dr.depth && n_points * int64_t(C) * int64_t(es) <= kStreamRowBytes;
  LaunchTimer t("accum_rows", s);
  return launch_accum_pipe(dtype, slots, grid, smem, s, x, ld_bytes, C, CB, keys, meta, cend, acc,
                           dr, stream_rows);
}

// cell-major fp32 rows -> channel-first output (zeros for empty cells).
int launch_rows_to_bev(const float *acc, int32_t dtype, int C, const int32_t *cell_start,
                       const int32_t *cell_end, int64_t n_cells, int n_z, int64_t n_xy,
                       int64_t out_stride_b, int64_t out_stride_c, int64_t out_stride_z, void *out,
                       hipStream_t s, MetaReport report = {}, bool raw16 = false) {
  if (int st = check_grid(ceil_div(n_cells, kCellTile), kThreads, "cell tiles")) return st;
  const unsigned tiles = unsigned(ceil_div(n_cells, kCellTile));
  const int CT = C < kTileChannels ? C : kTileChannels;
  const size_t es = dtype_size(dtype);
  const size_t smem = size_t(kCellTile) * size_t(CT + 1) * sizeof(uint32_t);
  if (raw16 && es != 2) return fail(BEVPOOL_EINVAL, "internal: 16-bit rows for a 32-bit output");
  // 16-byte row pieces: 4 fp32 or 8 16-bit channels
  const int per = raw16 ? 8 : 4;
  const bool vrow = (C % per == 0) && (CT % per == 0) &&
                    (reinterpret_cast<uintptr_t>(acc) % 16 == 0);
  const bool vbev = bev_vec_ok(out, es, n_xy, out_stride_b, out_stride_c, out_stride_z);
  LaunchTimer t("rows_to_bev", s);
#define BEVPOOL_R2B(T, VR, VB, R16)                                                            \
  hipLaunchKernelGGL((rows_to_bev_kernel<T, VR, VB, R16>), dim3(tiles), dim3(kThreads), smem,  \
                     s, acc, C, CT, cell_start, cell_end, n_cells, n_z, n_xy, out_stride_b,    \
                     out_stride_c, out_stride_z, static_cast<T::raw *>(out), report)
#define BEVPOOL_R2B_T(T, R16)                                                                  \
  if (vrow && vbev) BEVPOOL_R2B(T, true, true, R16);                                          \
  else if (vrow) BEVPOOL_R2B(T, true, false, R16);                                            \
  else if (vbev) BEVPOOL_R2B(T, false, true, R16);                                            \
  else BEVPOOL_R2B(T, false, false, R16);
  switch (dtype) {
    case BEVPOOL_F32:
      BEVPOOL_R2B_T(F32, false)
      break;
    case BEVPOOL_F16:
      if (raw16) {
        BEVPOOL_R2B_T(F16, true)
      } else {
        BEVPOOL_R2B_T(F16, false)
      }
      break;
    default:
      if (raw16) {
        BEVPOOL_R2B_T(BF16, true)
      } else {
        BEVPOOL_R2B_T(BF16, false)
      }
      break;
  }
#undef BEVPOOL_R2B_T
#undef BEVPOOL_R2B
  return check_launch("rows_to_bev");
}

// channel-first gradient -> cell-major rows of the occupied cells (raw bits).
int launch_bev_to_rows(const void *grad, size_t es, int64_t gsb, int64_t gsc, int64_t gsz, int C,
                       const int32_t *cell_start, const int32_t *cell_end, int64_t n_cells,
                       int n_z, int64_t n_xy, void *rows, hipStream_t s) {
  if (int st = check_grid(ceil_div(n_cells, kCellTile), kThreads, "cell tiles")) return st;
  const unsigned tiles = unsigned(ceil_div(n_cells, kCellTile));
  const int CT = C < kTileChannels ? C : kTileChannels;
  const size_t smem = size_t(kCellTile) * size_t(CT + 1) * es;
  const bool vrow = (size_t(C) * es % 16 == 0) && (size_t(CT) * es % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(rows) % 16 == 0);
  const bool vbev = bev_vec_ok(grad, es, n_xy, gsb, gsc, gsz);
  const bool occ_first = n_cells >= kOccFirstCells;
  LaunchTimer t("bev_to_rows", s);
#define BEVPOOL_B2R(TR, VR, VB)                                                                \
  hipLaunchKernelGGL((bev_to_rows_kernel<TR, VR, VB>), dim3(tiles), dim3(kThreads), smem, s,   \
                     static_cast<const TR *>(grad), C, CT, cell_start, cell_end, n_cells, n_z, \
                     n_xy, gsb, gsc, gsz, occ_first, static_cast<TR *>(rows))
#define BEVPOOL_B2R_T(TR)                                                                      \
  if (vrow && vbev) BEVPOOL_B2R(TR, true, true);                                              \
  else if (vrow) BEVPOOL_B2R(TR, true, false);                                                \
  else if (vbev) BEVPOOL_B2R(TR, false, true);                                                \
  else BEVPOOL_B2R(TR, false, false);
  if (es == 4) {
    BEVPOOL_B2R_T(uint32_t)
  } else {
    BEVPOOL_B2R_T(uint16_t)
  }
#undef BEVPOOL_B2R_T
#undef BEVPOOL_B2R
  return check_launch("bev_to_rows");
}

// Zero `bytes` bytes at p (4-byte aligned, a multiple of 4 bytes) with
// zero_fill_kernel.
int launch_zero_fill(void *p, size_t bytes, hipStream_t s) {
  if (bytes == 0) return BEVPOOL_OK;
  const bool vec = reinterpret_cast<uintptr_t>(p) % 16 == 0;
  const int64_t n16 = vec ? int64_t(bytes / 16) : 0;
  const int64_t n4 = int64_t((bytes - size_t(n16) * 16) / 4);
  const int64_t items = n16 > n4 ? n16 : n4;
  const int64_t blocks = ceil_div(items, kThreads) < 4096 ? ceil_div(items, kThreads) : 4096;
  LaunchTimer t("zero_fill", s);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                     static_cast<u32x4 *>(p), n16,
                     reinterpret_cast<uint32_t *>(static_cast<char *>(p) + n16 * 16), n4);
  return check_launch("zero_fill");
}

// Channels per lane of the legacy kernels: 1 (C <= 64), 2 (<= 128), else 4
// (with a loop over 256-channel blocks).
int legacy_cpl(int C) { return C <= 64 ? 1 : (C <= 128 ? 2 : 4); }

unsigned legacy_grid(int64_t cap) {
  const int64_t b = ceil_div(cap, kWaves);
  return unsigned(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

int check_legacy_args(int64_t n, int32_t C, const void *geom, const void *starts,
                      const void *lengths, int64_t n_intervals, int32_t b, int32_t d, int32_t h,
                      int32_t w, const void *out) {
  if (n < 0 || n > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "n=%lld out of range", (long long)n);
  if (C < 1) return fail(BEVPOOL_EINVAL, "C must be positive");
  if (b < 1 || d < 1 || h < 1 || w < 1)
    return fail(BEVPOOL_EINVAL, "b, d, h, w must be positive");
  if (int64_t(b) * d * h * w > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "b*d*h*w exceeds 2^31-1");
  if (n_intervals < 0 || n_intervals > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_intervals out of range");
  if (!out) return fail(BEVPOOL_EINVAL, "null output");
  if (n_intervals > 0 && (!geom || !starts || !lengths))
    return fail(BEVPOOL_EINVAL, "null geom_feats / interval arrays");
  return BEVPOOL_OK;
}

// Layout of the op-level buffers (bevpool_op_forward / bevpool_op_backward).
// The index buffer keeps what the backward needs: meta, ranks, sorted keys and
// cell ranges.  The scratch buffer holds the index-stage workspace and the
// cell rows; it is needed only during a call.
struct OpIndexLayout {
  size_t meta, rank, keys, cstart, cend, total;
};

OpIndexLayout op_index_layout(int64_t n, int64_t cells) {
  OpIndexLayout L;
  size_t o = 0;
  L.meta = o;
  o = align256(o + BEVPOOL_META_LEN * sizeof(int32_t));
  L.rank = o;
  o = align256(o + size_t(n) * sizeof(int32_t));
  L.keys = o;
  o = align256(o + size_t(n) * sizeof(uint64_t));
  L.cstart = o;
  o = align256(o + size_t(cells) * sizeof(int32_t));
  L.cend = o;
  o = align256(o + size_t(cells) * sizeof(int32_t));
  L.total = o;
  return L;
}

struct OpScratchLayout {
  size_t index_ws, rows, total;
};

OpScratchLayout op_scratch_layout(int64_t n, int64_t cells, int32_t C) {
  OpScratchLayout L;
  size_t o = 0;
  L.index_ws = o;
  o = align256(o + index_layout(n, cells).total);
  L.rows = o;
  o = align256(o + size_t(cells) * size_t(C) * sizeof(float));
  L.total = o;
  return L;
}

// Scratch of the allocation-free op-level forward: the index buffer
// (op_index_layout) and the scratch (op_scratch_layout) of one call live in
// this array, one copy per GPU, held until
// the process ends.  Host code never passes `scratch` itself to a kernel or
// a copy (in host code the name is a host-side stand-in, not a device
// address): it uses the device address hipGetSymbolAddress returns for the
// current device, cached per device by noalloc_scratch().
constexpr size_t kNoAllocScratchBytes = BEVPOOL_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved once per
// device, with that device current), or nullptr with the error recorded.
void *noalloc_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(BEVPOOL_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(BEVPOOL_EINVAL, "device %d beyond the %d devices the scratch table holds", dev,
         kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(BEVPOOL_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
           hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int bevpool_abi_version(void) { return BEVPOOL_ABI_VERSION; }

const char *bevpool_last_error(void) { return g_last_error.c_str(); }

size_t bevpool_index_workspace_bytes(int64_t n_points, int64_t n_cells) {
  if (n_points < 0) return 0;
  return index_layout(n_points, n_cells < 1 ? 1 : n_cells).total;
}

int bevpool_quantize_geom(const float *geom, int64_t n_points, int64_t geom_row_stride,
                          int64_t points_per_batch, int32_t n_batch, const float offset[3],
                          const float dx[3], const int32_t nx[3], int32_t *rank, int32_t *meta,
                          void *workspace, size_t workspace_bytes, void *stream) {
  g_last_error.clear();
  if (!offset || !dx || !nx) return fail(BEVPOOL_EINVAL, "null offset/dx/nx");
  if (n_batch < 1 || nx[0] < 1 || nx[1] < 1 || nx[2] < 1)
    return fail(BEVPOOL_EINVAL, "grid sizes must be positive (B=%d nx=%d,%d,%d)", n_batch, nx[0],
                nx[1], nx[2]);
  const int64_t n_cells = int64_t(n_batch) * nx[0] * nx[1] * nx[2];
  int st = check_index_args(n_points, n_cells, rank, meta, workspace, workspace_bytes);
  if (st) return st;
  if (n_points > 0 && (!geom || geom_row_stride < 3 || points_per_batch < 1 ||
                       ceil_div(n_points, points_per_batch) > n_batch))
    return fail(BEVPOOL_EINVAL, "bad geometry layout (row stride %lld, points/batch %lld)",
                (long long)geom_row_stride, (long long)points_per_batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const IndexLayout L = index_layout(n_points, n_cells);
  const DigitPlan plan = plan_digits(n_cells);
  {
    // also resets meta (block 0); an empty input still launches that block
    LaunchTimer t("quantize_geom", s);
    const unsigned grid = sort_grid(L.sort_blocks);
    // batch index = point / points_per_batch (every point index is < 2^31)
    const FastDiv ppb = make_fast_div(uint32_t(
        points_per_batch < 1 ? 1 : (points_per_batch > (int64_t(1) << 31) ? (int64_t(1) << 31)
                                                                          : points_per_batch)));
    const bool vec = geom_row_stride == 3 && n_points >= 4 &&
                     reinterpret_cast<uintptr_t>(geom) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(rank) % 16 == 0;
#define BEVPOOL_QUANT(V, IT)                                                                   \
  hipLaunchKernelGGL((quantize_geom_kernel<V, IT>), dim3(grid), dim3(kThreads), 0, s, geom,     \
                     n_points, geom_row_stride, ppb, offset[0], offset[1], offset[2], dx[0],     \
                     dx[1], dx[2], nx[0], nx[1], nx[2], rank, at<int32_t>(workspace, L.hist),   \
                     int(L.sort_blocks), plan.shift[0], plan.bits[0], meta)
    if (L.items == kItemsLarge) {
      if (vec) BEVPOOL_QUANT(true, kItemsLarge); else BEVPOOL_QUANT(false, kItemsLarge);
    } else {
      if (vec) BEVPOOL_QUANT(true, kItemsSmall); else BEVPOOL_QUANT(false, kItemsSmall);
    }
#undef BEVPOOL_QUANT
  }
  return check_launch("quantize_geom");
}

int bevpool_quantize_cameras(const float *frustum, int32_t D, int32_t fH, int32_t fW,
                             const float *rots, const float *trans, const float *intrins,
                             const float *post_rots, const float *post_trans,
                             const float *extra_rots, const float *extra_trans,
                             int32_t n_cams_per_batch, int32_t n_batch, const float offset[3],
                             const float dx[3], const int32_t nx[3], int32_t *rank,
                             int32_t *meta, void *workspace, size_t workspace_bytes,
                             void *stream) {
  g_last_error.clear();
  if (!offset || !dx || !nx) return fail(BEVPOOL_EINVAL, "null offset/dx/nx");
  if (n_batch < 1 || n_cams_per_batch < 1 || D < 1 || fH < 1 || fW < 1)
    return fail(BEVPOOL_EINVAL, "bad frustum/camera sizes");
  if (nx[0] < 1 || nx[1] < 1 || nx[2] < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t dhw = int64_t(D) * fH * fW;
  const int64_t n_points = dhw * n_cams_per_batch * n_batch;
  const int64_t n_cells = int64_t(n_batch) * nx[0] * nx[1] * nx[2];
  int st = check_index_args(n_points, n_cells, rank, meta, workspace, workspace_bytes);
  if (st) return st;
  if (!frustum || !rots || !trans || !intrins || !post_rots || !post_trans)
    return fail(BEVPOOL_EINVAL, "null frustum/camera matrices");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const IndexLayout L = index_layout(n_points, n_cells);
  const DigitPlan plan = plan_digits(n_cells);
  const CameraMats cm{rots, trans, intrins, post_rots, post_trans, extra_rots, extra_trans,
                      n_cams_per_batch};
  LaunchTimer t("quantize_cameras", s);
#define BEVPOOL_QCAM(IT)                                                                       \
  hipLaunchKernelGGL((quantize_frustum_kernel<IT>), dim3(sort_grid(L.sort_blocks)),           \
                     dim3(kThreads), 0, s, frustum, n_points, make_fast_div(uint32_t(dhw)),    \
                     make_fast_div(uint32_t(n_cams_per_batch)), cm, offset[0], offset[1],      \
                     offset[2], dx[0], dx[1], dx[2], nx[0], nx[1], nx[2], rank,                \
                     at<int32_t>(workspace, L.hist), int(L.sort_blocks), plan.shift[0],        \
                     plan.bits[0], meta)
  if (L.items == kItemsLarge) BEVPOOL_QCAM(kItemsLarge); else BEVPOOL_QCAM(kItemsSmall);
#undef BEVPOOL_QCAM
  return check_launch("quantize_cameras");
}

// tile_bad: count invalid ranks per tile in the index workspace (for
// sort_impl's first scatter to reduce into meta) instead of initialising meta
// here and counting into it with atomics.
static int coord_ranks_impl(const void *coords, int32_t coord_bytes, int64_t n_points,
                            int64_t coords_row_stride, int32_t B, int32_t D, int32_t H,
                            int32_t W, int32_t *rank, int32_t *meta, void *workspace,
                            size_t workspace_bytes, void *stream, bool tile_bad) {
  if (B < 1 || D < 1 || H < 1 || W < 1)
    return fail(BEVPOOL_EINVAL, "B, D, H, W must be positive");
  if (coord_bytes != 4 && coord_bytes != 8)
    return fail(BEVPOOL_EINVAL, "coord_bytes must be 4 or 8, got %d", coord_bytes);
  const int64_t n_cells = int64_t(B) * D * H * W;
  int st = check_index_args(n_points, n_cells, rank, meta, workspace, workspace_bytes);
  if (st) return st;
  if (n_points > 0 && (!coords || coords_row_stride < 4))
    return fail(BEVPOOL_EINVAL, "bad coords layout");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!tile_bad || n_points == 0) {  // no points: no scatter writes meta
    {
      LaunchTimer t("init_meta", s);
      hipLaunchKernelGGL(init_meta_kernel, dim3(1), dim3(64), 0, s, meta);
    }
    if ((st = check_launch("init_meta"))) return st;
  }
  if (n_points == 0) return BEVPOOL_OK;
  const IndexLayout L = index_layout(n_points, n_cells);
  const DigitPlan plan = plan_digits(n_cells);
  int32_t *bad = at<int32_t>(workspace, L.tile_bad);
  LaunchTimer t("coord_ranks", s);
#define BEVPOOL_CRANKS(TC, IT, TB)                                                             \
  hipLaunchKernelGGL((coord_ranks_kernel<TC, IT, TB>), dim3(sort_grid(L.sort_blocks)),         \
                     dim3(kThreads), 0, s, static_cast<const TC *>(coords), n_points,          \
                     coords_row_stride, int64_t(B), int64_t(D), int64_t(H), int64_t(W), rank,  \
                     meta, at<int32_t>(workspace, L.hist), int(L.sort_blocks), plan.shift[0],  \
                     plan.bits[0], bad)
#define BEVPOOL_CRANKS_T(TC, IT)                                                               \
  if (tile_bad) BEVPOOL_CRANKS(TC, IT, true); else BEVPOOL_CRANKS(TC, IT, false);
  if (coord_bytes == 4) {
    if (L.items == kItemsLarge) { BEVPOOL_CRANKS_T(int32_t, kItemsLarge) }
    else { BEVPOOL_CRANKS_T(int32_t, kItemsSmall) }
  } else {
    if (L.items == kItemsLarge) { BEVPOOL_CRANKS_T(int64_t, kItemsLarge) }
    else { BEVPOOL_CRANKS_T(int64_t, kItemsSmall) }
  }
#undef BEVPOOL_CRANKS_T
#undef BEVPOOL_CRANKS
  return check_launch("coord_ranks");
}

int bevpool_coord_ranks(const void *coords, int32_t coord_bytes, int64_t n_points,
                        int64_t coords_row_stride, int32_t B, int32_t D, int32_t H, int32_t W,
                        int32_t *rank, int32_t *meta, void *workspace, size_t workspace_bytes,
                        void *stream) {
  g_last_error.clear();
  return coord_ranks_impl(coords, coord_bytes, n_points, coords_row_stride, B, D, H, W, rank,
                          meta, workspace, workspace_bytes, stream, false);
}

// tile_bad: the per-tile invalid-rank counts of coord_ranks_impl(...,
// tile_bad = true) in this workspace; the first scatter then writes all of
// meta.  nullptr: meta was initialised by the rank kernel's call.
static int sort_impl(const int32_t *rank, int64_t n_points, int64_t n_cells, uint64_t *keys,
                     int32_t *cell_start, int32_t *cell_end, int32_t *meta, void *workspace,
                     size_t workspace_bytes, void *stream, bool tile_bad) {
  int st = check_index_args(n_points, n_cells, rank, meta, workspace, workspace_bytes);
  if (st) return st;
  if (!cell_start || !cell_end) return fail(BEVPOOL_EINVAL, "null cell_start/cell_end");
  if (n_points > 0 && !keys) return fail(BEVPOOL_EINVAL, "null keys");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const IndexLayout L = index_layout(n_points, n_cells);
  const DigitPlan plan = plan_digits(n_cells);
  int32_t *hist = at<int32_t>(workspace, L.hist);
  int32_t *totals = at<int32_t>(workspace, L.totals);
  int32_t *gstart = at<int32_t>(workspace, L.gstart);
  uint64_t *tmp = at<uint64_t>(workspace, L.keys_tmp);
  if (n_points == 0) {
    // no points: only the dense cell ranges need clearing
    LaunchTimer t("radix_scan", s);
    hipLaunchKernelGGL(radix_scan_kernel, dim3(64), dim3(kThreads), 0, s, hist, 0, totals,
                       cell_start, cell_end, n_cells);
    return check_launch("radix_scan");
  }
  const int nb = int(L.sort_blocks);
  const uint64_t *src = nullptr;
  const bool bucketed = plan.local_bits > 0;
  for (int pass = 0; pass < plan.passes; ++pass) {
    uint64_t *dst = bucketed ? tmp : (((plan.passes - 1 - pass) % 2 == 0) ? keys : tmp);
    const bool large = L.items == kItemsLarge;
    if (pass > 0) {
      LaunchTimer t("radix_hist", s);
#define BEVPOOL_RHIST(IT)                                                                      \
  hipLaunchKernelGGL((radix_hist_kernel<IT>), dim3(sort_grid(nb)), dim3(kThreads), 0, s, src,   \
                     meta, hist, nb, plan.shift[pass], plan.bits[pass])
      if (large) BEVPOOL_RHIST(kItemsLarge); else BEVPOOL_RHIST(kItemsSmall);
#undef BEVPOOL_RHIST
      if ((st = check_launch("radix_hist"))) return st;
    }
    {
      LaunchTimer t("radix_scan", s);
      hipLaunchKernelGGL(radix_scan_kernel, dim3(1u << plan.bits[pass]), dim3(kThreads), 0, s,
                         hist, nb, totals, cell_start, cell_end,
                         pass == 0 && !bucketed ? n_cells : 0);
      if ((st = check_launch("radix_scan"))) return st;
    }
    {
      LaunchTimer t("radix_scatter", s);
#define BEVPOOL_RSCAT(FROM_RANK, IT)                                                           \
  hipLaunchKernelGGL((radix_scatter_kernel<FROM_RANK, IT>), dim3(xcd_grid(nb)), dim3(kThreads), \
                     0, s, FROM_RANK ? rank : nullptr, FROM_RANK ? nullptr : src, n_points,    \
                     meta, dst, hist, totals, nb, plan.shift[pass], plan.bits[pass],           \
                     FROM_RANK && tile_bad ? at<int32_t>(workspace, L.tile_bad) : nullptr,     \
                     bucketed ? gstart : nullptr)
      if (pass == 0) {
        if (large) BEVPOOL_RSCAT(true, kItemsLarge); else BEVPOOL_RSCAT(true, kItemsSmall);
      } else {
        if (large) BEVPOOL_RSCAT(false, kItemsLarge); else BEVPOOL_RSCAT(false, kItemsSmall);
      }
#undef BEVPOOL_RSCAT
      if ((st = check_launch("radix_scatter"))) return st;
    }
    src = dst;
  }
  if (bucketed && plan.local_bits >= kSlicedBits) {
    // groups of 2^10 cells (up to ~65 K keys at 2 x 720 x 720), cut into
    // slices -> sorted keys and the dense cell ranges
    const int lb = plan.local_bits;
    const int n_groups = int(ceil_div(n_cells, int64_t(1) << lb));
    const int64_t n_slices = slice_bound(n_points, n_cells, lb);
    if ((st = check_grid(n_slices, kThreads, "bucket slices"))) return st;
    int32_t *scnt = at<int32_t>(workspace, L.slices);
    const size_t R4 = size_t(4) << lb;
    {
      LaunchTimer t("bucket_count", s);
      hipLaunchKernelGGL(bucket_count_kernel<kSliceWaves>, dim3(unsigned(n_slices)),
                         dim3(64 * kSliceWaves), R4, s, src, totals, n_groups, lb, scnt);
      if ((st = check_launch("bucket_count"))) return st;
    }
    {
      LaunchTimer t("bucket_scan", s);
      hipLaunchKernelGGL(bucket_scan_kernel, dim3(unsigned(n_groups)), dim3(kThreads), 0, s,
                         totals, n_groups, n_cells, lb, scnt, cell_start, cell_end);
      if ((st = check_launch("bucket_scan"))) return st;
    }
    LaunchTimer t("bucket_place", s);
    hipLaunchKernelGGL(bucket_place_kernel<kSliceWaves>, dim3(unsigned(n_slices)),
                       dim3(64 * kSliceWaves), kSliceWaves * R4, s, src, totals, n_groups, lb,
                       scnt, keys);
    return check_launch("bucket_place");
  }
  if (bucketed) {
    // groups of at most 2^9 cells -> sorted keys and the dense cell ranges
    LaunchTimer t("bucket_sort", s);
    const int64_t n_buckets = ceil_div(n_cells, int64_t(1) << plan.local_bits);
    hipLaunchKernelGGL(bucket_sort_kernel<16>, dim3(unsigned(n_buckets * kBucketParts)),
                       dim3(16 * 64), size_t(16 + 2) << plan.local_bits << 2, s, src, totals,
                       gstart, int(n_buckets), n_cells, keys, cell_start, cell_end,
                       plan.local_bits, kBucketParts, kBucketPartKeys);
    return check_launch("bucket_sort");
  }
  {
    LaunchTimer t("cell_ranges", s);
    const unsigned g = unsigned(ceil_div(n_points, int64_t(kThreads) * 4));
    if (reinterpret_cast<uintptr_t>(keys) % 16 == 0)
      hipLaunchKernelGGL(cell_ranges_kernel<true>, dim3(g), dim3(kThreads), 0, s, keys, meta,
                         cell_start, cell_end);
    else
      hipLaunchKernelGGL(cell_ranges_kernel<false>, dim3(g), dim3(kThreads), 0, s, keys, meta,
                         cell_start, cell_end);
  }
  return check_launch("cell_ranges");
}

int bevpool_sort(const int32_t *rank, int64_t n_points, int64_t n_cells, uint64_t *keys,
                 int32_t *cell_start, int32_t *cell_end, int32_t *meta, void *workspace,
                 size_t workspace_bytes, void *stream) {
  g_last_error.clear();
  return sort_impl(rank, n_points, n_cells, keys, cell_start, cell_end, meta, workspace,
                   workspace_bytes, stream, false);
}

// Device address for writing to `dst`: pinned host memory through its device
// address, device memory of the current device as is; anything else
// (pageable host memory the GPU cannot reach) is refused.
static int report_address(int32_t *dst, int32_t **dev_dst) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, dst) != hipSuccess) {
    (void)hipGetLastError();  // unknown pointer: clear the lookup's error
    return fail(BEVPOOL_EINVAL, "report destination is neither pinned host nor device memory");
  }
  if (a.type == hipMemoryTypeHost) {
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, dst, 0) != hipSuccess || !d) {
      (void)hipGetLastError();
      return fail(BEVPOOL_EHIP, "hipHostGetDevicePointer failed for the report destination");
    }
    *dev_dst = static_cast<int32_t *>(d);
    return BEVPOOL_OK;
  }
  if (a.type == hipMemoryTypeDevice) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != a.device)
      return fail(BEVPOOL_EINVAL, "report destination on device %d, current device %d",
                  a.device, dev);
    *dev_dst = dst;
    return BEVPOOL_OK;
  }
  return fail(BEVPOOL_EINVAL, "report destination is neither pinned host nor device memory");
}

int bevpool_meta_report(const int32_t *meta, int32_t *dst, void *stream) {
  g_last_error.clear();
  if (!meta || !dst) return fail(BEVPOOL_EINVAL, "null meta or destination");
  int32_t *dev_dst = nullptr;
  if (int st = report_address(dst, &dev_dst)) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(meta_report_kernel, dim3(1), dim3(64), 0, s, meta, dev_dst);
  return check_launch("meta_report");
}

int bevpool_intervals(const uint64_t *keys, int64_t n_points, const int32_t *cell_end,
                      int32_t *starts, int32_t *lengths, int32_t *cells, int32_t *meta,
                      void *workspace, size_t workspace_bytes, void *stream) {
  g_last_error.clear();
  if (n_points < 0 || n_points > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_points out of range");
  if (!meta) return fail(BEVPOOL_EINVAL, "meta is null");
  const IndexLayout L = index_layout(n_points, 1);
  if (workspace_bytes < L.total) return fail(BEVPOOL_ESPACE, "index workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t *bcount = at<int32_t>(workspace, L.bcount);
  if (n_points == 0) {
    // meta[N_INTERVALS] was zeroed by the rank stage
    return BEVPOOL_OK;
  }
  if (!keys || !cell_end || !starts || !lengths || !cells)
    return fail(BEVPOOL_EINVAL, "null interval argument");
  int st;
  {
    LaunchTimer t("count_starts", s);
    hipLaunchKernelGGL(count_starts_kernel, dim3(unsigned(L.cell_blocks)), dim3(kThreads), 0, s,
                       keys, meta, bcount);
    if ((st = check_launch("count_starts"))) return st;
  }
  {
    LaunchTimer t("scan_counts", s);
    hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(kThreads), 0, s, bcount, L.cell_blocks,
                       meta + BEVPOOL_META_N_INTERVALS);
    if ((st = check_launch("scan_counts"))) return st;
  }
  LaunchTimer t("interval_write", s);
  hipLaunchKernelGGL(interval_write_kernel, dim3(unsigned(L.cell_blocks)), dim3(kThreads), 0, s,
                     keys, meta, cell_end, bcount, starts, lengths, cells);
  return check_launch("interval_write");
}

size_t bevpool_forward_scratch_bytes(int64_t n_cells, int32_t C) {
  if (n_cells < 0 || C < 0) return 0;
  return size_t(n_cells) * size_t(C) * sizeof(float);
}

// bevpool_forward; `report` (optional) is written by the transpose's first
// block.
static int forward_impl(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                        int64_t n_points, const uint64_t *keys, const int32_t *cell_start,
                        const int32_t *cell_end, const int32_t *meta, int32_t n_batch,
                        int32_t n_z, int64_t n_xy, int64_t out_stride_b, int64_t out_stride_c,
                        int64_t out_stride_z, void *out, void *scratch, size_t scratch_bytes,
                        void *stream, MetaReport report) {
  if (dtype != BEVPOOL_F32 && dtype != BEVPOOL_F16 && dtype != BEVPOOL_BF16)
    return fail(BEVPOOL_EINVAL, "unsupported dtype code %d", dtype);
  if (C < 1) return fail(BEVPOOL_EINVAL, "C must be positive");
  if (n_batch < 1 || n_z < 1 || n_xy < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t n_cells = int64_t(n_batch) * n_z * n_xy;
  if (n_cells > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "too many cells");
  if (n_points < 0 || n_points > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_points out of range");
  if (!out || !cell_start || !cell_end || !meta) return fail(BEVPOOL_EINVAL, "null argument");
  if (n_points > 0 && (!feats || !keys || feats_row_stride < C))
    return fail(BEVPOOL_EINVAL, "bad feats layout");
  if (scratch_bytes < bevpool_forward_scratch_bytes(n_cells, C) || !scratch)
    return fail(BEVPOOL_ESPACE, "forward scratch too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float *acc = static_cast<float *>(scratch);
  int st;
  bool raw16 = false;  // cell rows hold 16-bit output values (pipelined accumulation)
  if (n_points > 0) {
    const size_t es = dtype_size(dtype);
    const bool vec16 = (size_t(C) * es) % 16 == 0 && (size_t(feats_row_stride) * es) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(feats) % 16 == 0;
    // plain block order: ranges that run at the same time then read rows from
    // one window of the feature tensor (an XCD-contiguous order measured slower)
    const unsigned grid = unsigned(ceil_div(n_points, kRangePoints));
    if (vec16) {
      st = launch_forward_pipe(dtype, static_cast<const char *>(feats),
                               int64_t(size_t(feats_row_stride) * es), C, n_points, keys, meta,
                               cell_end, acc, DepthRows{nullptr, {}, {}}, s);
      if (st) return st;
      raw16 = es == 2;
    } else {
      const int CB = C < kThreads ? C : kThreads;
      int R = 8192 / CB;
      if (R > 64) R = 64;
      if (R < 1) R = 1;
      const size_t smem = size_t(R) * CB * sizeof(float) + size_t(R + 1) * sizeof(int);
      LaunchTimer t("accum_rows", s);
      switch (dtype) {
        case BEVPOOL_F32:
          hipLaunchKernelGGL(accum_rows_kernel<F32>, dim3(grid), dim3(kThreads), smem, s,
                             static_cast<const uint32_t *>(feats), feats_row_stride, C, CB, R,
                             keys, meta, cell_end, acc, kRangePoints);
          break;
        case BEVPOOL_F16:
          hipLaunchKernelGGL(accum_rows_kernel<F16>, dim3(grid), dim3(kThreads), smem, s,
                             static_cast<const uint16_t *>(feats), feats_row_stride, C, CB, R,
                             keys, meta, cell_end, acc, kRangePoints);
          break;
        default:
          hipLaunchKernelGGL(accum_rows_kernel<BF16>, dim3(grid), dim3(kThreads), smem, s,
                             static_cast<const uint16_t *>(feats), feats_row_stride, C, CB, R,
                             keys, meta, cell_end, acc, kRangePoints);
          break;
      }
      if ((st = check_launch("accum_rows"))) return st;
    }
  }
  return launch_rows_to_bev(acc, dtype, C, cell_start, cell_end, n_cells, n_z, n_xy,
                            out_stride_b, out_stride_c, out_stride_z, out, s, report, raw16);
}

int bevpool_forward(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                    int64_t n_points, const uint64_t *keys, const int32_t *cell_start,
                    const int32_t *cell_end, const int32_t *meta, int32_t n_batch, int32_t n_z,
                    int64_t n_xy, int64_t out_stride_b, int64_t out_stride_c,
                    int64_t out_stride_z, void *out, void *scratch, size_t scratch_bytes,
                    void *stream) {
  g_last_error.clear();
  return forward_impl(feats, dtype, feats_row_stride, C, n_points, keys, cell_start, cell_end,
                      meta, n_batch, n_z, n_xy, out_stride_b, out_stride_c, out_stride_z, out,
                      scratch, scratch_bytes, stream, MetaReport{});
}

int bevpool_planar_rows(const float *src, int64_t stride_bn, int64_t stride_c, int32_t BN,
                        int32_t C, int64_t S, float *rows, void *stream) {
  g_last_error.clear();
  if (BN < 0 || C < 1 || S < 0) return fail(BEVPOOL_EINVAL, "bad planar shape");
  const int64_t n_rows = int64_t(BN) * S;
  if (n_rows == 0) return BEVPOOL_OK;
  if (!src || !rows) return fail(BEVPOOL_EINVAL, "null argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = C % 4 == 0 && S % 4 == 0 && stride_bn % 4 == 0 && stride_c % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(rows) % 16 == 0;
  LaunchTimer t("planar_rows", s);
  int st = check_grid(vec ? BN * ceil_div(S, C <= 128 ? kPlanarTile : 256) : ceil_div(n_rows * C, kThreads),
                      kThreads, "planar_rows");
  if (st) return st;
  if (vec && C <= 128) {
    const int64_t tiles_s = ceil_div(S, kPlanarTile);
    const size_t smem = size_t(kPlanarTile) * size_t(C + 1) * sizeof(float);
#define BEVPOOL_PT(K)                                                                          \
  case K:                                                                                      \
    hipLaunchKernelGGL((planar_tile_kernel<K>), dim3(unsigned(int64_t(BN) * tiles_s)),          \
                       dim3(kThreads), smem, s, src, C, S, tiles_s, stride_bn, stride_c, rows); \
    break;
    switch ((C * (kPlanarTile / 4) + kThreads - 1) / kThreads) {
      BEVPOOL_PT(1) BEVPOOL_PT(2) BEVPOOL_PT(3) BEVPOOL_PT(4)
      BEVPOOL_PT(5) BEVPOOL_PT(6) BEVPOOL_PT(7) BEVPOOL_PT(8)
      BEVPOOL_PT(9) BEVPOOL_PT(10) BEVPOOL_PT(11) BEVPOOL_PT(12)
      BEVPOOL_PT(13) BEVPOOL_PT(14) BEVPOOL_PT(15) BEVPOOL_PT(16)
      default:
        return fail(BEVPOOL_EINVAL, "internal: %d channels on the tiled path", C);
    }
#undef BEVPOOL_PT
  } else if (vec) {
    const int64_t tiles_s = ceil_div(S, 256);
    const int passes = (C + 15) / 16;  // 16-channel passes per thread
#define BEVPOOL_PR(IT)                                                                         \
  hipLaunchKernelGGL((planar_rows_kernel<true, IT>), dim3(unsigned(int64_t(BN) * tiles_s)),     \
                     dim3(kThreads), 0, s, src, C, S, tiles_s, n_rows, stride_bn, stride_c, rows)
    if (passes <= 1) BEVPOOL_PR(1);
    else if (passes <= 2) BEVPOOL_PR(2);
    else if (passes <= 3) BEVPOOL_PR(3);
    else if (passes <= 5) BEVPOOL_PR(5);
    else BEVPOOL_PR(4);
#undef BEVPOOL_PR
  } else {
    hipLaunchKernelGGL((planar_rows_kernel<false, 1>),
                       dim3(unsigned(ceil_div(n_rows * C, kThreads))), dim3(kThreads), 0, s, src,
                       C, S, int64_t(0), n_rows, stride_bn, stride_c, rows);
  }
  return check_launch("planar_rows");
}

int bevpool_context_rows(const float *context, int64_t stride_bn, int64_t stride_c, int32_t BN,
                         int32_t C, int64_t HW, float *rows, void *stream) {
  return bevpool_planar_rows(context, stride_bn, stride_c, BN, C, HW, rows, stream);
}

int bevpool_backward_planar(const float *grad, int64_t grad_stride_b, int64_t grad_stride_c,
                            int64_t grad_stride_z, int32_t C, const int32_t *rank,
                            int64_t n_points, const int32_t *cell_start,
                            const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                            int64_t S, float *x_grad, int64_t x_stride_bn, int64_t x_stride_c,
                            void *scratch, size_t scratch_bytes, void *stream) {
  g_last_error.clear();
  if (C < 1) return fail(BEVPOOL_EINVAL, "C must be positive");
  if (n_batch < 1 || n_z < 1 || n_xy < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t n_cells = int64_t(n_batch) * n_z * n_xy;
  if (n_cells > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "too many cells");
  if (S < 1 || n_points < 0 || n_points > int64_t(INT32_MAX) || n_points % S != 0)
    return fail(BEVPOOL_EINVAL, "n_points must be a multiple of S");
  if (n_points == 0) return BEVPOOL_OK;
  if (!grad || !rank || !cell_start || !cell_end || !x_grad)
    return fail(BEVPOOL_EINVAL, "null argument");
  if (!scratch || scratch_bytes < bevpool_backward_scratch_bytes(n_cells, C, BEVPOOL_F32))
    return fail(BEVPOOL_ESPACE, "backward scratch too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = C % 4 == 0 && S % 4 == 0 && x_stride_bn % 4 == 0 && x_stride_c % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(x_grad) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(rank) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(scratch) % 16 == 0;
  int st;
  if ((st = check_grid(vec ? ceil_div(n_points / 4, kThreads) + kXcds
                           : ceil_div(n_points * C, kThreads),
                       kThreads, "gather_planar")))
    return st;
  if ((st = launch_bev_to_rows(grad, 4, grad_stride_b, grad_stride_c, grad_stride_z, C,
                               cell_start, cell_end, n_cells, n_z, n_xy, scratch, s)))
    return st;
  const float *g = static_cast<const float *>(scratch);
  LaunchTimer t("gather_planar", s);
  if (vec) {
    const unsigned grid = xcd_grid(ceil_div(n_points / 4, kThreads));
#ifndef BEVPOOL_GP_IT
#define BEVPOOL_GP_IT 2
#endif
    hipLaunchKernelGGL((gather_planar_kernel<true, BEVPOOL_GP_IT>), dim3(grid), dim3(kThreads),
                       0, s, g, C, rank, n_points, S, x_stride_bn, x_stride_c, x_grad);
  } else {
    hipLaunchKernelGGL((gather_planar_kernel<false, 1>),
                       dim3(unsigned(ceil_div(n_points * C, kThreads))), dim3(kThreads), 0, s, g,
                       C, rank, n_points, S, x_stride_bn, x_stride_c, x_grad);
  }
  return check_launch("gather_planar");
}

int bevpool_forward_depth(const float *depth, const float *context_rows, int32_t C,
                          int64_t n_points, int32_t D, int64_t HW, const uint64_t *keys,
                          const int32_t *cell_start, const int32_t *cell_end,
                          const int32_t *meta, int32_t n_batch, int32_t n_z, int64_t n_xy,
                          int64_t out_stride_b, int64_t out_stride_c, int64_t out_stride_z,
                          float *out, void *scratch, size_t scratch_bytes, void *stream) {
  g_last_error.clear();
  if (C < 1 || C % 4 != 0) return fail(BEVPOOL_EINVAL, "C must be a positive multiple of 4");
  if (D < 1 || HW < 1) return fail(BEVPOOL_EINVAL, "bad depth layout (D=%d, HW=%lld)", D,
                                   (long long)HW);
  if (n_batch < 1 || n_z < 1 || n_xy < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t n_cells = int64_t(n_batch) * n_z * n_xy;
  if (n_cells > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "too many cells");
  if (n_points < 0 || n_points > int64_t(INT32_MAX) || n_points % (int64_t(D) * HW) != 0)
    return fail(BEVPOOL_EINVAL, "n_points must be a multiple of D*HW");
  if (!out || !cell_start || !cell_end || !meta) return fail(BEVPOOL_EINVAL, "null argument");
  if (n_points > 0 && (!depth || !context_rows || !keys))
    return fail(BEVPOOL_EINVAL, "null depth/context/keys");
  if (reinterpret_cast<uintptr_t>(context_rows) % 16 != 0)
    return fail(BEVPOOL_EINVAL, "context rows must be 16-byte aligned");
  if (scratch_bytes < bevpool_forward_scratch_bytes(n_cells, C) || !scratch)
    return fail(BEVPOOL_ESPACE, "forward scratch too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float *acc = static_cast<float *>(scratch);
  int st;
  if (n_points > 0) {
    const DepthRows dr{depth, make_fast_div(uint32_t(HW)), make_fast_div(uint32_t(D))};
    st = launch_forward_pipe(BEVPOOL_F32, reinterpret_cast<const char *>(context_rows),
                             int64_t(C) * 4, C, n_points, keys, meta, cell_end, acc, dr, s);
    if (st) return st;
  }
  return launch_rows_to_bev(acc, BEVPOOL_F32, C, cell_start, cell_end, n_cells, n_z, n_xy,
                            out_stride_b, out_stride_c, out_stride_z, out, s);
}

int bevpool_backward_depth(const float *grad, int64_t grad_stride_b, int64_t grad_stride_c,
                           int64_t grad_stride_z, int32_t C, const int32_t *rank,
                           int64_t n_points, int32_t D, int64_t HW, const float *depth,
                           const float *context_rows, const int32_t *cell_start,
                           const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                           float *grad_depth, float *grad_context, int64_t gctx_stride_bn,
                           int64_t gctx_stride_c, void *scratch, size_t scratch_bytes,
                           void *stream) {
  g_last_error.clear();
  if (C < 1 || C > 256) return fail(BEVPOOL_EINVAL, "C must be in [1, 256]");
  if (D < 1 || HW < 1) return fail(BEVPOOL_EINVAL, "bad depth layout");
  if (n_batch < 1 || n_z < 1 || n_xy < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t n_cells = int64_t(n_batch) * n_z * n_xy;
  if (n_cells > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "too many cells");
  if (n_points < 0 || n_points > int64_t(INT32_MAX) || n_points % (int64_t(D) * HW) != 0)
    return fail(BEVPOOL_EINVAL, "n_points must be a multiple of D*HW");
  if (n_points == 0) return BEVPOOL_OK;
  if (!grad || !rank || !depth || !context_rows || !cell_start || !cell_end || !grad_depth ||
      !grad_context)
    return fail(BEVPOOL_EINVAL, "null argument");
  if (!scratch || scratch_bytes < bevpool_backward_scratch_bytes(n_cells, C, BEVPOOL_F32))
    return fail(BEVPOOL_ESPACE, "backward scratch too small");
  const int64_t n_pix = n_points / D;
  const size_t smem = size_t(2 * int64_t(D) + C) * kDgPix * sizeof(float);
  if (smem > 65536)
    return fail(BEVPOOL_EINVAL, "depth bins and channels too many (2*D + C = %lld > 1024)",
                (long long)(2 * int64_t(D) + C));
  hipStream_t s = static_cast<hipStream_t>(stream);
  int st;
  if ((st = check_grid(ceil_div(n_pix, kDgPix) + kXcds, kThreads, "depth_grad"))) return st;
  if ((st = launch_bev_to_rows(grad, 4, grad_stride_b, grad_stride_c, grad_stride_z, C,
                               cell_start, cell_end, n_cells, n_z, n_xy, scratch, s)))
    return st;
  const unsigned grid = xcd_grid(ceil_div(n_pix, kDgPix));
  LaunchTimer t("depth_grad", s);
  const float *g = static_cast<const float *>(scratch);
  uint32_t *gd = reinterpret_cast<uint32_t *>(grad_depth);
#define BEVPOOL_DG(K, U)                                                                       \
  hipLaunchKernelGGL((depth_grad_kernel<K, U>), dim3(grid), dim3(kThreads), smem, s, g, C,     \
                     rank, depth, context_rows, D, HW, n_pix, gd, grad_context, gctx_stride_bn, \
                     gctx_stride_c)
  const int kk = (C + 15) / 16;
  if (kk <= 1) BEVPOOL_DG(1, 8);
  else if (kk <= 2) BEVPOOL_DG(2, 8);
  else if (kk <= 3) BEVPOOL_DG(3, 8);
  else if (kk <= 4) BEVPOOL_DG(4, 8);
  else if (kk <= 5) BEVPOOL_DG(5, 8);
  else if (kk <= 6) BEVPOOL_DG(6, 8);
  else if (kk <= 8) BEVPOOL_DG(8, 4);
  else if (kk <= 12) BEVPOOL_DG(12, 4);
  else BEVPOOL_DG(16, 4);
#undef BEVPOOL_DG
  return check_launch("depth_grad");
}

size_t bevpool_backward_scratch_bytes(int64_t n_cells, int32_t C, int32_t dtype) {
  if (n_cells < 0 || C < 0) return 0;
  return size_t(n_cells) * size_t(C) * dtype_size(dtype);
}

int bevpool_backward(const void *grad, int32_t dtype, int64_t grad_stride_b,
                     int64_t grad_stride_c, int64_t grad_stride_z, int32_t C,
                     const int32_t *rank, int64_t n_points, const int32_t *cell_start,
                     const int32_t *cell_end, int32_t n_batch, int32_t n_z, int64_t n_xy,
                     void *x_grad, int64_t x_grad_row_stride, int32_t zero_dropped,
                     void *scratch, size_t scratch_bytes, void *stream) {
  g_last_error.clear();
  if (dtype != BEVPOOL_F32 && dtype != BEVPOOL_F16 && dtype != BEVPOOL_BF16)
    return fail(BEVPOOL_EINVAL, "unsupported dtype code %d", dtype);
  if (C < 1) return fail(BEVPOOL_EINVAL, "C must be positive");
  if (n_batch < 1 || n_z < 1 || n_xy < 1) return fail(BEVPOOL_EINVAL, "bad grid");
  const int64_t n_cells = int64_t(n_batch) * n_z * n_xy;
  if (n_cells > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "too many cells");
  if (n_points < 0 || n_points > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_points out of range");
  if (n_points == 0) return BEVPOOL_OK;
  if (!grad || !rank || !cell_start || !cell_end || !x_grad)
    return fail(BEVPOOL_EINVAL, "null argument");
  if (x_grad_row_stride < C) return fail(BEVPOOL_EINVAL, "bad x_grad row stride");
  if (!scratch || scratch_bytes < bevpool_backward_scratch_bytes(n_cells, C, dtype))
    return fail(BEVPOOL_ESPACE, "backward scratch too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t es = dtype_size(dtype);
  // gather layout (decided first: the warm-up blocks mirror it)
  const size_t row_bytes = size_t(C) * es;
  const bool vec16 = (row_bytes % 16 == 0) && ((size_t(x_grad_row_stride) * es) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(x_grad) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(scratch) % 16 == 0);
  const int vpr = vec16 ? int(row_bytes / 16) : int(C);
  const int64_t total = n_points * vpr;
  const int64_t gather_blocks = ceil_div(total, int64_t(kThreads) * kGatherPer);
  int st;
  if ((st = check_grid(gather_blocks + kXcds, kThreads, "gather_rows"))) return st;
  const unsigned grid = xcd_grid(gather_blocks);
  const bool narrow = total < (int64_t(1) << 32);
  // cache warm-up (gather_warm_block): ranks per XCD + occupied rows
  GatherWarm w{};
  int rank_blocks = 0;
  if (BEVPOOL_XCD_MAP && reinterpret_cast<uintptr_t>(rank) % 16 == 0 && n_points >= 4) {
    w.rank16 = reinterpret_cast<const u32x4 *>(rank);
    w.n16 = n_points / 4;
    w.xcd_span = int64_t(grid / kXcds) * kThreads * kGatherPer;
    w.vpr = vpr;
    const int64_t pts = ceil_div(w.xcd_span, int64_t(vpr)) + 1;
    w.per_xcd = int(ceil_div(ceil_div(pts, 4), int64_t(kThreads) * 16));  // <= 16 pieces/thread
    rank_blocks = kXcds * w.per_xcd;
  }
  int row_blocks = 0;
  if (BEVPOOL_XCD_MAP && vec16) {
    w.rows16 = static_cast<const u32x4 *>(scratch);
    w.rowq = vpr;
    row_blocks = int(ceil_div(n_cells, kWarmCells));
  }
  int warm_blocks = rank_blocks + row_blocks;
  warm_blocks = int(ceil_div(warm_blocks, kXcds) * kXcds);  // keep XCD parity
  if ((st = check_grid(int64_t(grid) + warm_blocks, kThreads, "gather_rows"))) return st;
  if ((st = launch_bev_to_rows(grad, es, grad_stride_b, grad_stride_c, grad_stride_z, C,
                               cell_start, cell_end, n_cells, n_z, n_xy, scratch, s)))
    return st;
  LaunchTimer t("gather_rows", s);
#define BEVPOOL_GATHER(V, NARROW, LD)                                                          \
  hipLaunchKernelGGL((gather_rows_kernel<V, NARROW>), dim3(grid + unsigned(warm_blocks)),      \
                     dim3(kThreads), 0, s, static_cast<const V *>(scratch), vpr, rank,        \
                     n_points, static_cast<V *>(x_grad), LD, warm_blocks, w, cell_start,     \
                     cell_end, n_cells, 0, zero_dropped ? 1 : 0)
  if (vec16) {
    const int64_t ld = int64_t(size_t(x_grad_row_stride) * es / 16);
    if (narrow) BEVPOOL_GATHER(u32x4, true, ld); else BEVPOOL_GATHER(u32x4, false, ld);
  } else if (es == 4) {
    if (narrow) BEVPOOL_GATHER(uint32_t, true, x_grad_row_stride);
    else BEVPOOL_GATHER(uint32_t, false, x_grad_row_stride);
  } else {
    if (narrow) BEVPOOL_GATHER(uint16_t, true, x_grad_row_stride);
    else BEVPOOL_GATHER(uint16_t, false, x_grad_row_stride);
  }
#undef BEVPOOL_GATHER
  return check_launch("gather_rows");
}

int bevpool_legacy_forward(const float *x, int64_t n, int32_t C, const int32_t *geom_feats,
                           const int32_t *interval_starts, const int32_t *interval_lengths,
                           int64_t n_intervals, const int32_t *n_intervals_dev, int32_t b,
                           int32_t d, int32_t h, int32_t w, float *out, int32_t *meta,
                           void *stream) {
  g_last_error.clear();
  int st = check_legacy_args(n, C, geom_feats, interval_starts, interval_lengths, n_intervals, b,
                             d, h, w, out);
  if (st) return st;
  if (n_intervals > 0 && n > 0 && !x) return fail(BEVPOOL_EINVAL, "null x");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t cells = int64_t(b) * d * h * w;
  if ((st = launch_zero_fill(out, size_t(cells) * size_t(C) * sizeof(float), s))) return st;
  if (n_intervals == 0) return BEVPOOL_OK;
  LaunchTimer t("legacy_forward", s);
#define BEVPOOL_LF(K)                                                                          \
  hipLaunchKernelGGL((legacy_forward_kernel<K>), dim3(legacy_grid(n_intervals)), dim3(kThreads), \
                     0, s, x, n, C, geom_feats, interval_starts, interval_lengths, n_intervals,  \
                     n_intervals_dev, b, d, h, w, out, meta)
  switch (legacy_cpl(C)) {
    case 1: BEVPOOL_LF(1); break;
    case 2: BEVPOOL_LF(2); break;
    default: BEVPOOL_LF(4); break;
  }
#undef BEVPOOL_LF
  return check_launch("legacy_forward");
}

int bevpool_legacy_backward(const float *out_grad, int64_t n, int32_t C,
                            const int32_t *geom_feats, const int32_t *interval_starts,
                            const int32_t *interval_lengths, int64_t n_intervals,
                            const int32_t *n_intervals_dev, int32_t b, int32_t d, int32_t h,
                            int32_t w, float *x_grad, int32_t *meta, void *stream) {
  g_last_error.clear();
  int st = check_legacy_args(n, C, geom_feats, interval_starts, interval_lengths, n_intervals, b,
                             d, h, w, n > 0 ? x_grad : reinterpret_cast<float *>(1));
  if (st) return st;
  if (n_intervals > 0 && !out_grad) return fail(BEVPOOL_EINVAL, "null out_grad");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_zero_fill(x_grad, size_t(n) * size_t(C) * sizeof(float), s))) return st;
  if (n_intervals == 0 || n == 0) return BEVPOOL_OK;
  LaunchTimer t("legacy_backward", s);
#define BEVPOOL_LB(K)                                                                          \
  hipLaunchKernelGGL((legacy_backward_kernel<K>), dim3(legacy_grid(n_intervals)),              \
                     dim3(kThreads), 0, s, out_grad, n, C, geom_feats, interval_starts,        \
                     interval_lengths, n_intervals, n_intervals_dev, b, d, h, w, x_grad, meta)
  switch (legacy_cpl(C)) {
    case 1: BEVPOOL_LB(1); break;
    case 2: BEVPOOL_LB(2); break;
    default: BEVPOOL_LB(4); break;
  }
#undef BEVPOOL_LB
  return check_launch("legacy_backward");
}

size_t bevpool_runs_workspace_bytes(int64_t n) {
  if (n < 0) return 0;
  return align256(size_t(ceil_div(n, kThreads) + 1) * sizeof(int32_t));
}

int bevpool_runs(const void *ranks, int32_t rank_bytes, int64_t n, int32_t *starts,
                 int32_t *lengths, int32_t *meta, void *workspace, size_t workspace_bytes,
                 void *stream) {
  g_last_error.clear();
  if (rank_bytes != 4 && rank_bytes != 8)
    return fail(BEVPOOL_EINVAL, "rank_bytes must be 4 or 8, got %d", rank_bytes);
  if (n < 0 || n > int64_t(INT32_MAX)) return fail(BEVPOOL_EINVAL, "n out of range");
  if (!meta || !workspace) return fail(BEVPOOL_EINVAL, "null meta or workspace");
  if (workspace_bytes < bevpool_runs_workspace_bytes(n))
    return fail(BEVPOOL_ESPACE, "runs workspace %zu bytes < required %zu", workspace_bytes,
                bevpool_runs_workspace_bytes(n));
  if (n > 0 && (!ranks || !starts || !lengths))
    return fail(BEVPOOL_EINVAL, "null ranks / starts / lengths");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int st;
  {
    LaunchTimer t("init_meta", s);
    hipLaunchKernelGGL(init_meta_kernel, dim3(1), dim3(64), 0, s, meta);
    if ((st = check_launch("init_meta"))) return st;
  }
  if (n == 0) return BEVPOOL_OK;
  const int64_t blocks = ceil_div(n, kThreads);
  if ((st = check_grid(blocks, kThreads, "runs"))) return st;
  int32_t *bcount = static_cast<int32_t *>(workspace);
  {
    LaunchTimer t("run_count", s);
    if (rank_bytes == 4)
      hipLaunchKernelGGL(run_count_kernel<int32_t>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int32_t *>(ranks), n, bcount);
    else
      hipLaunchKernelGGL(run_count_kernel<int64_t>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int64_t *>(ranks), n, bcount);
    if ((st = check_launch("run_count"))) return st;
  }
  {
    LaunchTimer t("scan_counts", s);
    hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(kThreads), 0, s, bcount, blocks,
                       meta + BEVPOOL_META_N_INTERVALS);
    if ((st = check_launch("scan_counts"))) return st;
  }
  {
    LaunchTimer t("run_write", s);
    if (rank_bytes == 4)
      hipLaunchKernelGGL(run_write_kernel<int32_t>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int32_t *>(ranks), n, bcount, starts);
    else
      hipLaunchKernelGGL(run_write_kernel<int64_t>, dim3(unsigned(blocks)), dim3(kThreads), 0, s,
                         static_cast<const int64_t *>(ranks), n, bcount, starts);
    if ((st = check_launch("run_write"))) return st;
  }
  LaunchTimer t("run_length", s);
  hipLaunchKernelGGL(run_length_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, s, starts, n,
                     meta + BEVPOOL_META_N_INTERVALS, lengths);
  return check_launch("run_length");
}


// Checks shared by the op-level entry points.
static int op_check_sizes(int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W,
                          int32_t C) {
  if (B < 1 || D < 1 || H < 1 || W < 1) return fail(BEVPOOL_EINVAL, "B, D, H, W must be positive");
  if (C < 1) return fail(BEVPOOL_EINVAL, "C must be positive");
  if (n_points < 0 || n_points > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "n_points=%lld out of range", (long long)n_points);
  if (int64_t(B) * D * H * W > int64_t(INT32_MAX))
    return fail(BEVPOOL_EINVAL, "B*D*H*W exceeds 2^31-1");
  return BEVPOOL_OK;
}

// bevpool_op_forward with the report destination already resolved to a
// device address (or null).
static int op_forward_impl(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                           const void *coords, int32_t coord_bytes, int64_t coords_row_stride,
                           int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W,
                           void *out, void *index, size_t index_bytes, void *scratch,
                           size_t scratch_bytes, int32_t *report_dev, void *stream) {
  if (int st = op_check_sizes(n_points, B, D, H, W, C)) return st;
  const int64_t cells = int64_t(B) * D * H * W;
  if (!index || !scratch) return fail(BEVPOOL_EINVAL, "null index or scratch buffer");
  const OpIndexLayout L = op_index_layout(n_points, cells);
  if (index_bytes < L.total)
    return fail(BEVPOOL_ESPACE, "op index buffer %zu bytes < required %zu", index_bytes, L.total);
  const OpScratchLayout S = op_scratch_layout(n_points, cells, C);
  if (scratch_bytes < S.total)
    return fail(BEVPOOL_ESPACE, "op scratch %zu bytes < required %zu", scratch_bytes, S.total);
  char *ix = static_cast<char *>(index);
  char *sc = static_cast<char *>(scratch);
  int32_t *meta = reinterpret_cast<int32_t *>(ix + L.meta);
  int32_t *rank = reinterpret_cast<int32_t *>(ix + L.rank);
  uint64_t *keys = reinterpret_cast<uint64_t *>(ix + L.keys);
  int32_t *cstart = reinterpret_cast<int32_t *>(ix + L.cstart);
  int32_t *cend = reinterpret_cast<int32_t *>(ix + L.cend);
  void *iws = sc + S.index_ws;
  const size_t iws_bytes = index_layout(n_points, cells).total;
  // meta is written by the first scatter (no separate initialising launch)
  int st = coord_ranks_impl(coords, coord_bytes, n_points, coords_row_stride, B, D, H, W, rank,
                            meta, iws, iws_bytes, stream, true);
  if (st) return st;
  if ((st = sort_impl(rank, n_points, cells, keys, cstart, cend, meta, iws, iws_bytes, stream,
                      true)))
    return st;
  const int64_t hw = int64_t(H) * W;
  MetaReport rep;
  rep.meta = meta;
  rep.dst = report_dev;
  return forward_impl(feats, dtype, feats_row_stride, C, n_points, keys, cstart, cend, meta, B, D,
                      hw, int64_t(C) * D * hw, int64_t(D) * hw, hw, out, sc + S.rows,
                      size_t(cells) * size_t(C) * sizeof(float), stream, rep);
}

size_t bevpool_op_index_bytes(int64_t n_points, int64_t n_cells) {
  if (n_points < 0 || n_cells < 0) return 0;
  return op_index_layout(n_points, n_cells).total;
}

size_t bevpool_op_scratch_bytes(int64_t n_points, int64_t n_cells, int32_t C) {
  if (n_points < 0 || n_cells < 0 || C < 0) return 0;
  return op_scratch_layout(n_points, n_cells, C).total;
}

size_t bevpool_op_workspace_bytes(int64_t n_points, int64_t n_cells, int32_t C) {
  if (n_points < 0 || n_cells < 0 || C < 0) return 0;
  return op_index_layout(n_points, n_cells).total + op_scratch_layout(n_points, n_cells, C).total;
}

int bevpool_op_forward(const void *feats, int32_t dtype, int64_t feats_row_stride, int32_t C,
                       const void *coords, int32_t coord_bytes, int64_t coords_row_stride,
                       int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W, void *out,
                       void *index, size_t index_bytes, void *scratch, size_t scratch_bytes,
                       int32_t *report, void *stream) {
  g_last_error.clear();
  int32_t *report_dev = nullptr;
  if (report) {
    if (int st = report_address(report, &report_dev)) return st;
  }
  return op_forward_impl(feats, dtype, feats_row_stride, C, coords, coord_bytes,
                         coords_row_stride, n_points, B, D, H, W, out, index, index_bytes,
                         scratch, scratch_bytes, report_dev, stream);
}

int bevpool_op_forward_noalloc(const void *feats, int32_t dtype, int64_t feats_row_stride,
                               int32_t C, const void *coords, int32_t coord_bytes,
                               int64_t coords_row_stride, int64_t n_points, int32_t B, int32_t D,
                               int32_t H, int32_t W, void *out, void *stream) {
  g_last_error.clear();
  if (int st = op_check_sizes(n_points, B, D, H, W, C)) return st;
  const int64_t cells = int64_t(B) * D * H * W;
  const size_t index_bytes = op_index_layout(n_points, cells).total;
  const size_t need = index_bytes + op_scratch_layout(n_points, cells, C).total;
  if (need > kNoAllocScratchBytes)
    return fail(BEVPOOL_ESPACE,
                "the allocation-free forward needs %zu bytes of scratch for n_points=%lld, "
                "B*D*H*W=%lld, C=%d; its static scratch holds %zu (use bevpool_op_forward)",
                need, (long long)n_points, (long long)cells, C, kNoAllocScratchBytes);
  char *ws = static_cast<char *>(noalloc_scratch());
  if (!ws) return BEVPOOL_EHIP;
  g_no_alloc_call = true;
  // index first (index_bytes is a multiple of 256), then the call's scratch
  const int st = op_forward_impl(feats, dtype, feats_row_stride, C, coords, coord_bytes,
                                 coords_row_stride, n_points, B, D, H, W, out, ws, index_bytes,
                                 ws + index_bytes, kNoAllocScratchBytes - index_bytes, nullptr,
                                 stream);
  g_no_alloc_call = false;
  return st;
}

int bevpool_op_backward(const void *grad, int32_t dtype, int64_t grad_stride_b,
                        int64_t grad_stride_c, int64_t grad_stride_z, int32_t C,
                        int64_t n_points, int32_t B, int32_t D, int32_t H, int32_t W,
                        void *x_grad, int64_t x_grad_row_stride, int32_t zero_dropped,
                        const void *index, size_t index_bytes, void *scratch,
                        size_t scratch_bytes, void *stream) {
  g_last_error.clear();
  if (int st = op_check_sizes(n_points, B, D, H, W, C)) return st;
  const int64_t cells = int64_t(B) * D * H * W;
  if (!index) return fail(BEVPOOL_EINVAL, "null index buffer");
  const OpIndexLayout L = op_index_layout(n_points, cells);
  if (index_bytes < L.total)
    return fail(BEVPOOL_ESPACE, "op index buffer %zu bytes < required %zu", index_bytes, L.total);
  const char *ix = static_cast<const char *>(index);
  return bevpool_backward(grad, dtype, grad_stride_b, grad_stride_c, grad_stride_z, C,
                          reinterpret_cast<const int32_t *>(ix + L.rank), n_points,
                          reinterpret_cast<const int32_t *>(ix + L.cstart),
                          reinterpret_cast<const int32_t *>(ix + L.cend), B, D, int64_t(H) * W,
                          x_grad, x_grad_row_stride, zero_dropped, scratch, scratch_bytes,
                          stream);
}

int bevpool_timing_enable(int enable) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing_enabled = enable != 0;
  return BEVPOOL_OK;
}

int bevpool_timing_reset(void) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (auto &r : g_timing_pending) {
    (void)hipEventSynchronize(r.stop);
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_timing_pending.clear();
  g_timing_totals.clear();
  return BEVPOOL_OK;
}

int bevpool_timing_read(char *names, int name_stride, double *total_ms, int64_t *launches,
                        int max_entries) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (auto &r : g_timing_pending) {
    if (hipEventSynchronize(r.stop) != hipSuccess)
      return fail(BEVPOOL_EHIP, "hipEventSynchronize failed");
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      return fail(BEVPOOL_EHIP, "hipEventElapsedTime failed");
    bool found = false;
    for (auto &kv : g_timing_totals) {
      if (kv.first == r.name) {
        kv.second.ms += ms;
        kv.second.launches += 1;
        found = true;
        break;
      }
    }
    if (!found) {
      TimingTotal tt;
      tt.ms = ms;
      tt.launches = 1;
      g_timing_totals.emplace_back(r.name, tt);
    }
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_timing_pending.clear();
  int n = 0;
  for (auto &kv : g_timing_totals) {
    if (n >= max_entries) break;
    if (names && name_stride > 0) {
      snprintf(names + size_t(n) * name_stride, size_t(name_stride), "%s", kv.first.c_str());
    }
    if (total_ms) total_ms[n] = kv.second.ms;
    if (launches) launches[n] = kv.second.launches;
    ++n;
  }
  return n;
}

}  // extern "C"
