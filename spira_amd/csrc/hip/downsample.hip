// Stride downsampling of packed voxel keys: sorted unique (key & stride mask).
//
// Reference semantics: torch/cuda_arg_sort_coordinates.cu:68-105 (mask every
// key with the per-axis stride mask, sort, unique) and :107-200 (one such
// downsample per target stride).
//
// Sorted input (the usual case: the keys of an ordered tensor) makes the
// masked keys sorted by their x field already: every run of keys with equal
// masked x ("segment") is contiguous, and only the (y, z) part inside a
// segment needs sorting.  The segmented path:
//   plan:    ds_tiles_kernel   per 1024-key tile: segment-start count, OR of
//                              the masked keys' varying bits, sortedness,
//                              longest segment starting in the tile;
//            ds_starts_kernel  segment starts in key order (one block per
//                              tile) + block 0 reduces the tiles into the plan;
//   (the host reads the plan: a few bytes)
//   execute: ds_segment_kernel one 1024-thread block per segment: the
//                              segment's varying bits as 32- or 64-bit sort
//                              keys in registers, stable LDS radix passes of
//                              8 bits (ballot-built peer masks for the ranks),
//                              then unique + compaction;
//            ds_offsets_kernel exclusive scan of the per-segment counts;
//            ds_copy_kernel    segments into the output.
// Unsorted input, or a segment longer than the largest block tile, takes the
// general path: mask, device-wide radix sort (rocPRIM), unique.
#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <rocprim/rocprim.hpp>

namespace spira_hip {

template <typename CT>
__global__ void mask_kernel(int64_t n, const CT *__restrict__ in, CT mask, CT *__restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = in[i] & mask;
}

template <typename CT> CT stride_mask(int sx, int sy, int sz) {
  // per-axis clear of the low log2(stride) bits (torch/cuda_arg_sort_coordinates.cu:86-89)
  CT xm = Layout<CT>::XONES & ~static_cast<CT>(static_cast<uint32_t>(sx - 1));
  CT ym = Layout<CT>::YONES & ~static_cast<CT>(static_cast<uint32_t>(sy - 1));
  CT zm = Layout<CT>::ZONES & ~static_cast<CT>(static_cast<uint32_t>(sz - 1));
  return static_cast<CT>((xm << Layout<CT>::XS) | (ym << Layout<CT>::YS) | zm);
}

// bits of the x field kept by the mask: a contiguous top range, so the keys
// of one segment are exactly the key interval [h, h | ~xmask]
template <typename CT> CT x_keep_mask(CT mask) {
  return mask & static_cast<CT>(Layout<CT>::XONES << Layout<CT>::XS);
}

static inline bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }
static inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

constexpr int kTile = 1024;       // keys per plan tile (256 threads x 4)
constexpr int kSegThreads = 1024;  // threads of a segment block

__global__ void zero_count_kernel(uint32_t *c) { *c = 0; }

// ---------------------------------------------------------------------------
// plan
// ---------------------------------------------------------------------------
template <typename CT>
__global__ __launch_bounds__(256) void ds_tiles_kernel(const CT *__restrict__ keys, int64_t n, CT mask, CT xmask,
                                                       uint32_t *__restrict__ tile_starts,
                                                       CT *__restrict__ tile_vary,
                                                       uint32_t *__restrict__ tile_flags) {
  __shared__ uint32_t s_cnt, s_unsorted, s_maxseg;
  __shared__ CT s_vary[4];
  const int tid = threadIdx.x;
  if (tid == 0) s_cnt = 0, s_unsorted = 0, s_maxseg = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  const CT m0 = keys[0] & mask;
  CT vary = 0;
  uint32_t cnt = 0, unsorted = 0, maxseg = 0;
#pragma unroll
  for (int j = 0; j < kTile / 256; ++j) {
    const int64_t i = base + j * 256 + tid;
    if (i < n) {
      const CT k = keys[i];
      vary |= (k & mask) ^ m0;
      const bool start = i == 0 || (keys[i - 1] & xmask) != (k & xmask);
      if (i > 0 && keys[i - 1] > k) unsorted = 1;
      if (start) {
        ++cnt;
        // segment end: first key above the segment's key interval (exact when
        // the keys are sorted; otherwise the plan is rejected on `unsorted`)
        const CT hi = (k & xmask) | static_cast<CT>(~xmask);
        int64_t lo = i + 1, up = n;
        while (lo < up) {
          const int64_t mid = (lo + up) >> 1;
          if (keys[mid] <= hi) lo = mid + 1; else up = mid;
        }
        const int64_t len = lo - i;
        const uint32_t l32 = len > 0x7FFFFFFF ? 0x7FFFFFFFu : static_cast<uint32_t>(len);
        maxseg = l32 > maxseg ? l32 : maxseg;
      }
    }
  }
  // block reductions
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    vary |= static_cast<CT>(__shfl_xor(vary, o, 64));
    cnt += __shfl_xor(cnt, o, 64);
    unsorted |= __shfl_xor(unsorted, o, 64);
    const uint32_t m = __shfl_xor(maxseg, o, 64);
    maxseg = m > maxseg ? m : maxseg;
  }
  if (lane_id() == 0) {
    s_vary[tid >> 6] = vary;
    atomicAdd(&s_cnt, cnt);
    atomicOr(&s_unsorted, unsorted);
    atomicMax(&s_maxseg, maxseg);
  }
  __syncthreads();
  if (tid == 0) {
    tile_starts[blockIdx.x] = s_cnt;
    tile_vary[blockIdx.x] = s_vary[0] | s_vary[1] | s_vary[2] | s_vary[3];
    tile_flags[2 * blockIdx.x] = s_unsorted;
    tile_flags[2 * blockIdx.x + 1] = s_maxseg;
  }
}

template <typename CT>
__global__ __launch_bounds__(256) void ds_starts_kernel(const CT *__restrict__ keys, int64_t n, CT xmask,
                                                        int64_t ntiles, const uint32_t *__restrict__ tile_starts,
                                                        const CT *__restrict__ tile_vary,
                                                        const uint32_t *__restrict__ tile_flags,
                                                        uint32_t *__restrict__ seg_start,
                                                        spira_hip_downsample_plan_t *__restrict__ plan) {
  __shared__ uint32_t s_wave[4][kTile / 256];
  __shared__ uint64_t s_red[4][4];
  const int tid = threadIdx.x, w = tid >> 6;
  const int64_t t = blockIdx.x;
  // segments starting before this tile
  uint64_t before = 0;
  for (int64_t u = tid; u < t; u += 256) before += tile_starts[u];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) before += __shfl_xor(before, o, 64);
  if (lane_id() == 0) s_red[0][w] = before;
  // starts of this tile, ranked in key order (round j, then wave, then lane)
  const int64_t base = t * kTile;
  bool st[kTile / 256];
  int pre[kTile / 256];
#pragma unroll
  for (int j = 0; j < kTile / 256; ++j) {
    const int64_t i = base + j * 256 + tid;
    st[j] = i < n && (i == 0 || (keys[i - 1] & xmask) != (keys[i] & xmask));
    const uint64_t b = ballot(st[j]);
    pre[j] = lane_prefix(b);
    if (lane_id() == 0) s_wave[w][j] = __popcll(b);
  }
  __syncthreads();
  const uint64_t off0 = s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3];
#pragma unroll
  for (int j = 0; j < kTile / 256; ++j) {
    if (!st[j]) continue;
    uint64_t off = off0;
    for (int jj = 0; jj < j; ++jj) off += s_wave[0][jj] + s_wave[1][jj] + s_wave[2][jj] + s_wave[3][jj];
    for (int ww = 0; ww < w; ++ww) off += s_wave[ww][j];
    seg_start[off + pre[j]] = static_cast<uint32_t>(base + j * 256 + tid);
  }
  if (t != 0) return;
  // block 0: the plan
  uint64_t nseg = 0;
  CT vary = 0;
  uint32_t unsorted = 0, maxseg = 0;
  for (int64_t u = tid; u < ntiles; u += 256) {
    nseg += tile_starts[u];
    vary |= tile_vary[u];
    unsorted |= tile_flags[2 * u];
    maxseg = tile_flags[2 * u + 1] > maxseg ? tile_flags[2 * u + 1] : maxseg;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    nseg += __shfl_xor(nseg, o, 64);
    vary |= static_cast<CT>(__shfl_xor(vary, o, 64));
    unsorted |= __shfl_xor(unsorted, o, 64);
    const uint32_t m = __shfl_xor(maxseg, o, 64);
    maxseg = m > maxseg ? m : maxseg;
  }
  __syncthreads();
  if (lane_id() == 0) {
    s_red[1][w] = nseg;
    s_red[2][w] = static_cast<uint64_t>(vary);
    s_red[3][w] = (static_cast<uint64_t>(unsorted) << 32) | maxseg;
  }
  __syncthreads();
  if (tid == 0) {
    uint64_t ns = 0, vy = 0;
    uint32_t us = 0, ms = 0;
    for (int q = 0; q < 4; ++q) {
      ns += s_red[1][q];
      vy |= s_red[2][q];
      us |= static_cast<uint32_t>(s_red[3][q] >> 32);
      const uint32_t m = static_cast<uint32_t>(s_red[3][q]);
      ms = m > ms ? m : ms;
    }
    plan->unsorted = us;
    plan->num_segments = static_cast<uint32_t>(ns);
    plan->max_segment = ms;
    plan->reserved = 0;
    plan->varying = vy;
    seg_start[ns] = static_cast<uint32_t>(n);
  }
}

// ---------------------------------------------------------------------------
// execute
// ---------------------------------------------------------------------------
template <typename KT> __device__ __forceinline__ uint32_t digit_of(KT k, int shift) {
  return static_cast<uint32_t>(k >> shift) & 255u;
}

// One block per segment.  Sort key: bits [lo, lo + nbits) of the masked key
// (the bits that vary over the whole input below the x field; every other
// bit is constant inside a segment).  Item j of lane l in wave w holds
// segment position w*C + j*64 + l (C = ITEMS*64): position order is
// (wave, round, lane), which the ranks keep (stable LSD passes).
template <typename CT, typename KT, int ITEMS>
__global__ __launch_bounds__(kSegThreads) void ds_segment_kernel(const CT *__restrict__ keys, CT mask, int lo,
                                                                 int nbits, const uint32_t *__restrict__ seg_start,
                                                                 CT *__restrict__ tmp,
                                                                 uint32_t *__restrict__ seg_count) {
  constexpr int W = kSegThreads / 64, C = ITEMS * 64;
  __shared__ KT buf[W * C];
  __shared__ uint32_t cnt[W][256];
  __shared__ uint32_t dbase[256];
  __shared__ uint32_t wsum[W];
  const int tid = threadIdx.x, w = tid >> 6, lane = lane_id();
  const int64_t s = blockIdx.x;
  const int64_t start = seg_start[s];
  const int len = static_cast<int>(seg_start[s + 1] - start);
  // rounds of this wave holding segment positions
  int rounds = (len - w * C + 63) >> 6;
  rounds = rounds < 0 ? 0 : (rounds > ITEMS ? ITEMS : rounds);
  const KT rmask = nbits >= static_cast<int>(8 * sizeof(KT)) ? static_cast<KT>(~KT(0))
                                                             : static_cast<KT>((KT(1) << nbits) - 1);
  KT key[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int p = w * C + j * 64 + lane;
    key[j] = p < len ? static_cast<KT>(((keys[start + p] & mask) >> lo)) & rmask : static_cast<KT>(~KT(0));
  }
  const int npass = (nbits + 7) >> 3;
  for (int pass = 0; pass < npass; ++pass) {
    const int shift = 8 * pass;
#pragma unroll
    for (int q = 0; q < 4; ++q) cnt[w][lane + 64 * q] = 0;
    uint32_t rank[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (j < rounds) {
        const uint32_t d = digit_of(key[j], shift);
        uint64_t peers = ~uint64_t(0);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const uint64_t bb = ballot((d >> b) & 1u);
          peers &= ((d >> b) & 1u) ? bb : ~bb;
        }
        const int lower = lane_prefix(peers);
        const uint32_t prev = cnt[w][d];
        rank[j] = prev + lower;
        if (lower == 0) cnt[w][d] = prev + __popcll(peers);
      }
    }
    __syncthreads();
    if (tid < 256) {
      // exclusive over waves per digit, then over digits
      uint32_t run = 0;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) {
        const uint32_t c = cnt[ww][tid];
        cnt[ww][tid] = run;
        run += c;
      }
      uint32_t inc = run;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
      }
      if (lane == 63) wsum[w] = inc;
      dbase[tid] = inc - run;
    }
    __syncthreads();
    if (tid < 256) {
      uint32_t add = 0;
      for (int ww = 0; ww < w; ++ww) add += wsum[ww];
      dbase[tid] += add;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (j < rounds) {
        const uint32_t d = digit_of(key[j], shift);
        buf[dbase[d] + cnt[w][d] + rank[j]] = key[j];
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j)
      if (j < rounds) key[j] = buf[w * C + j * 64 + lane];
    __syncthreads();
  }
  // unique + compaction in position order
  if (npass == 0) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j)
      if (j < rounds) buf[w * C + j * 64 + lane] = key[j];
    __syncthreads();
  }
  bool head[ITEMS];
  uint32_t total = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int p = w * C + j * 64 + lane;
    head[j] = j < rounds && p < len && (p == 0 || buf[p - 1] != key[j]);
    total += __popcll(ballot(head[j]));
  }
  if (lane == 0) wsum[w] = total;
  __syncthreads();
  uint32_t out = 0;
  for (int ww = 0; ww < w; ++ww) out += wsum[ww];
  const CT keep = static_cast<CT>(~(static_cast<CT>(rmask) << lo));
  const CT hi_bits = (keys[start] & mask) & keep;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint64_t b = ballot(head[j]);
    if (head[j]) tmp[start + out + lane_prefix(b)] = hi_bits | (static_cast<CT>(key[j]) << lo);
    out += __popcll(b);
  }
  if (tid == 0) {
    uint32_t all = 0;
    for (int ww = 0; ww < W; ++ww) all += wsum[ww];
    seg_count[s] = all;
  }
}

// exclusive scan of the segment counts (one block); total -> *d_count
__global__ __launch_bounds__(1024) void ds_offsets_kernel(const uint32_t *__restrict__ seg_count, int64_t nseg,
                                                          uint32_t *__restrict__ seg_off,
                                                          uint32_t *__restrict__ d_count) {
  __shared__ uint32_t wsum[16];
  __shared__ uint32_t carry;
  const int tid = threadIdx.x, w = tid >> 6, lane = lane_id();
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int64_t b = 0; b < nseg; b += 1024) {
    const int64_t i = b + tid;
    const uint32_t v = i < nseg ? seg_count[i] : 0;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t u = __shfl_up(inc, o, 64);
      if (lane >= o) inc += u;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    uint32_t add = carry;
    for (int ww = 0; ww < w; ++ww) add += wsum[ww];
    if (i < nseg) seg_off[i] = add + inc - v;
    __syncthreads();
    if (tid == 1023) carry = add + inc;
    __syncthreads();
  }
  if (tid == 0) *d_count = carry;
}

template <typename CT>
__global__ __launch_bounds__(256) void ds_copy_kernel(const CT *__restrict__ tmp,
                                                      const uint32_t *__restrict__ seg_start,
                                                      const uint32_t *__restrict__ seg_count,
                                                      const uint32_t *__restrict__ seg_off, CT *__restrict__ out) {
  const int64_t s = blockIdx.x;
  const int64_t src = seg_start[s], dst = seg_off[s];
  const uint32_t c = seg_count[s];
  for (uint32_t i = threadIdx.x; i < c; i += 256) out[dst + i] = tmp[src + i];
}

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------
template <typename CT> static size_t general_temp_bytes(int64_t n) {
  size_t sort_b = 0, uniq_b = 0;
  (void)rocprim::radix_sort_keys(nullptr, sort_b, static_cast<const CT *>(nullptr), static_cast<CT *>(nullptr),
                                 static_cast<size_t>(n), 0, 8 * sizeof(CT));
  (void)rocprim::unique(nullptr, uniq_b, static_cast<const CT *>(nullptr), static_cast<CT *>(nullptr),
                        static_cast<uint32_t *>(nullptr), static_cast<size_t>(n));
  return sort_b > uniq_b ? sort_b : uniq_b;
}

template <typename CT> struct DsParts {
  spira_hip_downsample_plan_t *plan;  // used by the one-call entry point
  uint32_t *tile_starts, *tile_flags, *seg_start, *seg_count, *seg_off;
  CT *tile_vary, *tmp;
  CT *masked, *sorted;  // general path
  void *temp;
  size_t temp_bytes, total;
};

template <typename CT> static DsParts<CT> ds_parts(int64_t n, void *base) {
  DsParts<CT> p{};
  const int64_t ntiles = div_up(n, kTile);
  char *b = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = b ? b + off : nullptr;
    off += align256(bytes);
    return q;
  };
  p.plan = reinterpret_cast<spira_hip_downsample_plan_t *>(take(sizeof(spira_hip_downsample_plan_t)));
  p.tile_starts = reinterpret_cast<uint32_t *>(take(ntiles * sizeof(uint32_t)));
  p.tile_flags = reinterpret_cast<uint32_t *>(take(2 * ntiles * sizeof(uint32_t)));
  p.tile_vary = reinterpret_cast<CT *>(take(ntiles * sizeof(CT)));
  p.seg_start = reinterpret_cast<uint32_t *>(take((n + 1) * sizeof(uint32_t)));
  p.seg_count = reinterpret_cast<uint32_t *>(take(n * sizeof(uint32_t)));
  p.seg_off = reinterpret_cast<uint32_t *>(take(n * sizeof(uint32_t)));
  p.tmp = reinterpret_cast<CT *>(take(n * sizeof(CT)));
  p.masked = reinterpret_cast<CT *>(take(n * sizeof(CT)));
  p.sorted = reinterpret_cast<CT *>(take(n * sizeof(CT)));
  p.temp_bytes = general_temp_bytes<CT>(n);
  p.temp = take(p.temp_bytes);
  p.total = off;
  return p;
}

template <typename CT>
static int check_args(int64_t n, int sx, int sy, int sz, void *ws, size_t ws_bytes, const char *who) {
  SPIRA_HIP_REQUIRE(n >= 0 && n < (int64_t(1) << 31), std::string(who) + ": n out of range");
  SPIRA_HIP_REQUIRE(is_pow2(sx) && is_pow2(sy) && is_pow2(sz), std::string(who) + ": strides must be powers of two");
  if (n > 0)
    SPIRA_HIP_REQUIRE(ws != nullptr && ws_bytes >= ds_parts<CT>(n, nullptr).total,
                      std::string(who) + ": workspace too small");
  return kOk;
}

template <typename CT>
static int plan_impl(const CT *keys, int64_t n, int sx, int sy, int sz, spira_hip_downsample_plan_t *plan_dev,
                     void *ws, size_t ws_bytes, hipStream_t s) {
  if (int rc = check_args<CT>(n, sx, sy, sz, ws, ws_bytes, "downsample_plan")) return rc;
  SPIRA_HIP_REQUIRE(plan_dev != nullptr, "downsample_plan: plan must not be null");
  SPIRA_HIP_REQUIRE(n > 0, "downsample_plan: no keys");
  DsParts<CT> p = ds_parts<CT>(n, ws);
  const CT mask = stride_mask<CT>(sx, sy, sz), xmask = x_keep_mask<CT>(mask);
  const int64_t ntiles = div_up(n, kTile);
  hipLaunchKernelGGL(ds_tiles_kernel<CT>, dim3(static_cast<unsigned>(ntiles)), dim3(256), 0, s, keys, n, mask,
                     xmask, p.tile_starts, p.tile_vary, p.tile_flags);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(ds_starts_kernel<CT>, dim3(static_cast<unsigned>(ntiles)), dim3(256), 0, s, keys, n, xmask,
                     ntiles, p.tile_starts, p.tile_vary, p.tile_flags, p.seg_start, plan_dev);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

template <typename CT, typename KT, int ITEMS>
static void launch_segments(const CT *keys, CT mask, int lo, int nbits, const DsParts<CT> &p, int64_t nseg,
                            hipStream_t s) {
  hipLaunchKernelGGL((ds_segment_kernel<CT, KT, ITEMS>), dim3(static_cast<unsigned>(nseg)), dim3(kSegThreads), 0, s,
                     keys, mask, lo, nbits, p.seg_start, p.tmp, p.seg_count);
}

// largest segment each (key type, items) variant holds: 1024 threads x ITEMS
template <typename CT>
static int execute_impl(const CT *keys, int64_t n, int sx, int sy, int sz, const spira_hip_downsample_plan_t *plan,
                        CT *out, uint32_t *d_count, void *ws, size_t ws_bytes, hipStream_t s) {
  if (int rc = check_args<CT>(n, sx, sy, sz, ws, ws_bytes, "downsample")) return rc;
  SPIRA_HIP_REQUIRE(d_count != nullptr, "downsample: count must not be null");
  if (n == 0) {
    hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, s, d_count);
    SPIRA_HIP_LAUNCH_CHECK();
    return kOk;
  }
  SPIRA_HIP_REQUIRE(plan != nullptr, "downsample: plan must not be null");
  DsParts<CT> p = ds_parts<CT>(n, ws);
  const CT mask = stride_mask<CT>(sx, sy, sz);
  const int64_t nseg = plan->num_segments;
  const uint64_t low = plan->varying & ((uint64_t(1) << Layout<CT>::XS) - 1);
  const int lo = low ? __builtin_ctzll(low) : 0;
  const int nbits = low ? 64 - __builtin_clzll(low) - lo : 0;
  const uint32_t ms = plan->max_segment;
  bool fast = !plan->unsorted && nseg >= 1 && nseg <= n;
  if (fast) {
    if (nbits <= 32) {
      if (ms <= 4 * kSegThreads)
        launch_segments<CT, uint32_t, 4>(keys, mask, lo, nbits, p, nseg, s);
      else if (ms <= 16 * kSegThreads)
        launch_segments<CT, uint32_t, 16>(keys, mask, lo, nbits, p, nseg, s);
      else if (ms <= 32 * kSegThreads)
        launch_segments<CT, uint32_t, 32>(keys, mask, lo, nbits, p, nseg, s);
      else
        fast = false;
    } else {
      if (ms <= 4 * kSegThreads)
        launch_segments<CT, uint64_t, 4>(keys, mask, lo, nbits, p, nseg, s);
      else if (ms <= 16 * kSegThreads)
        launch_segments<CT, uint64_t, 16>(keys, mask, lo, nbits, p, nseg, s);
      else
        fast = false;
    }
  }
  if (fast) {
    SPIRA_HIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(ds_offsets_kernel, dim3(1), dim3(1024), 0, s, p.seg_count, nseg, p.seg_off, d_count);
    SPIRA_HIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(ds_copy_kernel<CT>, dim3(static_cast<unsigned>(nseg)), dim3(256), 0, s, p.tmp, p.seg_start,
                       p.seg_count, p.seg_off, out);
    SPIRA_HIP_LAUNCH_CHECK();
    return kOk;
  }
  // general path
  hipLaunchKernelGGL(mask_kernel<CT>, dim3(div_up(n, 256)), dim3(256), 0, s, n, keys, mask, p.masked);
  SPIRA_HIP_LAUNCH_CHECK();
  size_t b = p.temp_bytes;
  SPIRA_HIP_TRY(rocprim::radix_sort_keys(p.temp, b, p.masked, p.sorted, static_cast<size_t>(n), 0, 8 * sizeof(CT), s));
  b = p.temp_bytes;
  SPIRA_HIP_TRY(rocprim::unique(p.temp, b, p.sorted, out, d_count, static_cast<size_t>(n), rocprim::equal_to<CT>(), s));
  return kOk;
}

template <typename CT>
static int downsample_impl(const CT *keys, int64_t n, int sx, int sy, int sz, CT *out, uint32_t *d_count, void *ws,
                           size_t ws_bytes, hipStream_t s) {
  if (int rc = check_args<CT>(n, sx, sy, sz, ws, ws_bytes, "downsample")) return rc;
  if (n == 0) return execute_impl<CT>(keys, n, sx, sy, sz, nullptr, out, d_count, ws, ws_bytes, s);
  DsParts<CT> p = ds_parts<CT>(n, ws);
  if (int rc = plan_impl<CT>(keys, n, sx, sy, sz, p.plan, ws, ws_bytes, s)) return rc;
  spira_hip_downsample_plan_t h{};
  SPIRA_HIP_TRY(hipMemcpyAsync(&h, p.plan, sizeof(h), hipMemcpyDeviceToHost, s));
  SPIRA_HIP_TRY(hipStreamSynchronize(s));
  return execute_impl<CT>(keys, n, sx, sy, sz, &h, out, d_count, ws, ws_bytes, s);
}

// ---------------------------------------------------------------------------
// chained downsample: a sorted key set to a chain of nested strides, each
// level computed from the previous level's output, with no host read.
//
// For stride b from a key set at stride a (b = a * r per axis, powers of two;
// level 1 takes a = 1): the keys of one output run (equal masked x and y)
// come from the r_x * r_y input rows (x0 + i a_x, y0 + j a_y), and inside one
// row the masked keys are non-decreasing (the row is sorted by z and masking
// z is monotone).  So the run's masked keys are a merge of r_x r_y sorted
// rows: each key's place is the run's start (the number of keys of earlier
// runs) plus its index in its own row plus, per other row of the run, the
// number of that row's keys ordered before it (ties go to the earlier row);
// all by binary searches over the sorted input.  Duplicates are then
// adjacent: a scan of the run starts (computed from the merged keys as the
// scan reads them) and a compaction leave the sorted unique keys.
// ---------------------------------------------------------------------------
constexpr int kChainMaxRows = 16;  // input rows per output run and level

template <typename CT>
__device__ __forceinline__ int64_t key_lower_bound(const CT *__restrict__ a, int64_t lo, int64_t hi, CT v) {
  while (lo < hi) {
    const int64_t m = (lo + hi) >> 1;
    if (a[m] < v) lo = m + 1;
    else hi = m;
  }
  return lo;
}

// first position in [lo, hi) whose masked key is >= v (UPPER: > v); the
// masked keys of the range are non-decreasing
template <typename CT, bool UPPER>
__device__ __forceinline__ int64_t masked_bound(const CT *__restrict__ a, int64_t lo, int64_t hi, CT mask, CT v) {
  while (lo < hi) {
    const int64_t m = (lo + hi) >> 1;
    const CT w = a[m] & mask;
    if (UPPER ? (w <= v) : (w < v)) lo = m + 1;
    else hi = m;
  }
  return lo;
}

// key of (x, y, 0); x or y past its field: one past every key of the
// previous x (or of all keys)
template <typename CT> __device__ __forceinline__ bool row_key(uint64_t x, uint64_t y, CT &k) {
  if (y > Layout<CT>::YONES) {
    ++x;
    y = 0;
  }
  if (x > Layout<CT>::XONES) return false;
  k = static_cast<CT>((static_cast<CT>(x) << Layout<CT>::XS) | (static_cast<CT>(y) << Layout<CT>::YS));
  return true;
}

template <typename CT>
__device__ __forceinline__ int64_t lb_row(const CT *__restrict__ in, int64_t lo, int64_t n, uint64_t x, uint64_t y) {
  CT k;
  return row_key<CT>(x, y, k) ? key_lower_bound(in, lo, n, k) : n;
}

// Rank of key i in its output run by binary searches over the whole input
// (any ratios); -1 if the ranks cannot be formed (unsorted input).
template <typename CT>
__device__ int64_t chain_rank_search(const CT *__restrict__ in, int64_t n, int64_t i, CT key, CT mask, uint32_t ax,
                                     uint32_t ay, int rx, int ry) {
  const CT k = key & mask;
  const uint64_t x = static_cast<uint64_t>((key >> Layout<CT>::XS) & Layout<CT>::XONES);
  const uint64_t y = static_cast<uint64_t>((key >> Layout<CT>::YS) & Layout<CT>::YONES);
  const uint64_t x0 = x & ~(static_cast<uint64_t>(ax) * rx - 1);
  const uint64_t y0 = y & ~(static_cast<uint64_t>(ay) * ry - 1);
  const int own = static_cast<int>((x - x0) / ax) * ry + static_cast<int>((y - y0) / ay);
  // rows of the run in key order: q = ix * ry + iy, [rs[q], re[q])
  int64_t rs[kChainMaxRows], re[kChainMaxRows];
  int64_t pos = lb_row<CT>(in, 0, n, x0, 0);  // keys of columns before x0
  int64_t col = pos;
  for (int ix = 0; ix < rx; ++ix) {
    const uint64_t xi = x0 + static_cast<uint64_t>(ix) * ax;
    const int64_t cs = ix == 0 ? col : lb_row<CT>(in, col, n, xi, 0);
    int64_t b = lb_row<CT>(in, cs, n, xi, y0);
    pos += b - cs;  // keys of column xi with y < y0 (earlier runs)
    for (int iy = 0; iy < ry; ++iy) {
      const int q = ix * ry + iy;
      rs[q] = b;
      b = lb_row<CT>(in, b, n, xi, y0 + static_cast<uint64_t>(iy + 1) * ay);
      re[q] = b;
    }
    col = cs;
  }
  int64_t rank = pos + (i - rs[own]);
  const int nrows = rx * ry;
  for (int q = 0; q < nrows; ++q) {
    if (q < own) rank += masked_bound<CT, true>(in, rs[q], re[q], mask, k) - rs[q];
    else if (q > own) rank += masked_bound<CT, false>(in, rs[q], re[q], mask, k) - rs[q];
  }
  return rank;
}

template <typename CT>
__global__ __launch_bounds__(256) void chain_merge_kernel(const CT *__restrict__ in, const uint32_t *__restrict__ n_dev,
                                                          int64_t n_cap, CT mask, uint32_t ax, uint32_t ay, int rx,
                                                          int ry, CT *__restrict__ merged,
                                                          uint32_t *__restrict__ unsorted) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
  if (i >= n) return;
  const CT key = in[i];
  if (unsorted && i > 0 && in[i - 1] > key) atomicOr(unsorted, 1u);
  const CT k = key & mask;
  if (rx == 1 && ry == 1) {  // one row per run: the masked keys are in order already
    merged[i] = k;
    return;
  }
  const int64_t rank = chain_rank_search<CT>(in, n, i, key, mask, ax, ay, rx, ry);
  // A sorted input makes the ranks a permutation of [0, n); unsorted input
  // (reported through `unsorted` at level 1) can push them out of range, and
  // such a key is dropped rather than written out of bounds.
  if (rank < 0 || rank >= n) {
    if (unsorted) atomicOr(unsorted, 1u);
    return;
  }
  merged[rank] = k;
}

// ----- x-tables: the columns (keys of one x) of a level's sorted input
//
// xs[c] / xe[c] = first / one-past-last position of column x = xmin + c * ax
// (xmin: the x of the first key, ax: the level's input stride), for c <
// kXtCap.  Only present columns are written; a reader accepts an entry only
// if the keys around its two ends show that it bounds exactly column x, so
// stale entries (absent columns, earlier levels) are never used.  With
// sorted input the entries of present columns are always fresh.
constexpr int64_t kXtCap = int64_t(1) << 16;

template <typename CT> __device__ __forceinline__ uint64_t key_x(CT k) {
  return static_cast<uint64_t>((k >> Layout<CT>::XS) & Layout<CT>::XONES);
}

// table slot of column x, or -1 (x below xmin, off the stride grid, past
// the table)
__device__ __forceinline__ int64_t xt_slot(uint64_t x, uint64_t xmin, uint32_t ax) {
  if (x < xmin) return -1;
  const uint64_t d = x - xmin;
  if (d % ax != 0) return -1;
  const uint64_t c = d / ax;
  return c < static_cast<uint64_t>(kXtCap) ? static_cast<int64_t>(c) : -1;
}

// the level-1 table from the input keys (stride 1)
template <typename CT>
__global__ __launch_bounds__(256) void chain_xtable_kernel(const CT *__restrict__ in, int64_t n,
                                                           int32_t *__restrict__ xs, int32_t *__restrict__ xe) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t x = key_x(in[i]);
  const int64_t c = xt_slot(x, key_x(in[0]), 1u);
  if (c < 0) return;
  if (i == 0 || key_x(in[i - 1]) != x) xs[c] = static_cast<int32_t>(i);
  if (i == n - 1 || key_x(in[i + 1]) != x) xe[c] = static_cast<int32_t>(i + 1);
}

// Column x of `in` from the table: true with [c, e) if the table holds it.
template <typename CT>
__device__ __forceinline__ bool xt_column(const CT *__restrict__ in, int64_t n, const int32_t *__restrict__ xs,
                                          const int32_t *__restrict__ xe, int64_t slot, uint64_t x, int64_t &c,
                                          int64_t &e) {
  c = xs[slot];
  e = xe[slot];
  if (c < 0 || c >= n || e <= c || e > n) return false;
  if (key_x(in[c]) != x || (c > 0 && key_x(in[c - 1]) == x)) return false;
  return key_x(in[e - 1]) == x && (e == n || key_x(in[e]) != x);
}

// First position in [lo, hi) whose key is >= v, for two ranges at once
// (their loads overlap).  With GALLOP the probes first step from lo in
// doubling strides (the answer is expected near lo: a row's end from its
// start), then bisect once a probe reaches v; the answer stays in
// [lo, lo + len] and len shrinks every round.
template <typename CT, bool GALLOP>
__device__ __forceinline__ void lower_bound2(const CT *__restrict__ a, int64_t (&lo)[2], const int64_t (&hi)[2],
                                             const CT (&v)[2]) {
  int64_t len[2] = {hi[0] - lo[0], hi[1] - lo[1]};
  int64_t step[2] = {GALLOP ? 1 : 0, GALLOP ? 1 : 0};  // 0: bisecting
  while (len[0] > 0 || len[1] > 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (len[t] > 0) {
        const int64_t h = step[t] > 0 ? (step[t] < len[t] ? step[t] : len[t]) - 1 : len[t] >> 1;
        if (a[lo[t] + h] < v[t]) {
          lo[t] += h + 1;
          len[t] -= h + 1;
          step[t] <<= 1;
        } else {
          len[t] = h;
          step[t] = 0;
        }
      }
    }
  }
}

// Per row q of a run [rs[q], re[q]) (masked keys non-decreasing): the
// number of keys ordered before masked key k of row `own` (ties go to the
// earlier row), all four rows' galloping searches side by side.
template <typename CT>
__device__ __forceinline__ int64_t masked_counts4(const CT *__restrict__ a, const int64_t (&rs)[4],
                                                  const int64_t (&re)[4], int own, CT mask, CT k) {
  int64_t lo[4], len[4], step[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    lo[q] = rs[q];
    len[q] = q == own ? 0 : re[q] - rs[q];
    step[q] = 1;
  }
  while (len[0] > 0 || len[1] > 0 || len[2] > 0 || len[3] > 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (len[q] > 0) {
        const int64_t h = step[q] > 0 ? (step[q] < len[q] ? step[q] : len[q]) - 1 : len[q] >> 1;
        const CT w = a[lo[q] + h] & mask;
        if (q < own ? (w <= k) : (w < k)) {
          lo[q] += h + 1;
          len[q] -= h + 1;
          step[q] <<= 1;
        } else {
          len[q] = h;
          step[q] = 0;
        }
      }
    }
  }
  int64_t c = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) c += q == own ? 0 : lo[q] - rs[q];
  return c;
}

// Level merge for x and y ratios of 2 (the networks' chains): the run's four
// rows are found inside their columns, which the x-table gives, with the two
// columns searched side by side; a key whose columns lie past the table
// takes the whole-input searches.
template <typename CT>
__global__ __launch_bounds__(256) void chain_merge2_kernel(const CT *__restrict__ in, const uint32_t *__restrict__ n_dev,
                                                           int64_t n_cap, CT mask, uint32_t ax, uint32_t ay,
                                                           const int32_t *__restrict__ xs,
                                                           const int32_t *__restrict__ xe, CT *__restrict__ merged,
                                                           uint32_t *__restrict__ unsorted) {
  constexpr int RX = 2, RY = 2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
  if (i >= n) return;
  const CT key = in[i];
  if (unsorted && i > 0 && in[i - 1] > key) atomicOr(unsorted, 1u);
  const CT k = key & mask;
  const uint64_t x = key_x(key);
  const uint64_t y = static_cast<uint64_t>((key >> Layout<CT>::YS) & Layout<CT>::YONES);
  const uint64_t x0 = x & ~(static_cast<uint64_t>(ax) * RX - 1);
  const uint64_t y0 = y & ~(static_cast<uint64_t>(ay) * RY - 1);
  const int oxi = static_cast<int>((x - x0) / ax);
  const int own = oxi * RY + static_cast<int>((y - y0) / ay);
  const uint64_t xmin = key_x(in[0]);
  int64_t cs[RX] = {0, 0}, ce[RX] = {0, 0};
  bool present[RX] = {false, false};
  bool known = true;
#pragma unroll
  for (int ix = 0; ix < RX; ++ix) {
    const uint64_t xi = x0 + static_cast<uint64_t>(ix) * ax;
    if (xi < xmin) continue;  // below the first key: absent
    const int64_t slot = xt_slot(xi, xmin, ax);
    if (slot < 0) {
      known = false;
      continue;
    }
    present[ix] = xt_column<CT>(in, n, xs, xe, slot, xi, cs[ix], ce[ix]);
    if (!present[ix]) cs[ix] = ce[ix] = 0;
  }
  int64_t rank;
  if (!known) {
    rank = chain_rank_search<CT>(in, n, i, key, mask, ax, ay, RX, RY);
  } else if (!present[oxi]) {
    rank = -1;  // the key's own column is not where sorted input puts it
  } else {
    int64_t b[RX] = {cs[0], cs[1]};
    CT v[RX];
#pragma unroll
    for (int ix = 0; ix < RX; ++ix)
      v[ix] = static_cast<CT>(((x0 + static_cast<uint64_t>(ix) * ax) << Layout<CT>::XS) | (y0 << Layout<CT>::YS));
    lower_bound2<CT, false>(in, b, ce, v);  // absent columns: empty ranges
    int64_t pos = present[0] ? cs[0] : cs[1];  // keys of columns before x0
#pragma unroll
    for (int ix = 0; ix < RX; ++ix) pos += b[ix] - cs[ix];  // keys of column xi with y < y0
    int64_t rs[RX * RY], re[RX * RY];
#pragma unroll
    for (int iy = 0; iy < RY; ++iy) {
      const uint64_t yn = y0 + static_cast<uint64_t>(iy + 1) * ay;
#pragma unroll
      for (int ix = 0; ix < RX; ++ix) {
        rs[ix * RY + iy] = b[ix];
        v[ix] = static_cast<CT>(((x0 + static_cast<uint64_t>(ix) * ax) << Layout<CT>::XS) |
                                ((yn > Layout<CT>::YONES ? 0 : yn) << Layout<CT>::YS));
      }
      if (yn > Layout<CT>::YONES) {
#pragma unroll
        for (int ix = 0; ix < RX; ++ix) b[ix] = ce[ix];  // the rows run to the column's end
      } else {
        lower_bound2<CT, true>(in, b, ce, v);
      }
#pragma unroll
      for (int ix = 0; ix < RX; ++ix) re[ix * RY + iy] = b[ix];
    }
    rank = pos + (i - rs[own]) + masked_counts4<CT>(in, rs, re, own, mask, k);
  }
  if (rank < 0 || rank >= n) {
    if (unsorted) atomicOr(unsorted, 1u);
    return;
  }
  merged[rank] = k;
}

// Merged key p starts a run of equal keys (the unique keys of the level):
// read by the scan straight from the merged keys and again by the
// compaction, so no flag array is written.
template <typename CT> struct ChainFirst {
  const CT *merged;
  const uint32_t *n_dev;
  int64_t n_cap;
  __host__ __device__ uint32_t operator()(int64_t p) const {
    const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
    return (p < n && (p == 0 || merged[p] != merged[p - 1])) ? 1u : 0u;
  }
};
template <typename CT>
using ChainFlags = rocprim::transform_iterator<rocprim::counting_iterator<int64_t>, ChainFirst<CT>, uint32_t>;

// Unique keys to the level's output, and the next level's x-table (stride
// ax_next) from the merged keys: a column starts at the first unique key of
// a new x and ends after the last merged key of that x.
template <typename CT>
__global__ __launch_bounds__(256) void chain_compact_kernel(const CT *__restrict__ merged,
                                                            const uint32_t *__restrict__ pos,
                                                            const uint32_t *__restrict__ n_dev, int64_t n_cap,
                                                            CT *__restrict__ out, uint32_t *__restrict__ count,
                                                            uint32_t ax_next, int32_t *__restrict__ xs,
                                                            int32_t *__restrict__ xe) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n_cap) return;
  const uint32_t flag = ChainFirst<CT>{merged, n_dev, n_cap}(p);
  if (flag) out[pos[p]] = merged[p];
  if (p == n_cap - 1) *count = pos[p] + flag;
  const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
  if (!xs || p >= n) return;
  const uint64_t x = key_x(merged[p]);
  const int64_t c = xt_slot(x, key_x(merged[0]), ax_next);
  if (c < 0) return;
  if (flag && (p == 0 || key_x(merged[p - 1]) != x)) xs[c] = static_cast<int32_t>(pos[p]);
  if (p == n - 1 || key_x(merged[p + 1]) != x) xe[c] = static_cast<int32_t>(pos[p] + flag);
}

// Compaction without a device-wide scan (inputs of at most kCompactMaxTiles
// tiles): chain_count_kernel counts the run starts of each 2048-key tile;
// chain_compact2_kernel sums the counts of the tiles before its own (at most
// a few per thread), scans its tile in the block, and writes what
// chain_compact_kernel writes.
constexpr int kCompactTile = 2048;
constexpr int kCompactItems = kCompactTile / 256;
constexpr int64_t kCompactMaxTiles = 1024;

// merged[p0 - 1 .. p0 + kCompactItems] (entries outside [0, n_cap): 0)
template <typename CT>
__device__ __forceinline__ void load_run(const CT *__restrict__ merged, int64_t n_cap, int64_t p0,
                                         CT (&m)[kCompactItems + 2]) {
#pragma unroll
  for (int r = 0; r < kCompactItems + 2; ++r) {
    const int64_t p = p0 - 1 + r;
    const bool in = p >= 0 && p < n_cap;
    const CT v = merged[in ? p : 0];
    m[r] = in ? v : CT(0);
  }
}

template <typename CT>
__global__ __launch_bounds__(256) void chain_count_kernel(const CT *__restrict__ merged,
                                                          const uint32_t *__restrict__ n_dev, int64_t n_cap,
                                                          uint32_t *__restrict__ tile_counts) {
  __shared__ uint32_t red[4];
  const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kCompactTile + threadIdx.x * kCompactItems;
  CT m[kCompactItems + 2];
  load_run<CT>(merged, n_cap, p0, m);
  uint32_t c = 0;
#pragma unroll
  for (int r = 0; r < kCompactItems; ++r) {
    const int64_t p = p0 + r;
    c += (p < n && (p == 0 || m[r + 1] != m[r])) ? 1u : 0u;
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) c += __shfl_xor(c, d, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) tile_counts[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

template <typename CT>
__global__ __launch_bounds__(256) void chain_compact2_kernel(const CT *__restrict__ merged,
                                                             const uint32_t *__restrict__ tile_counts,
                                                             const uint32_t *__restrict__ n_dev, int64_t n_cap,
                                                             CT *__restrict__ out, uint32_t *__restrict__ count,
                                                             uint32_t ax_next, int32_t *__restrict__ xs,
                                                             int32_t *__restrict__ xe) {
  __shared__ uint32_t before[4], wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t n = n_dev ? static_cast<int64_t>(*n_dev) : n_cap;
  // run starts of the tiles before this one
  uint32_t b = 0;
  for (int t = tid; t < static_cast<int>(blockIdx.x); t += 256) b += tile_counts[t];
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) b += __shfl_xor(b, d, 64);
  // this thread's keys and run starts
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kCompactTile + tid * kCompactItems;
  CT m[kCompactItems + 2];
  load_run<CT>(merged, n_cap, p0, m);
  bool f[kCompactItems];
  uint32_t c = 0;
#pragma unroll
  for (int r = 0; r < kCompactItems; ++r) {
    const int64_t p = p0 + r;
    f[r] = p < n && (p == 0 || m[r + 1] != m[r]);
    c += f[r] ? 1u : 0u;
  }
  // exclusive prefix of c over the block
  uint32_t incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wtot[w] = incl;
  if (lane == 0) before[w] = b;
  __syncthreads();
  uint32_t pos = before[0] + before[1] + before[2] + before[3] + incl - c;
  for (int q = 0; q < w; ++q) pos += wtot[q];
  const uint64_t xmin = key_x(merged[0]);
#pragma unroll
  for (int r = 0; r < kCompactItems; ++r) {
    const int64_t p = p0 + r;
    if (f[r]) out[pos] = m[r + 1];
    if (p == n_cap - 1) *count = pos + (f[r] ? 1u : 0u);
    if (xs && p < n) {
      const uint64_t x = key_x(m[r + 1]);
      const int64_t cx = xt_slot(x, xmin, ax_next);
      if (cx >= 0) {
        if (f[r] && (p == 0 || key_x(m[r]) != x)) xs[cx] = static_cast<int32_t>(pos);
        if (p == n - 1 || key_x(m[r + 2]) != x) xe[cx] = static_cast<int32_t>(pos + (f[r] ? 1u : 0u));
      }
    }
    pos += f[r] ? 1u : 0u;
  }
}

template <typename CT> static size_t chain_scan_bytes(int64_t n) {
  size_t b = 0;
  const ChainFlags<CT> flags(rocprim::counting_iterator<int64_t>(0), ChainFirst<CT>{nullptr, nullptr, n});
  (void)rocprim::exclusive_scan(nullptr, b, flags, static_cast<uint32_t *>(nullptr), 0u, static_cast<size_t>(n),
                                rocprim::plus<uint32_t>());
  return b;
}

template <typename CT> struct ChainParts {
  CT *merged;
  uint32_t *pos;
  int32_t *xs, *xe;  // x-table of the current level's input
  void *temp;
  size_t temp_bytes, total;
};

template <typename CT> static ChainParts<CT> chain_parts(int64_t n, void *base) {
  ChainParts<CT> p{};
  char *b = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = b ? b + off : nullptr;
    off += align256(bytes);
    return q;
  };
  p.merged = reinterpret_cast<CT *>(take(n * sizeof(CT)));
  p.pos = reinterpret_cast<uint32_t *>(take(n * sizeof(uint32_t)));
  p.xs = reinterpret_cast<int32_t *>(take(kXtCap * sizeof(int32_t)));
  p.xe = reinterpret_cast<int32_t *>(take(kXtCap * sizeof(int32_t)));
  p.temp_bytes = chain_scan_bytes<CT>(n);
  p.temp = take(p.temp_bytes);
  p.total = off;
  return p;
}

// a level's stride ratio on one axis; 0 if the strides do not chain
static int chain_ratio(int prev, int cur) {
  if (!is_pow2(prev) || !is_pow2(cur) || cur % prev != 0) return 0;
  return cur / prev;
}

template <typename CT>
static int chain_impl(const CT *keys, int64_t n, int levels, const int32_t *strides, void *const *outs,
                      uint32_t *d_counts, uint32_t *d_unsorted, void *ws, size_t ws_bytes, hipStream_t s) {
  SPIRA_HIP_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "downsample_chain: n out of range");
  SPIRA_HIP_REQUIRE(levels >= 1 && strides && outs && d_counts && d_unsorted, "downsample_chain: bad arguments");
  int prev[3] = {1, 1, 1};
  for (int l = 0; l < levels; ++l) {
    int r[3];
    for (int a = 0; a < 3; ++a) {
      r[a] = chain_ratio(prev[a], strides[3 * l + a]);
      prev[a] = strides[3 * l + a];
    }
    SPIRA_HIP_REQUIRE(r[0] > 0 && r[1] > 0 && r[2] > 0 && r[0] * r[1] <= kChainMaxRows,
                      "downsample_chain: each stride must be a power of two and a multiple of the previous one, "
                      "with at most 16 input rows (x ratio times y ratio) per output run");
    SPIRA_HIP_REQUIRE(outs[l] != nullptr, "downsample_chain: missing output array");
  }
  if (n == 0) {
    for (int l = 0; l < levels; ++l) hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, s, d_counts + l);
    SPIRA_HIP_LAUNCH_CHECK();
    return kOk;
  }
  SPIRA_HIP_REQUIRE(ws != nullptr && ws_bytes >= chain_parts<CT>(n, nullptr).total,
                    "downsample_chain: workspace too small");
  ChainParts<CT> p = chain_parts<CT>(n, ws);
  const dim3 grid(static_cast<unsigned>(div_up(n, 256)));
  hipLaunchKernelGGL(chain_xtable_kernel<CT>, grid, dim3(256), 0, s, keys, n, p.xs, p.xe);
  SPIRA_HIP_LAUNCH_CHECK();
  int a[3] = {1, 1, 1};
  for (int l = 0; l < levels; ++l) {
    const int *b = strides + 3 * l;
    const CT *in = l == 0 ? keys : static_cast<const CT *>(outs[l - 1]);
    const uint32_t *n_dev = l == 0 ? nullptr : d_counts + (l - 1);
    const CT mask = stride_mask<CT>(b[0], b[1], b[2]);
    if (b[0] / a[0] == 2 && b[1] / a[1] == 2)
      hipLaunchKernelGGL(chain_merge2_kernel<CT>, grid, dim3(256), 0, s, in, n_dev, n, mask,
                         static_cast<uint32_t>(a[0]), static_cast<uint32_t>(a[1]), p.xs, p.xe, p.merged,
                         l == 0 ? d_unsorted : nullptr);
    else
      hipLaunchKernelGGL(chain_merge_kernel<CT>, grid, dim3(256), 0, s, in, n_dev, n, mask,
                         static_cast<uint32_t>(a[0]), static_cast<uint32_t>(a[1]), b[0] / a[0], b[1] / a[1], p.merged,
                         l == 0 ? d_unsorted : nullptr);
    SPIRA_HIP_LAUNCH_CHECK();
    const int64_t ctiles = div_up(n, kCompactTile);
    if (ctiles <= kCompactMaxTiles) {
      // (the tile counts take the front of the positions array)
      hipLaunchKernelGGL(chain_count_kernel<CT>, dim3(static_cast<unsigned>(ctiles)), dim3(256), 0, s, p.merged,
                         n_dev, n, p.pos);
      SPIRA_HIP_LAUNCH_CHECK();
      hipLaunchKernelGGL(chain_compact2_kernel<CT>, dim3(static_cast<unsigned>(ctiles)), dim3(256), 0, s, p.merged,
                         p.pos, n_dev, n, static_cast<CT *>(outs[l]), d_counts + l, static_cast<uint32_t>(b[0]), p.xs,
                         p.xe);
      SPIRA_HIP_LAUNCH_CHECK();
    } else {
      size_t tb = p.temp_bytes;
      const ChainFlags<CT> flags(rocprim::counting_iterator<int64_t>(0), ChainFirst<CT>{p.merged, n_dev, n});
      SPIRA_HIP_TRY(rocprim::exclusive_scan(p.temp, tb, flags, p.pos, 0u, static_cast<size_t>(n),
                                            rocprim::plus<uint32_t>(), s));
      hipLaunchKernelGGL(chain_compact_kernel<CT>, grid, dim3(256), 0, s, p.merged, p.pos, n_dev, n,
                         static_cast<CT *>(outs[l]), d_counts + l, static_cast<uint32_t>(b[0]), p.xs, p.xe);
      SPIRA_HIP_LAUNCH_CHECK();
    }
    for (int q = 0; q < 3; ++q) a[q] = b[q];
  }
  return kOk;
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_downsample_workspace(int64_t n, int key_bits, size_t *bytes) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample: key_bits must be 32 or 64");
  *bytes = n <= 0 ? 0 : (key_bits == 64 ? ds_parts<uint64_t>(n, nullptr).total : ds_parts<uint32_t>(n, nullptr).total);
  return kOk;
}

int spira_hip_downsample(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz, void *out_keys,
                         uint32_t *d_count, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample: key_bits must be 32 or 64");
  if (key_bits == 64)
    return downsample_impl<uint64_t>(static_cast<const uint64_t *>(keys), n, sx, sy, sz,
                                     static_cast<uint64_t *>(out_keys), d_count, workspace, workspace_bytes, stream);
  return downsample_impl<uint32_t>(static_cast<const uint32_t *>(keys), n, sx, sy, sz,
                                   static_cast<uint32_t *>(out_keys), d_count, workspace, workspace_bytes, stream);
}

int spira_hip_downsample_plan(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz,
                              spira_hip_downsample_plan_t *plan, void *workspace, size_t workspace_bytes,
                              hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample_plan: key_bits must be 32 or 64");
  if (key_bits == 64)
    return plan_impl<uint64_t>(static_cast<const uint64_t *>(keys), n, sx, sy, sz, plan, workspace, workspace_bytes,
                               stream);
  return plan_impl<uint32_t>(static_cast<const uint32_t *>(keys), n, sx, sy, sz, plan, workspace, workspace_bytes,
                             stream);
}

int spira_hip_downsample_execute(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz,
                                 const spira_hip_downsample_plan_t *plan, void *out_keys, uint32_t *d_count,
                                 void *workspace, size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample: key_bits must be 32 or 64");
  if (key_bits == 64)
    return execute_impl<uint64_t>(static_cast<const uint64_t *>(keys), n, sx, sy, sz, plan,
                                  static_cast<uint64_t *>(out_keys), d_count, workspace, workspace_bytes, stream);
  return execute_impl<uint32_t>(static_cast<const uint32_t *>(keys), n, sx, sy, sz, plan,
                                static_cast<uint32_t *>(out_keys), d_count, workspace, workspace_bytes, stream);
}

int spira_hip_downsample_chain_workspace(int64_t n, int key_bits, size_t *bytes) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample_chain: key_bits must be 32 or 64");
  *bytes = n <= 0 ? 0
                  : (key_bits == 64 ? chain_parts<uint64_t>(n, nullptr).total : chain_parts<uint32_t>(n, nullptr).total);
  return kOk;
}

int spira_hip_downsample_chain(const void *keys, int64_t n, int key_bits, int levels, const int32_t *strides,
                               void *const *out_keys, uint32_t *d_counts, uint32_t *d_unsorted, void *workspace,
                               size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "downsample_chain: key_bits must be 32 or 64");
  if (key_bits == 64)
    return chain_impl<uint64_t>(static_cast<const uint64_t *>(keys), n, levels, strides, out_keys, d_counts,
                                d_unsorted, workspace, workspace_bytes, stream);
  return chain_impl<uint32_t>(static_cast<const uint32_t *>(keys), n, levels, strides, out_keys, d_counts, d_unsorted,
                              workspace, workspace_bytes, stream);
}

}  // extern "C"
