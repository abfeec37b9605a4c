// Kernel-map search and kernel-map post-processing for gfx950.
//
// Search (reference semantics: query_sorted.cuh:8-297, binary_search.cuh:10-21):
// for target t and xy-offset o, c = tgt[t] + off[o] (mod 2^bits),
// idx = lower_bound(src, c); entry(iz=0) = idx if src[idx] == c, then for
// iz = 1..kz-1: idx += (src[idx] <= c); c += sz; entry(iz) = idx if
// src[idx] == c.  Indices at or past the end of src give -1.
//
// MI355X design: a block owns a tile of 64 consecutive (sorted) targets and
// runs one wave64 per dx-group of offsets (kx waves), so that every tile's
// searches proceed in parallel and a CU holds enough waves to overlap the
// dependent L2/HBM round trips of the searches.  Per wave:
//  1. the wave reduces the min / max query key of its group (all queries of
//     the group lie between them, so their lower bounds lie between the lower
//     bounds of min and max, whatever modular wrap occurs);
//  2. both bounds are found by a wave-cooperative 64-ary search: each step
//     every lane probes one evenly spaced key per bound and a ballot picks
//     the sub-range, so a bound costs ~log64(S) dependent round trips instead
//     of log2(S);
//  3. the source window [lb(min), lb(max)+kz) is staged in the wave's LDS
//     slot with coalesced loads; each lane then runs its lower-bound search
//     and z-scan out of LDS.  Windows larger than the slot fall back to a
//     per-lane search in global memory restricted to the window (same
//     results);
//  4. [K, Tp] layouts store rows with coalesced 256-byte wave stores and emit
//     per-(row, tile) valid counts for compaction (ballot + popcount);
//     [Tp, K] layouts stage the tile's 64 x K block in LDS and the block
//     writes it out contiguously.

#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <rocprim/rocprim.hpp>

#include <algorithm>
#include <vector>

namespace spira_hip {

constexpr int kGroupMax = 8;      // dx groups (kx <= 8)
constexpr int kOffsetsMax = 128;  // offsets per map (K <= 128 for the no-z layout)
constexpr int kWindowCap = 512;   // LDS window entries per wave

template <typename CT> struct SearchParams {
  const CT *src;
  const CT *tgt;
  int32_t *map;
  int32_t *tile_counts;
  int64_t S, T, Tp, ntiles;
  int G, GS, O, K;
  int os_layout;  // 1: [Tp, K]; 0: [K, Tp]
  int zmajor;     // column iz*O + o in the [Tp, K] layout
  int use_perm;
  CT sz;
  CT off[kOffsetsMax];
  int32_t perm[kOffsetsMax];
};

template <typename CT> __device__ __forceinline__ CT max_key() { return static_cast<CT>(~static_cast<CT>(0)); }

// Range of lower_bound(src, v) from 64 wave-uniform samples: lane i holds
// src[base + i * step] (positions < end) or max_key past the end.  On return
// lb(v) lies in [blo, bhi].
template <typename CT>
__device__ __forceinline__ void sample_bucket(CT sample, CT v, int64_t base, int64_t step, int64_t end,
                                              int64_t &blo, int64_t &bhi) {
  const uint64_t m = ballot(sample >= v);
  const int j = m ? __builtin_ctzll(m) : 64;
  blo = j == 0 ? base : base + (j - 1) * step + 1;
  const int64_t p = base + j * step;
  bhi = p < end ? p : end;
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <typename CT>
__device__ __forceinline__ int lds_lower_bound(const CT *win, int n, CT v) {
  int base = 0, len = n;
  while (len > 0) {
    int half = len >> 1;
    if (win[base + half] < v) {
      base += half + 1;
      len -= half + 1;
    } else {
      len = half;
    }
  }
  return base;
}

template <typename CT>
__device__ __forceinline__ int64_t global_lower_bound(const CT *__restrict__ src, int64_t lo, int64_t hi, CT v) {
  while (lo < hi) {
    int64_t m = (lo + hi) >> 1;
    if (src[m] >= v) hi = m;
    else lo = m + 1;
  }
  return lo;
}

// Layout variants of the search kernel (compile-time, so that the store
// path carries no per-entry layout tests).
enum SearchLayout : int {
  kLayoutOsZ = 0,  // [Tp, K], column iz*O + o (output-stationary, z-major)
  kLayoutWs = 1,   // [K, Tp], row k (or perm[k]), plus per-(row, tile) counts
  kLayoutNoz = 2,  // [Tp, K], column k, full offsets and no z-scan (KZ = 1)
};

// The search of one 64-target tile (one block).  GS: offsets per dx-group
// when known at compile time (the dy range of the common kernels), else 0
// (runtime p.GS, in chunks of kChunk).  P: SearchParams or SearchJob (the
// fields the tile reads).
template <typename CT, int KZ, int GS, int LAYOUT, class P>
__device__ __forceinline__ void search_tile(const P &p, const int64_t tile) {
  constexpr int kChunk = GS > 0 ? GS : 4;
  extern __shared__ __align__(16) char smem[];
  const int g = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // dx-group of this wave
  const int gs = GS > 0 ? GS : p.GS;
  CT *win = reinterpret_cast<CT *>(smem) + g * kWindowCap;
  int32_t *stage = reinterpret_cast<int32_t *>(smem + p.G * kWindowCap * sizeof(CT));

  const int lane = threadIdx.x & 63;
  const int64_t t = tile * 64 + lane;
  const bool valid = t < p.T;
  // level-1 samples of the sources (independent of the queries, so this load
  // overlaps the target-key load): lane i holds src[i * s1]
  const int64_t s1 = (p.S + 63) / 64;
  const CT l1 = lane * s1 < p.S ? p.src[lane * s1] : max_key<CT>();
  const CT key = valid ? p.tgt[t] : CT(0);
  const CT sz = p.sz;

  if (ballot(valid) == 0) {
    // fully padded tile: every entry is -1
    if constexpr (LAYOUT != kLayoutWs) {
      for (int i = threadIdx.x; i < 64 * p.K; i += blockDim.x) p.map[tile * 64 * p.K + i] = -1;
    } else {
      for (int r = g; r < p.K; r += p.G) {
        p.map[r * p.Tp + t] = -1;
        if (p.tile_counts && lane == 0) p.tile_counts[r * p.ntiles + tile] = 0;
      }
    }
    return;
  }

  // 1. query bounds of this wave's group
  CT vals[2];
  {
    CT mn = max_key<CT>(), mx = CT(0);
    for (int j = 0; j < gs; ++j) {
      CT q = key + p.off[g * gs + j];
      if (valid) {
        mn = q < mn ? q : mn;
        mx = q > mx ? q : mx;
      }
    }
    vals[0] = wave_min(mn);
    vals[1] = wave_max(mx);
  }
  // 2. lower-bound ranges of both: level 1 from the samples above, level 2
  //    from 64 samples inside each level-1 bucket (one dependent round trip)
  int64_t lb[2];
  {
    int64_t blo[2], bhi[2];
    sample_bucket(l1, vals[0], 0, s1, p.S, blo[0], bhi[0]);
    sample_bucket(l1, vals[1], 0, s1, p.S, blo[1], bhi[1]);
    CT l2[2];
    int64_t s2[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      s2[b] = (bhi[b] - blo[b] + 63) / 64;
      if (s2[b] < 1) s2[b] = 1;
      const int64_t q = blo[b] + lane * s2[b];
      l2[b] = q < bhi[b] ? p.src[q] : max_key<CT>();
    }
    int64_t lo2, hi2;
    sample_bucket(l2[0], vals[0], blo[0], s2[0], bhi[0], lo2, hi2);
    lb[0] = lo2;
    sample_bucket(l2[1], vals[1], blo[1], s2[1], bhi[1], lo2, hi2);
    lb[1] = hi2;  // upper end of lb(max)'s range
  }

  // 3. stage the window, search, z-scan, store
  // the window bounds are wave-uniform (ballot results); saying so keeps
  // them, the window branch and the search trip counts in scalar registers
  const int64_t lo = uniform64(lb[0]);
  int64_t hi = uniform64(lb[1]) + KZ;
  if (hi > p.S) hi = p.S;
  const int n = static_cast<int>(hi - lo);
  const bool in_lds = (hi - lo) <= kWindowCap;
  if (in_lds) {
    // every load of the window is issued before the first LDS write
    CT r[kWindowCap / 64];
#pragma unroll
    for (int i = 0; i < kWindowCap / 64; ++i) {
      const int q = lane + 64 * i;
      r[i] = q < n ? p.src[lo + q] : CT(0);
    }
#pragma unroll
    for (int i = 0; i < kWindowCap / 64; ++i) {
      const int q = lane + 64 * i;
      if (q < n) win[q] = r[i];
    }
    // the window is private to this wave: LDS keeps a wave's accesses in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // one entry: [Tp, K] layouts stage the tile block in LDS; [K, Tp] writes
  // coalesced rows and the row's valid count of this tile
  auto emit = [&](int o, int iz, int32_t r) {
    if constexpr (LAYOUT == kLayoutOsZ) {
      stage[lane * p.K + iz * p.O + o] = r;
    } else if constexpr (LAYOUT == kLayoutNoz) {
      stage[lane * p.K + o] = r;
    } else {
      const int k = o * KZ + iz;
      const int row = p.use_perm ? p.perm[k] : k;
      p.map[row * p.Tp + t] = r;
      if (p.tile_counts) {
        const uint64_t m = ballot(r >= 0);
        if (lane == 0) p.tile_counts[row * p.ntiles + tile] = __builtin_popcountll(m);
      }
    }
  };

  if (in_lds) {
    // The group's offsets in chunks, the chunk's lower bounds and z-scans
    // interleaved so that their dependent LDS reads overlap.  The lower bound
    // is the branch-free form over the wave-uniform window length (every lane
    // runs the same steps).  Padded lanes, and offsets past the group, query
    // the group minimum, which keeps every index inside the window.
    for (int j0 = 0; j0 < gs; j0 += kChunk) {
      CT c[kChunk];
      int base[kChunk];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const bool act = valid && (GS > 0 || j0 + j < gs);
        c[j] = act ? CT(key + p.off[g * gs + j0 + j]) : vals[0];
        base[j] = 0;
      }
      for (int len = n; len > 1;) {
        const int half = len >> 1;
        CT w[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) w[j] = win[base[j] + half - 1];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) base[j] = w[j] < c[j] ? base[j] + half : base[j];
        len -= half;
      }
      int idx[kChunk];
      CT v[kChunk];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        v[j] = n > 0 ? win[base[j]] : CT(0);
        idx[j] = base[j] + ((n > 0 && v[j] < c[j]) ? 1 : 0);
      }
      // z-scan (query_sorted.cuh:8-163).  An index at the window end is past
      // the end of the sources: the window holds lb(max) + KZ entries unless
      // it ends at S.
#pragma unroll
      for (int iz = 0; iz < KZ; ++iz) {
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
          if (iz > 0) {
            if (idx[j] < n && v[j] <= c[j]) ++idx[j];
            c[j] += sz;
          }
          v[j] = idx[j] < n ? win[idx[j]] : CT(0);
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
          if (GS > 0 || j0 + j < gs) {
            const int32_t r = (valid && idx[j] < n && v[j] == c[j]) ? static_cast<int32_t>(lo + idx[j]) : -1;
            emit(g * gs + j0 + j, iz, r);
          }
        }
      }
    }
  } else {
    // window larger than the LDS slot (rare): per-lane search in global
    // memory, restricted to the window (same results)
    for (int j = 0; j < gs; ++j) {
      const int o = g * gs + j;
      CT c = valid ? CT(key + p.off[o]) : vals[0];
      int64_t idx = global_lower_bound(p.src, lo, hi, c);
      CT v = idx < p.S ? p.src[idx] : CT(0);
      emit(o, 0, (valid && idx < p.S && v == c) ? static_cast<int32_t>(idx) : -1);
#pragma unroll
      for (int iz = 1; iz < KZ; ++iz) {
        if (idx < p.S && v <= c) ++idx;
        c += sz;
        v = idx < p.S ? p.src[idx] : CT(0);
        emit(o, iz, (valid && idx < p.S && v == c) ? static_cast<int32_t>(idx) : -1);
      }
    }
  }

  if constexpr (LAYOUT != kLayoutWs) {
    __syncthreads();
    int32_t *dst = p.map + tile * 64 * p.K;
    const int total = 64 * p.K;  // multiple of 4
    const int4 *s4 = reinterpret_cast<const int4 *>(stage);
    int4 *d4 = reinterpret_cast<int4 *>(dst);
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i *sv = reinterpret_cast<const v4i *>(s4);
    v4i *dv = reinterpret_cast<v4i *>(d4);
    for (int i = threadIdx.x; i < total / 4; i += blockDim.x) __builtin_nontemporal_store(sv[i], dv + i);
  }
}

template <typename CT, int KZ, int GS, int LAYOUT>
__global__ __launch_bounds__(64 * kGroupMax) void kmap_search_kernel(const SearchParams<CT> p) {
  search_tile<CT, KZ, GS, LAYOUT>(p, blockIdx.x);
}

// Several output-stationary maps of one kernel shape in one launch: job j
// owns tiles [tile_start[j], tile_start[j + 1]) of the grid, so that the
// searches of a network's small maps overlap instead of running back to back.
constexpr int kJobOffsets = 27;  // xy offsets (kx * ky; the z-scan covers z): up to 5 x 5
constexpr int kJobsMax = 8;
template <typename CT> struct SearchJob {
  const CT *src;
  const CT *tgt;
  int32_t *map;
  int32_t *tile_counts;  // (unused: the output-stationary layout has none)
  int64_t S, T, Tp, ntiles;
  int G, GS, O, K;
  int use_perm;
  CT sz;
  CT off[kJobOffsets];
};
template <typename CT> struct SearchBatch {
  int n;
  int64_t tile_start[kJobsMax + 1];
  SearchJob<CT> job[kJobsMax];
};

static_assert(sizeof(SearchBatch<uint64_t>) <= 4096, "batch parameters must fit the kernel argument block");

template <typename CT, int KZ, int GS>
__global__ __launch_bounds__(64 * kGroupMax) void kmap_search_batch_kernel(const SearchBatch<CT> b) {
  const int64_t tile = blockIdx.x;
  int j = 0;
  for (int q = 1; q < b.n; ++q) j = tile >= b.tile_start[q] ? q : j;
  search_tile<CT, KZ, GS, kLayoutOsZ>(b.job[j], tile - b.tile_start[j]);
}

template <typename CT> static void make_offsets(int kx, int ky, int kz, int sx, int sy, int sz, bool full, CT *out) {
  // offset tables of torch/cuda_sparse_convolution_mapping.cu:10-50 (xy only,
  // z pinned to kz_min*sz) and :114-157 (full): x outer, y, z inner; packed
  // with modular arithmetic exactly like the key arithmetic.
  auto kmin = [](int k) { return (k % 2 == 1) ? -(k / 2) : -(k / 2) + 1; };
  int idx = 0;
  for (int ix = kmin(kx); ix <= kx / 2; ++ix)
    for (int iy = kmin(ky); iy <= ky / 2; ++iy) {
      if (full) {
        for (int iz = kmin(kz); iz <= kz / 2; ++iz)
          out[idx++] = static_cast<CT>(static_cast<CT>(ix * sx) * (CT(1) << Layout<CT>::XS) +
                                       static_cast<CT>(iy * sy) * (CT(1) << Layout<CT>::YS) +
                                       static_cast<CT>(iz * sz));
      } else {
        out[idx++] = static_cast<CT>(static_cast<CT>(ix * sx) * (CT(1) << Layout<CT>::XS) +
                                     static_cast<CT>(iy * sy) * (CT(1) << Layout<CT>::YS) +
                                     static_cast<CT>(kmin(kz) * sz));
      }
    }
}

template <typename CT, int KZ, int LAYOUT>
static void launch_search_l(int gs, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const SearchParams<CT> &p) {
  switch (gs) {
    case 1: hipLaunchKernelGGL((kmap_search_kernel<CT, KZ, 1, LAYOUT>), grid, block, lds, stream, p); break;
    case 2: hipLaunchKernelGGL((kmap_search_kernel<CT, KZ, 2, LAYOUT>), grid, block, lds, stream, p); break;
    case 3: hipLaunchKernelGGL((kmap_search_kernel<CT, KZ, 3, LAYOUT>), grid, block, lds, stream, p); break;
    case 5: hipLaunchKernelGGL((kmap_search_kernel<CT, KZ, 5, LAYOUT>), grid, block, lds, stream, p); break;
    default: hipLaunchKernelGGL((kmap_search_kernel<CT, KZ, 0, LAYOUT>), grid, block, lds, stream, p); break;
  }
}

template <typename CT, int KZ>
static void launch_search_kz(int gs, int lay, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                             const SearchParams<CT> &p) {
  if (lay == kLayoutOsZ) launch_search_l<CT, KZ, kLayoutOsZ>(gs, grid, block, lds, stream, p);
  else launch_search_l<CT, KZ, kLayoutWs>(gs, grid, block, lds, stream, p);
}

// KZ = 1 serves the full-offset layout (no z-scan) and kernels of depth 1
template <typename CT>
static void launch_search(int kz, int gs, int lay, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                          const SearchParams<CT> &p) {
  switch (kz) {
    case 1:
      if (lay == kLayoutNoz) hipLaunchKernelGGL((kmap_search_kernel<CT, 1, 0, kLayoutNoz>), grid, block, lds, stream, p);
      else launch_search_kz<CT, 1>(gs, lay, grid, block, lds, stream, p);
      break;
    case 2: launch_search_kz<CT, 2>(gs, lay, grid, block, lds, stream, p); break;
    case 3: launch_search_kz<CT, 3>(gs, lay, grid, block, lds, stream, p); break;
    case 4: launch_search_kz<CT, 4>(gs, lay, grid, block, lds, stream, p); break;
    default: launch_search_kz<CT, 5>(gs, lay, grid, block, lds, stream, p); break;
  }
}

template <typename CT>
static int search_impl(const CT *src, int64_t S, const CT *tgt, int64_t T, int kx, int ky, int kz, int sx, int sy,
                       int sz, int layout, const int32_t *row_perm, int32_t *map, int32_t *tile_counts,
                       hipStream_t stream) {
  SPIRA_HIP_REQUIRE(S >= 0 && T >= 0 && S < (int64_t(1) << 31) && T < (int64_t(1) << 31),
                    "kmap_search: sizes out of range");
  SPIRA_HIP_REQUIRE(kx >= 1 && ky >= 1 && kz >= 1, "kmap_search: kernel size must be positive");
  SPIRA_HIP_REQUIRE(kx <= kGroupMax, "kmap_search: kernel size along x is limited to 8");
  SPIRA_HIP_REQUIRE(layout >= SPIRA_KMAP_OS && layout <= SPIRA_KMAP_NOZ, "kmap_search: unknown layout");
  const int K = kx * ky * kz;
  SPIRA_HIP_REQUIRE(K <= kOffsetsMax, "kmap_search: kernel volume is limited to 128 offsets");
  SearchParams<CT> p{};
  p.src = src;
  p.tgt = tgt;
  p.map = map;
  p.S = S;
  p.T = T;
  p.Tp = round_up(T, 128);
  p.ntiles = p.Tp / 64;
  p.K = K;
  p.sz = static_cast<CT>(static_cast<uint32_t>(sz));
  int KZ = kz;
  if (layout == SPIRA_KMAP_NOZ) {
    make_offsets<CT>(kx, ky, kz, sx, sy, sz, true, p.off);
    p.G = kx;
    p.GS = ky * kz;
    p.O = K;
    KZ = 1;
    p.os_layout = 1;
    p.zmajor = 0;
  } else {
    SPIRA_HIP_REQUIRE(kz <= 5, "Currently Kernel Size in Z axis can only be 1..5");
    make_offsets<CT>(kx, ky, kz, sx, sy, sz, false, p.off);
    p.G = kx;
    p.GS = ky;
    p.O = kx * ky;
    p.os_layout = layout == SPIRA_KMAP_OS;
    p.zmajor = layout == SPIRA_KMAP_OS;
  }
  if (layout == SPIRA_KMAP_HYBRID) {
    SPIRA_HIP_REQUIRE(row_perm != nullptr, "kmap_search: hybrid layout needs a row permutation");
    for (int k = 0; k < K; ++k) {
      SPIRA_HIP_REQUIRE(row_perm[k] >= 0 && row_perm[k] < K, "kmap_search: bad row permutation");
      p.perm[k] = row_perm[k];
    }
    p.use_perm = 1;
  }
  p.tile_counts = p.os_layout ? nullptr : tile_counts;
  if (p.Tp == 0) return kOk;
  const size_t lds = p.G * kWindowCap * sizeof(CT) + (p.os_layout ? 64 * K * sizeof(int32_t) : 0);
  dim3 grid(static_cast<unsigned>(p.ntiles)), block(64 * p.G);
  const int lay = layout == SPIRA_KMAP_NOZ ? kLayoutNoz : (p.os_layout ? kLayoutOsZ : kLayoutWs);
  launch_search<CT>(KZ, p.GS, lay, grid, block, lds, stream, p);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

// Batched output-stationary searches: jobs of the kernel shapes that have a
// batch kernel (2x2x2, 3x3x3, 5x5x5) are grouped by shape, at most kJobsMax per
// launch, in their order; every other job is one search_impl call.
template <typename CT>
static int search_batch_impl(int n, const spira_hip_kmap_job_t *jobs, hipStream_t stream) {
  std::vector<char> done(static_cast<size_t>(n), 0);
  auto batchable = [](const spira_hip_kmap_job_t &j) {
    return (j.kx == 2 && j.ky == 2 && j.kz == 2) || (j.kx == 3 && j.ky == 3 && j.kz == 3) ||
           (j.kx == 5 && j.ky == 5 && j.kz == 5);
  };
  for (int a = 0; a < n; ++a) {
    if (done[a]) continue;
    const spira_hip_kmap_job_t &ja = jobs[a];
    if (!batchable(ja)) {
      done[a] = 1;
      const int rc = search_impl<CT>(static_cast<const CT *>(ja.sources), ja.num_sources,
                                     static_cast<const CT *>(ja.targets), ja.num_targets, ja.kx, ja.ky, ja.kz, ja.sx,
                                     ja.sy, ja.sz, SPIRA_KMAP_OS, nullptr, ja.kernel_map, nullptr, stream);
      if (rc) return rc;
      continue;
    }
    SearchBatch<CT> b{};
    int64_t tiles = 0;
    for (int c = a; c < n && b.n < kJobsMax; ++c) {
      const spira_hip_kmap_job_t &jc = jobs[c];
      if (done[c] || jc.kx != ja.kx || jc.ky != ja.ky || jc.kz != ja.kz) continue;
      SPIRA_HIP_REQUIRE(jc.num_sources >= 0 && jc.num_targets >= 0 && jc.num_sources < (int64_t(1) << 31) &&
                            jc.num_targets < (int64_t(1) << 31),
                        "kmap_search_batch: sizes out of range");
      SPIRA_HIP_REQUIRE(jc.num_targets == 0 || (jc.kernel_map != nullptr && jc.targets != nullptr &&
                                                 (jc.num_sources == 0 || jc.sources != nullptr)),
                        "kmap_search_batch: missing array");
      done[c] = 1;
      SearchJob<CT> &p = b.job[b.n];
      p.src = static_cast<const CT *>(jc.sources);
      p.tgt = static_cast<const CT *>(jc.targets);
      p.map = jc.kernel_map;
      p.tile_counts = nullptr;
      p.S = jc.num_sources;
      p.T = jc.num_targets;
      p.Tp = round_up(p.T, 128);
      p.ntiles = p.Tp / 64;
      p.K = jc.kx * jc.ky * jc.kz;
      p.G = jc.kx;
      p.GS = jc.ky;
      p.O = jc.kx * jc.ky;
      p.use_perm = 0;
      p.sz = static_cast<CT>(static_cast<uint32_t>(jc.sz));
      make_offsets<CT>(jc.kx, jc.ky, jc.kz, jc.sx, jc.sy, jc.sz, false, p.off);
      b.tile_start[b.n] = tiles;
      tiles += p.ntiles;
      ++b.n;
    }
    b.tile_start[b.n] = tiles;
    if (tiles == 0) continue;
    SPIRA_HIP_REQUIRE(tiles < (int64_t(1) << 31), "kmap_search_batch: too many tiles");
    const int K = ja.kx * ja.ky * ja.kz;
    const size_t lds = ja.kx * kWindowCap * sizeof(CT) + 64 * K * sizeof(int32_t);
    const dim3 grid(static_cast<unsigned>(tiles)), block(64 * ja.kx);
    if (ja.kz == 2) hipLaunchKernelGGL((kmap_search_batch_kernel<CT, 2, 2>), grid, block, lds, stream, b);
    else if (ja.kz == 3) hipLaunchKernelGGL((kmap_search_batch_kernel<CT, 3, 3>), grid, block, lds, stream, b);
    else hipLaunchKernelGGL((kmap_search_batch_kernel<CT, 5, 5>), grid, block, lds, stream, b);
    SPIRA_HIP_LAUNCH_CHECK();
  }
  return kOk;
}

// ---------------------------------------------------------------------------
// post-processing
// ---------------------------------------------------------------------------
__global__ void fill_i32_kernel(int32_t *__restrict__ p, int64_t n, int32_t v) {
  int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    *reinterpret_cast<int4 *>(p + i) = make_int4(v, v, v, v);
  } else {
    for (int64_t j = i; j < n && j < i + 4; ++j) p[j] = v;
  }
}

static int fill_i32(int32_t *p, int64_t n, int32_t v, hipStream_t s) {
  if (n <= 0) return kOk;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(div_up(div_up(n, 4), 256)), dim3(256), 0, s, p, n, v);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

// nbsizes[r] = per-row totals; naddrs / qnaddrs exclusive scans (quantum q)
// (query_sorted_index.cu:146-209 with quantifier_wstat.cuh:8-41).
__global__ void row_totals_kernel(const int32_t *__restrict__ tile_counts, const int32_t *__restrict__ tile_offsets,
                                  int R, int64_t ntiles, int q, int32_t *__restrict__ nbsizes,
                                  int32_t *__restrict__ naddrs, int32_t *__restrict__ qnaddrs,
                                  int32_t *__restrict__ sizes) {
  // one block; R <= 128
  __shared__ int32_t tot[kOffsetsMax];
  int r = threadIdx.x;
  if (r < R) {
    int64_t last = (static_cast<int64_t>(r) + 1) * ntiles - 1;
    int32_t end = tile_offsets[last] + tile_counts[last];
    int32_t beg = tile_offsets[static_cast<int64_t>(r) * ntiles];
    tot[r] = end - beg;
    nbsizes[r] = end - beg;
  }
  __syncthreads();
  if (r == 0) {
    int32_t acc = 0, qacc = 0;
    for (int i = 0; i < R; ++i) {
      if (naddrs) naddrs[i] = acc;
      if (qnaddrs) qnaddrs[i] = qacc;
      acc += tot[i];
      qacc += (tot[i] + q - 1) / q * q;
    }
    if (naddrs) naddrs[R] = acc;
    if (qnaddrs) qnaddrs[R] = qacc;
    if (sizes) {
      sizes[0] = acc;
      sizes[1] = qacc;
    }
  }
}

// one wave per (row, tile): stable compaction in (row, t) order
__global__ __launch_bounds__(256) void emit_pairs_kernel(const int32_t *__restrict__ map, int64_t Tp, int row0,
                                                         int R, int64_t ntiles,
                                                         const int32_t *__restrict__ tile_offsets,
                                                         int32_t *__restrict__ in_idx,
                                                         int32_t *__restrict__ out_idx) {
  const int64_t w = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (w >= R * ntiles) return;
  const int lane = lane_id();
  const int64_t r = w / ntiles, tile = w % ntiles;
  const int64_t t = tile * 64 + lane;
  const int32_t v = map[(row0 + r) * Tp + t];
  const bool ok = v != -1;
  const uint64_t m = ballot(ok);
  if (ok) {
    const int64_t pos = tile_offsets[w] + lane_prefix(m);
    in_idx[pos] = v;
    out_idx[pos] = static_cast<int32_t>(t);
  }
}

// masks: rank of each valid entry within its row (generate_masks_from_kernel_map.cuh:10-62)
__global__ __launch_bounds__(256) void emit_masks_kernel(const int32_t *__restrict__ map, int64_t S, int64_t T,
                                                         int64_t Tp, int row0, int R, int Km, int half,
                                                         int64_t ntiles, const int32_t *__restrict__ tile_offsets,
                                                         int32_t *__restrict__ smask, int32_t *__restrict__ tmask) {
  const int64_t w = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (w >= R * ntiles) return;
  const int lane = lane_id();
  const int64_t r = w / ntiles, tile = w % ntiles;
  const int64_t t = tile * 64 + lane;
  const int32_t v = map[(row0 + r) * Tp + t];
  const bool ok = v != -1;
  const uint64_t m = ballot(ok);
  if (ok) {
    const int32_t rank = tile_offsets[w] - tile_offsets[r * ntiles] + lane_prefix(m);
    smask[r * S + v] = rank;
    tmask[r * T + t] = rank;
    if (half && 2 * r + 1 != Km) {
      smask[(Km - 1 - r) * S + t] = rank;
      tmask[(Km - 1 - r) * T + v] = rank;
    }
  }
}

// transposed OS map: out[s, k] = t where map[t, k] = s (convert_transposed_os.cuh:7-16)
__global__ void convert_transposed_kernel(const int32_t *__restrict__ map, int64_t n, int K,
                                          int32_t *__restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int32_t s = map[i];
  if (s < 0) return;
  out[static_cast<int64_t>(s) * K + i % K] = static_cast<int32_t>(i / K);
}

// The inverse of a map whose entries partition the sources (every source in
// exactly one entry: a down-sampling map whose kernel is its stride), in one
// pass: the entry (t, k) of source s writes all of row s (t at column k, -1
// elsewhere), and the padding rows [S, Sp) are -1.  Threads [0, n) take
// entries, [n, n + pad) padding words.
__global__ void convert_transposed_partition_kernel(const int32_t *__restrict__ map, int64_t n, int K, int64_t S,
                                                    int64_t Sp, int32_t *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) {
    const int64_t w = S * K + (i - n);
    if (w < Sp * K) out[w] = -1;
    return;
  }
  const int32_t s = map[i];
  if (s < 0 || s >= S) return;
  const int k = static_cast<int>(i % K);
  const int32_t t = static_cast<int32_t>(i / K);
  int32_t *row = out + static_cast<int64_t>(s) * K;
  if (K % 4 == 0) {  // 16-byte row chunks (rows start 16-byte aligned)
    int4 *row4 = reinterpret_cast<int4 *>(row);
    for (int q = 0; q < K / 4; ++q) {
      const int b = 4 * q;
      row4[q] = make_int4(b == k ? t : -1, b + 1 == k ? t : -1, b + 2 == k ? t : -1, b + 3 == k ? t : -1);
    }
  } else {
    for (int j = 0; j < K; ++j) row[j] = j == k ? t : -1;
  }
}

// ---- row order of a partition map's inverse, without a sort.  The inverse
// of a map whose entries partition the sources has one valid entry per row
// (column k, the entry's offset), so its stable (count, mask) row order is
// the rows grouped by k, each group in source order, which is coarse-row
// order.  Two launches over 256-row tiles of the coarse map:
//   tp_count_kernel  per (k, tile) valid counts (and the inverse's padding
//                    rows, -1);
//   tp_emit_kernel   each block sums the counts (its tile's base in each
//                    bucket, the bucket totals), then each entry's position
//                    (bucket base + rank in the tile): the order, the ordered
//                    map row and the inverse row; block 0 also writes every
//                    128-row group's column union (from the bucket bounds).
constexpr int kTpTile = 256;
constexpr int kTpMaxK = 8;
constexpr int kTpMaxCounts = 16384;  // K * ntiles: each emit block sums them all

// the row of a partition inverse: t at column k, -1 elsewhere
__device__ __forceinline__ void tp_row(int32_t *row, int K, int k, int32_t t) {
  if (K % 4 == 0) {
    int4 *row4 = reinterpret_cast<int4 *>(row);
    for (int q = 0; q < K / 4; ++q) {
      const int b = 4 * q;
      row4[q] = make_int4(b == k ? t : -1, b + 1 == k ? t : -1, b + 2 == k ? t : -1, b + 3 == k ? t : -1);
    }
  } else {
    for (int j = 0; j < K; ++j) row[j] = j == k ? t : -1;
  }
}

__global__ __launch_bounds__(kTpTile) void tp_count_kernel(const int32_t *__restrict__ map, int64_t Tc, int K,
                                                           int ntiles, int32_t *__restrict__ cnt, int64_t S,
                                                           int64_t Sp, int32_t *__restrict__ inverse,
                                                           int32_t *__restrict__ ordered_map) {
  __shared__ int32_t part[kTpTile / 64][kTpMaxK];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTpTile + tid;
  for (int k = 0; k < K; ++k) {
    const bool v = t < Tc && map[t * K + k] >= 0;
    const uint64_t m = ballot(v);
    if (lane == 0) part[w][k] = __builtin_popcountll(m);
  }
  __syncthreads();
  if (tid < K) {
    int c = 0;
    for (int q = 0; q < kTpTile / 64; ++q) c += part[q][tid];
    cnt[tid * ntiles + blockIdx.x] = c;
  }
  // every inverse and ordered-map word starts at -1: the emit pass rewrites
  // the row of each source it finds, so a source that lies in no entry (a map
  // whose entries do not partition its sources) keeps an all -1 row
  const int64_t step = static_cast<int64_t>(gridDim.x) * kTpTile;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kTpTile + tid; i < Sp * K; i += step) inverse[i] = -1;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kTpTile + tid; i < S * K; i += step) ordered_map[i] = -1;
}

__global__ __launch_bounds__(kTpTile) void tp_emit_kernel(const int32_t *__restrict__ map, int64_t Tc, int K,
                                                          int ntiles, const int32_t *__restrict__ cnt, int64_t S,
                                                          int32_t *__restrict__ order,
                                                          int32_t *__restrict__ ordered_map,
                                                          int32_t *__restrict__ inverse,
                                                          uint64_t *__restrict__ masks) {
  __shared__ int32_t part[kTpTile / 64][kTpMaxK];
  __shared__ int32_t red[kTpTile / 64][2 * kTpMaxK];
  __shared__ int32_t base[kTpMaxK + 1], tile_base[kTpMaxK];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTpTile + tid;
  // the thread's map row, loaded first so that it overlaps the counts' loads
  // (loops over the compile-time maximum, so that src / rank stay in registers)
  int32_t src[kTpMaxK];
#pragma unroll
  for (int k = 0; k < kTpMaxK; ++k) src[k] = (k < K && t < Tc) ? map[t * K + k] : -1;
  // this tile's position in each bucket: the counts of the tiles before it,
  // and the buckets' totals (every block sums the K * ntiles counts itself)
  {
    int before[kTpMaxK], total[kTpMaxK];
#pragma unroll
    for (int k = 0; k < kTpMaxK; ++k) before[k] = total[k] = 0;
    for (int q = tid; q < ntiles; q += kTpTile) {
#pragma unroll
      for (int k = 0; k < kTpMaxK; ++k) {
        const int c = k < K ? cnt[k * ntiles + q] : 0;
        total[k] += c;
        before[k] += q < static_cast<int>(blockIdx.x) ? c : 0;
      }
    }
#pragma unroll
    for (int k = 0; k < kTpMaxK; ++k) {
      for (int d = 32; d > 0; d >>= 1) {
        before[k] += __shfl_xor(before[k], d, 64);
        total[k] += __shfl_xor(total[k], d, 64);
      }
      if (lane == 0) {
        red[w][k] = before[k];
        red[w][kTpMaxK + k] = total[k];
      }
    }
    __syncthreads();
    if (tid == 0) {
      int run = 0;
      for (int k = 0; k < K; ++k) {
        int b = 0, tot = 0;
        for (int q = 0; q < kTpTile / 64; ++q) {
          b += red[q][k];
          tot += red[q][kTpMaxK + k];
        }
        base[k] = run;
        tile_base[k] = run + b;
        run += tot;
      }
      base[K] = run;
    }
    __syncthreads();
  }
  // Entries that do not partition the sources (fewer valid entries than
  // sources: some source lies in no entry): the order is the identity, the
  // ordered map is the inverse, every group's union holds all K columns, and
  // each entry writes only its own word (rows start at -1, count pass).
  if (base[K] != S) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * kTpTile;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kTpTile + tid; i < S; i += step)
      order[i] = static_cast<int32_t>(i);
    if (blockIdx.x == 0)
      for (int64_t g = tid; g < (S + 127) / 128; g += kTpTile) {
        masks[2 * g] = K >= 64 ? ~uint64_t(0) : (uint64_t(1) << K) - 1;
        masks[2 * g + 1] = 0;
      }
#pragma unroll
    for (int k = 0; k < kTpMaxK; ++k) {
      const int32_t s = src[k];
      if (s < 0 || s >= S) continue;
      inverse[static_cast<int64_t>(s) * K + k] = static_cast<int32_t>(t);
      ordered_map[static_cast<int64_t>(s) * K + k] = static_cast<int32_t>(t);
    }
    return;
  }
  // block 0: the column union of every 128-row group of the ordered rows
  // (from the k bucket bounds)
  if (blockIdx.x == 0) {
    const int64_t total = base[K];
    const int64_t G = (S + 127) / 128;
    for (int64_t g = tid; g < G; g += kTpTile) {
      const int64_t lo = g * 128, hi = lo + 128 < total ? lo + 128 : total;
      uint64_t bits = 0;
      for (int k = 0; k < K; ++k)
        if (base[k + 1] > base[k] && base[k] < hi && base[k + 1] > lo) bits |= uint64_t(1) << k;
      masks[2 * g] = bits;
      masks[2 * g + 1] = 0;
    }
  }
  int rank[kTpMaxK];
#pragma unroll
  for (int k = 0; k < kTpMaxK; ++k) {
    const uint64_t m = ballot(src[k] >= 0);
    rank[k] = lane_prefix(m);
    if (lane == 0 && k < K) part[w][k] = __builtin_popcountll(m);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kTpMaxK; ++k) {
    const int32_t s = src[k];
    if (s < 0 || s >= S) continue;
    int pos = tile_base[k] + rank[k];
    for (int q = 0; q < w; ++q) pos += part[q][k];
    if (pos >= S) continue;  // (a source in two entries; then the counts do not sum to S)
    order[pos] = s;
    tp_row(ordered_map + static_cast<int64_t>(pos) * K, K, k, static_cast<int32_t>(t));
    tp_row(inverse + static_cast<int64_t>(s) * K, K, k, static_cast<int32_t>(t));
  }
}

// Row-order key of an output-stationary map row: the bitmask of its valid
// columns (the first 63 columns, with bit 63 flagging any valid column past
// them), so that sorting groups rows with identical neighbour patterns.
// Sort key of a map row: rows with more neighbours first (their blocks run
// longest, so they are dispatched first), then rows with the same neighbour
// pattern together.  Key = (K - popcount) << P | pattern, where the pattern
// keeps the first P = min(K, 57) columns; row_key_bits(K) bits in all.
__host__ __device__ __forceinline__ int row_pattern_bits(int K) { return K < 57 ? K : 57; }
__host__ __device__ __forceinline__ int row_key_bits(int K) {
  int c = 1;  // bits of the largest count field value K
  while ((1 << c) <= K) ++c;
  return row_pattern_bits(K) + c;
}
// One block stages RB consecutive map rows in LDS with coalesced loads (RB =
// 256 rows for K <= 32, else 64), then thread t < RB builds row t's key.
// (block `blk` of one map: rows [blk * RB, blk * RB + RB); keys[r] and
// iota[r] for local row r; key_hi is ORed into every key)
template <typename KT>
__device__ __forceinline__ void row_mask_block(const int32_t *__restrict__ map, int64_t T, int K, int RB, int64_t blk,
                                               KT *__restrict__ keys, int32_t *__restrict__ iota, KT key_hi,
                                               int32_t iota_base, int32_t *rows_lds) {
  const int64_t row0 = blk * RB;
  const int nr = static_cast<int>((T - row0) < RB ? (T - row0) : RB);
  // the block's rows are one contiguous run of nr * K words: 16-byte loads
  // where the run is 16-byte aligned, several in flight per thread
  const int32_t *src = map + row0 * K;
  const int n = nr * K;
  int head = 0;
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const int n4 = n / 4;
#pragma unroll 4
    for (int e = threadIdx.x; e < n4; e += 256)
      reinterpret_cast<int4 *>(rows_lds)[e] = reinterpret_cast<const int4 *>(src)[e];
    head = n4 * 4;
  }
  for (int e = head + static_cast<int>(threadIdx.x); e < n; e += 256) rows_lds[e] = src[e];
  __syncthreads();
  if (threadIdx.x >= nr) return;
  const int32_t *row = rows_lds + threadIdx.x * K;
  const int P = row_pattern_bits(K);
  uint64_t m = 0;
  int cnt = 0;
  for (int j = 0; j < K; ++j) {
    const bool v = row[j] >= 0;
    cnt += v;
    if (v && j < P) m |= uint64_t(1) << j;
  }
  keys[row0 + threadIdx.x] = key_hi | static_cast<KT>((static_cast<uint64_t>(K - cnt) << P) | m);
  iota[row0 + threadIdx.x] = iota_base + static_cast<int32_t>(row0 + threadIdx.x);
}

// One block stages RB consecutive map rows in LDS with coalesced loads (RB =
// 256 rows for K <= 32, else 64), then thread t < RB builds row t's key.
template <typename KT>
__global__ __launch_bounds__(256) void row_mask_kernel(const int32_t *__restrict__ map, int64_t T, int K, int RB,
                                                       KT *__restrict__ keys, int32_t *__restrict__ iota) {
  extern __shared__ int32_t rows_lds[];
  row_mask_block<KT>(map, T, K, RB, blockIdx.x, keys, iota, KT(0), 0, rows_lds);
}

// ----- row order of maps of at most 8 offsets: a counting sort
//
// With K <= 8 the (count, column mask) key has at most 256 values, so the
// stable sort by (count descending, mask ascending) is one counting pass:
// per-tile bucket counts, one exclusive scan of them in (bucket, tile)
// order (rocPRIM), and a stable scatter.  Bucket of mask m = its place in that order
// (the masks with more columns first).
constexpr int kSmallRowsPerTile = 1024;  // 256 threads x 4 rows

// bucket of every 8-bit mask, built per block in LDS
__device__ __forceinline__ void small_bucket_table(uint8_t *rank_s) {
  const int m = threadIdx.x;  // blockDim.x == 256
  const int c = __builtin_popcount(m);
  int r = 0;
  for (int v = 0; v < 256; ++v) {
    const int cv = __builtin_popcount(v);
    r += (cv > c) || (cv == c && v < m);
  }
  rank_s[m] = static_cast<uint8_t>(r);
}

__device__ __forceinline__ int small_mask(const int32_t *__restrict__ map, int64_t row, int K) {
  int m = 0;
  for (int j = 0; j < K; ++j) m |= (map[row * K + j] >= 0 ? 1 : 0) << j;
  return m;
}

// hist[b * ntiles + tile] = rows of the tile in bucket b
__global__ __launch_bounds__(256) void small_hist_kernel(const int32_t *__restrict__ map, int64_t T, int K,
                                                         int64_t ntiles, int32_t *__restrict__ hist) {
  __shared__ uint8_t rank_s[256];
  __shared__ int cnt_s[256];
  small_bucket_table(rank_s);
  cnt_s[threadIdx.x] = 0;
  __syncthreads();
  const int64_t tile = blockIdx.x;
#pragma unroll
  for (int q = 0; q < kSmallRowsPerTile / 256; ++q) {
    const int64_t row = tile * kSmallRowsPerTile + q * 256 + threadIdx.x;
    if (row < T) atomicAdd(&cnt_s[rank_s[small_mask(map, row, K)]], 1);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * ntiles + tile] = cnt_s[threadIdx.x];
}

// sorted[offs[b * ntiles + tile] + (rank of the row among the tile's rows of
// bucket b)] = row; rows keep their order within a bucket (row quarters in
// turn, then waves, then lanes)
__global__ __launch_bounds__(256) void small_scatter_kernel(const int32_t *__restrict__ map, int64_t T, int K,
                                                            int64_t ntiles, const int32_t *__restrict__ offs,
                                                            int32_t *__restrict__ sorted) {
  __shared__ uint8_t rank_s[256];
  __shared__ int base_s[256];
  __shared__ int wcnt_s[4][256];
  small_bucket_table(rank_s);
  base_s[threadIdx.x] = 0;
  const int64_t tile = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int q = 0; q < kSmallRowsPerTile / 256; ++q) {
#pragma unroll
    for (int w = 0; w < 4; ++w) wcnt_s[w][threadIdx.x] = 0;
    __syncthreads();
    const int64_t row = tile * kSmallRowsPerTile + q * 256 + threadIdx.x;
    const bool valid = row < T;
    const int b = valid ? rank_s[small_mask(map, row, K)] : 0;
    // lanes of the wave with the same bucket (eight ballots on its bits)
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t m = __ballot(valid && ((b >> bit) & 1));
      peers &= ((b >> bit) & 1) ? m : ~m;
    }
    const int rank = __builtin_popcountll(peers & below);
    if (valid && (peers >> lane) == 1) wcnt_s[wave][b] = rank + 1;  // the last lane of the group
    __syncthreads();
    if (valid) {
      int pos = offs[static_cast<int64_t>(b) * ntiles + tile] + base_s[b] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt_s[w][b];
      sorted[pos] = static_cast<int32_t>(row);
    }
    __syncthreads();
    base_s[threadIdx.x] += wcnt_s[0][threadIdx.x] + wcnt_s[1][threadIdx.x] + wcnt_s[2][threadIdx.x] +
                           wcnt_s[3][threadIdx.x];
  }
}

// Per group of 128 sorted rows: the 128-bit union of their valid columns
// (gm[g * 2 + w]) and a sort key that puts the groups with the most columns
// first (128 - popcount) and keeps a trailing partial group last (255).
// K <= 57: the unions come from the sort keys (their low K bits are the
// rows' column masks), one wave per group.
template <typename KT>
__device__ __forceinline__ void group_union_wave(const KT *__restrict__ keys_sorted, int K, int64_t T, int64_t g,
                                                 uint64_t *__restrict__ gm, uint32_t *__restrict__ gkey,
                                                 int32_t *__restrict__ giota) {
  const int lane = threadIdx.x & 63;
  uint64_t m = 0;
  if (keys_sorted) {
    const uint64_t pm = (uint64_t(1) << K) - 1;
    for (int r = lane; r < 128; r += 64) {
      const int64_t row = g * 128 + r;
      if (row < T) m |= static_cast<uint64_t>(keys_sorted[row]) & pm;
    }
    for (int o = 32; o > 0; o >>= 1) m |= static_cast<uint64_t>(__shfl_xor(m, o, 64));
    if (lane == 0) {
      gm[g * 2] = m;
      gm[g * 2 + 1] = 0;
    }
  }
  if (lane == 0) {
    const int pc = __popcll(gm[g * 2]) + __popcll(gm[g * 2 + 1]);
    gkey[g] = (g + 1) * 128 > T ? 255u : static_cast<uint32_t>(128 - pc);
    if (giota) giota[g] = static_cast<int32_t>(g);
  }
}

template <typename KT>
__global__ __launch_bounds__(256) void group_union_keys_kernel(const KT *__restrict__ keys_sorted, int K,
                                                               int64_t T, uint64_t *__restrict__ gm,
                                                               uint32_t *__restrict__ gkey,
                                                               int32_t *__restrict__ giota) {
  const int64_t G = (T + 127) / 128;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (g >= G) return;
  group_union_wave<KT>(keys_sorted, K, T, g, gm, gkey, giota);
}

// Stable counting sort of the G group keys (values < 256): gperm = the
// group ids by key.  The block stages the keys in LDS and builds their
// histogram per quarter of the groups; one wave scans it in (key, quarter)
// order; then each wave walks its quarter in chunks of 64 keys, each lane
// placed at its bin's running base plus its rank among the chunk's lanes
// with the same key (peer masks from eight ballots); the highest lane of
// each key advances the base.
constexpr int kGroupOrderMax = 49152;
__device__ __forceinline__ void group_order_block(const uint32_t *__restrict__ gkey, int G,
                                                  int32_t *__restrict__ gperm) {
  // the four waves rank one contiguous quarter of the groups each; a key's
  // places start at its base plus its count in the quarters before
  __shared__ int base_s[4][256];
  __shared__ uint8_t key_s[kGroupOrderMax];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qlen = (G + 3) / 4;
#pragma unroll
  for (int w = 0; w < 4; ++w) base_s[w][threadIdx.x] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < G; i += 256) {
    const uint32_t k = gkey[i] & 255;
    key_s[i] = static_cast<uint8_t>(k);
    atomicAdd(&base_s[i / qlen][k], 1);
  }
  __syncthreads();
  if (wave == 0) {
    // bases: exclusive scan over (key, quarter); lane l owns keys 4l .. 4l+3
    int c[4][4], t = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        c[q][w] = base_s[w][lane * 4 + q];
        t += c[q][w];
      }
    int incl = t;
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    int run = incl - t;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        base_s[w][lane * 4 + q] = run;
        run += c[q][w];
      }
  }
  __syncthreads();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  const int q0 = wave * qlen, q1 = (q0 + qlen) < G ? (q0 + qlen) : G;
  int *base = base_s[wave];
  for (int c0 = q0; c0 < q1; c0 += 64) {
    const int i = c0 + lane;
    const bool valid = i < q1;
    const int k = valid ? static_cast<int>(key_s[i]) : 0;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t b = __ballot(valid && ((k >> bit) & 1));
      peers &= ((k >> bit) & 1) ? b : ~b;
    }
    const int pos = valid ? base[k] + __popcll(peers & below) : 0;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      gperm[pos] = i;
      if ((peers >> lane) == 1) base[k] += __popcll(peers);  // the highest lane of its key
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(256) void group_order_kernel(const uint32_t *__restrict__ gkey, int G,
                                                          int32_t *__restrict__ gperm) {
  group_order_block(gkey, G, gperm);
}

// Logical row L of the final order is sorted row gperm[L / 128] * 128 +
// L % 128 (groups permuted, rows inside a group kept): order[L] = that
// target, ordered[L, :] = its map row, gmask[L / 128] = its group's union.
// Without gperm the groups keep their sorted places.  A block covers 2
// groups: its threads walk the 256 x K ordered elements linearly (coalesced
// stores, row-contiguous loads).  gm_in / gmask may be null (no masks); with
// gperm == null and gm_in == null the unions are computed here instead, by
// an OR-reduction of the column bits through LDS (K <= 128).
// (block `blk` of one map; `sorted` holds the map's targets + sorted_base)
__device__ __forceinline__ void order_rows_block(const int32_t *__restrict__ map, const int32_t *__restrict__ sorted,
                                                 int32_t sorted_base, const int32_t *__restrict__ gperm, int64_t T,
                                                 int K, int32_t *__restrict__ order, int32_t *__restrict__ ordered,
                                                 const uint64_t *__restrict__ gm_in, uint64_t *__restrict__ gmask,
                                                 int64_t blk) {
  __shared__ uint64_t red[2][2][4];  // [group][word][wave]
  __shared__ int32_t src_s[256];
  const int64_t row0 = blk * 256;
  const int64_t rows = (T - row0) < 256 ? (T - row0) : 256;
  if (threadIdx.x < rows) {
    const int64_t L = row0 + threadIdx.x;
    const int64_t sp = gperm ? static_cast<int64_t>(gperm[L / 128]) * 128 + (L % 128) : L;
    const int32_t t = sorted[sp] - sorted_base;
    src_s[threadIdx.x] = t;
    if (order) order[L] = t;
  }
  __syncthreads();
  const bool reduce = gmask && !gm_in;
  const int64_t n = rows * K;
  uint64_t m[2][2] = {{0, 0}, {0, 0}};
  if (ordered || reduce) {
    // element e = r * K + c of the block's rows (e < 256 K: 32-bit), walked
    // with an incremental (r, c) instead of a division per element
    const int ni = static_cast<int>(n);
    const int dr = 256 / K, dc = 256 - dr * K;
    int r = static_cast<int>(threadIdx.x) / K, c = static_cast<int>(threadIdx.x) - r * K;
    int32_t *dst = ordered ? ordered + row0 * K : nullptr;
    // U elements per round: all U loads are issued before the first store,
    // so that a thread keeps U row gathers in flight
    constexpr int U = 8;
    for (int e0 = threadIdx.x; e0 < ni; e0 += 256 * U) {
      int32_t v[U];
      int cu[U], ru[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ru[u] = r;
        cu[u] = c;
        v[u] = (e0 + u * 256 < ni) ? map[static_cast<int64_t>(src_s[r]) * K + c] : -1;
        r += dr;
        c += dc;
        if (c >= K) {
          c -= K;
          ++r;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (e0 + u * 256 >= ni) continue;
        if (ordered) dst[e0 + u * 256] = v[u];
        if (reduce && v[u] >= 0 && cu[u] < 128) {
          const int gi = ru[u] >= 128 ? 1 : 0;
          if (cu[u] < 64) m[gi][0] |= uint64_t(1) << cu[u];
          else m[gi][1] |= uint64_t(1) << (cu[u] - 64);
        }
      }
    }
  }
  if (!gmask) return;
  if (gm_in) {
    if (threadIdx.x < 4) {
      const int gi = threadIdx.x >> 1, w = threadIdx.x & 1;
      const int64_t g = row0 / 128 + gi;
      if (g * 128 < T) gmask[g * 2 + w] = gm_in[(gperm ? gperm[g] : g) * 2 + w];
    }
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint64_t v = m[gi][w];
      for (int o = 32; o > 0; o >>= 1) v |= static_cast<uint64_t>(__shfl_xor(v, o, 64));
      if (lane == 0) red[gi][w][wave] = v;
    }
  __syncthreads();
  if (threadIdx.x < 4) {
    const int gi = threadIdx.x >> 1, w = threadIdx.x & 1;
    const int64_t g = row0 / 128 + gi;
    if (g * 128 < T) gmask[g * 2 + w] = red[gi][w][0] | red[gi][w][1] | red[gi][w][2] | red[gi][w][3];
  }
}

__global__ __launch_bounds__(256) void order_rows_kernel(const int32_t *__restrict__ map,
                                                         const int32_t *__restrict__ sorted,
                                                         const int32_t *__restrict__ gperm, int64_t T, int K,
                                                         int32_t *__restrict__ order, int32_t *__restrict__ ordered,
                                                         const uint64_t *__restrict__ gm_in,
                                                         uint64_t *__restrict__ gmask) {
  order_rows_block(map, sorted, 0, gperm, T, K, order, ordered, gm_in, gmask, blockIdx.x);
}

// ----- row orders of several maps in one chain of launches
//
// The maps' rows are concatenated, each key prefixed with its map's index
// above the 32 key bits (maps of at most 27 offsets), so that one sort orders
// every map at once and leaves map m's rows at its own row range; the group
// unions, the group order (one block per map) and the ordered rows then run
// as one launch each over all maps.  Every map's result equals
// spira_hip_kmap_row_order's for it alone.
constexpr int kRowBatchMax = 16;
struct RowBatchSeg {
  const int32_t *map;
  int64_t T;
  int K;
  int32_t *order;
  uint64_t *gmask;
  int32_t *ordered;
  int64_t row_base;    // the map's first row among the concatenated rows
  int64_t group_base;  // its first 128-row group
};
struct RowBatch {
  int n;
  RowBatchSeg seg[kRowBatchMax];
  int64_t mask_blk[kRowBatchMax + 1];   // block prefixes: key blocks (256 rows),
  int64_t group_blk[kRowBatchMax + 1];  // group-union blocks (4 groups),
  int64_t rows_blk[kRowBatchMax + 1];   // ordered-row blocks (256 rows)
};
__device__ __forceinline__ int batch_seg(const int64_t *pre, int n, int64_t b) {
  int m = 0;
  while (m + 1 < n && pre[m + 1] <= b) ++m;
  return m;
}

__global__ __launch_bounds__(256) void row_mask_batch_kernel(const RowBatch bt, uint64_t *__restrict__ keys,
                                                             int32_t *__restrict__ iota) {
  extern __shared__ int32_t rows_lds[];
  const int m = batch_seg(bt.mask_blk, bt.n, blockIdx.x);
  const RowBatchSeg &sg = bt.seg[m];
  row_mask_block<uint64_t>(sg.map, sg.T, sg.K, 256, blockIdx.x - bt.mask_blk[m], keys + sg.row_base,
                           iota + sg.row_base, static_cast<uint64_t>(m) << 32, static_cast<int32_t>(sg.row_base),
                           rows_lds);
}

__global__ __launch_bounds__(256) void group_union_batch_kernel(const RowBatch bt,
                                                                const uint64_t *__restrict__ keys_sorted,
                                                                uint64_t *__restrict__ gm,
                                                                uint32_t *__restrict__ gkey) {
  const int m = batch_seg(bt.group_blk, bt.n, blockIdx.x);
  const RowBatchSeg &sg = bt.seg[m];
  const int64_t g = (blockIdx.x - bt.group_blk[m]) * 4 + (threadIdx.x >> 6);
  if (g >= (sg.T + 127) / 128) return;
  group_union_wave<uint64_t>(keys_sorted + sg.row_base, sg.K, sg.T, g, gm + 2 * sg.group_base,
                             gkey + sg.group_base, nullptr);
}

__global__ __launch_bounds__(256) void group_order_batch_kernel(const RowBatch bt, const uint32_t *__restrict__ gkey,
                                                                int32_t *__restrict__ gperm) {
  const RowBatchSeg &sg = bt.seg[blockIdx.x];
  group_order_block(gkey + sg.group_base, static_cast<int>((sg.T + 127) / 128), gperm + sg.group_base);
}

__global__ __launch_bounds__(256) void order_rows_batch_kernel(const RowBatch bt, const int32_t *__restrict__ sorted,
                                                               const int32_t *__restrict__ gperm,
                                                               const uint64_t *__restrict__ gm) {
  const int m = batch_seg(bt.rows_blk, bt.n, blockIdx.x);
  const RowBatchSeg &sg = bt.seg[m];
  order_rows_block(sg.map, sorted + sg.row_base, static_cast<int32_t>(sg.row_base), gperm + sg.group_base, sg.T,
                   sg.K, sg.order, sg.ordered, gm + 2 * sg.group_base, sg.gmask, blockIdx.x - bt.rows_blk[m]);
}

// Workspace of the row order: sort keys (in / out), row ids, sorted rows,
// the group pass (unions, keys in / out, ids, permutation) and the larger of
// the two sorts' temporary storage.
struct RowOrderParts {
  uint64_t *keys, *keys_out, *gm;
  int32_t *iota, *sorted, *giota, *gperm;
  uint32_t *gkey, *gkey_out;
  void *tmp;
  size_t tmp_bytes, total;
};
static RowOrderParts row_order_parts(int64_t T, void *base) {
  const int64_t G = (T + 127) / 128;
  size_t b1 = 0, b2 = 0, b3 = 0;
  (void)rocprim::radix_sort_pairs(nullptr, b1, static_cast<const uint64_t *>(nullptr),
                                  static_cast<uint64_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(T), 0, 64);
  (void)rocprim::radix_sort_pairs(nullptr, b3, static_cast<const uint32_t *>(nullptr),
                                  static_cast<uint32_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(T), 0, 32);
  (void)rocprim::radix_sort_pairs(nullptr, b2, static_cast<const uint32_t *>(nullptr),
                                  static_cast<uint32_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(G), 0, 8);
  RowOrderParts r{};
  const int64_t small_counts = 256 * ((T + kSmallRowsPerTile - 1) / kSmallRowsPerTile);
  size_t b4 = 0;
  (void)rocprim::exclusive_scan(nullptr, b4, static_cast<const int32_t *>(nullptr), static_cast<int32_t *>(nullptr), 0,
                                static_cast<size_t>(small_counts), rocprim::plus<int32_t>());
  r.tmp_bytes = std::max(std::max(std::max(b1, b2), b3), b4);
  char *p = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = p ? p + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return q;
  };
  // (also the bucket counts of the counting sort of maps of <= 8 offsets
  // and their scan: 256 per 1024-row tile)
  const size_t kb = std::max<size_t>(T * sizeof(uint64_t), small_counts * sizeof(int32_t));
  r.keys = reinterpret_cast<uint64_t *>(take(kb));
  r.keys_out = reinterpret_cast<uint64_t *>(take(kb));
  r.iota = reinterpret_cast<int32_t *>(take(T * sizeof(int32_t)));
  r.sorted = reinterpret_cast<int32_t *>(take(T * sizeof(int32_t)));
  r.gm = reinterpret_cast<uint64_t *>(take(G * 2 * sizeof(uint64_t)));
  r.gkey = reinterpret_cast<uint32_t *>(take(G * sizeof(uint32_t)));
  r.gkey_out = reinterpret_cast<uint32_t *>(take(G * sizeof(uint32_t)));
  r.giota = reinterpret_cast<int32_t *>(take(G * sizeof(int32_t)));
  r.gperm = reinterpret_cast<int32_t *>(take(G * sizeof(int32_t)));
  r.tmp = take(r.tmp_bytes);
  r.total = off;
  return r;
}

struct RowBatchParts {
  uint64_t *keys, *keys_out, *gm;
  int32_t *iota, *sorted, *gperm;
  uint32_t *gkey;
  void *tmp;
  size_t tmp_bytes, total;
};
static RowBatchParts row_batch_parts(int64_t N, int64_t G, int nmaps, void *base) {
  size_t b = 0;
  const int hi = 32 + (nmaps > 1 ? 32 - __builtin_clz(static_cast<unsigned>(nmaps - 1)) : 0);
  (void)rocprim::radix_sort_pairs(nullptr, b, static_cast<const uint64_t *>(nullptr),
                                  static_cast<uint64_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(N), 0, hi);
  RowBatchParts r{};
  r.tmp_bytes = b;
  char *p = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = p ? p + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return q;
  };
  r.keys = reinterpret_cast<uint64_t *>(take(N * 8));
  r.keys_out = reinterpret_cast<uint64_t *>(take(N * 8));
  r.iota = reinterpret_cast<int32_t *>(take(N * 4));
  r.sorted = reinterpret_cast<int32_t *>(take(N * 4));
  r.gm = reinterpret_cast<uint64_t *>(take(G * 16));
  r.gkey = reinterpret_cast<uint32_t *>(take(G * 4));
  r.gperm = reinterpret_cast<int32_t *>(take(G * 4));
  r.tmp = take(r.tmp_bytes);
  r.total = off;
  return r;
}

// Validates a batch of row-order jobs and fills the launch table.
static int make_row_batch(int n, const spira_hip_row_order_job_t *jobs, RowBatch &bt, int64_t &N, int64_t &G) {
  SPIRA_HIP_REQUIRE(n >= 1 && n <= kRowBatchMax, "kmap_row_order_batch: 1 to 16 maps");
  SPIRA_HIP_REQUIRE(jobs != nullptr, "kmap_row_order_batch: null jobs");
  bt = RowBatch{};
  bt.n = n;
  N = G = 0;
  int64_t mb = 0, gb = 0, rb = 0;
  for (int m = 0; m < n; ++m) {
    const spira_hip_row_order_job_t &j = jobs[m];
    SPIRA_HIP_REQUIRE(j.out_in_map && j.order && j.group_masks && j.ordered_map,
                      "kmap_row_order_batch: null map or output");
    SPIRA_HIP_REQUIRE(j.num_targets >= 1 && j.num_offsets >= 1 && row_key_bits(j.num_offsets) <= 32,
                      "kmap_row_order_batch: every map needs targets and at most 27 offsets");
    const int64_t Gm = div_up(j.num_targets, 128);
    SPIRA_HIP_REQUIRE(Gm <= kGroupOrderMax, "kmap_row_order_batch: too many rows in one map");
    bt.seg[m] = RowBatchSeg{j.out_in_map, j.num_targets, j.num_offsets, j.order, j.group_masks, j.ordered_map, N, G};
    bt.mask_blk[m] = mb;
    bt.group_blk[m] = gb;
    bt.rows_blk[m] = rb;
    mb += div_up(j.num_targets, 256);
    gb += div_up(Gm, 4);
    rb += div_up(j.num_targets, 256);
    N += j.num_targets;
    G += Gm;
  }
  bt.mask_blk[n] = mb;
  bt.group_blk[n] = gb;
  bt.rows_blk[n] = rb;
  SPIRA_HIP_REQUIRE(N < (int64_t(1) << 31), "kmap_row_order_batch: too many rows");
  return kOk;
}

static size_t scan_temp_bytes(int64_t n) {
  size_t b = 0;
  (void)rocprim::exclusive_scan(nullptr, b, static_cast<const int32_t *>(nullptr), static_cast<int32_t *>(nullptr), 0,
                          static_cast<size_t>(n), rocprim::plus<int32_t>());
  return b;
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_kmap_search(const void *sources, int64_t num_sources, const void *targets, int64_t num_targets,
                          int key_bits, int kx, int ky, int kz, int sx, int sy, int sz, int layout,
                          const int32_t *row_perm, int32_t *kernel_map, int32_t *tile_counts, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "kmap_search: key_bits must be 32 or 64");
  if (key_bits == 64)
    return search_impl<uint64_t>(static_cast<const uint64_t *>(sources), num_sources,
                                 static_cast<const uint64_t *>(targets), num_targets, kx, ky, kz, sx, sy, sz, layout,
                                 row_perm, kernel_map, tile_counts, stream);
  return search_impl<uint32_t>(static_cast<const uint32_t *>(sources), num_sources,
                               static_cast<const uint32_t *>(targets), num_targets, kx, ky, kz, sx, sy, sz, layout,
                               row_perm, kernel_map, tile_counts, stream);
}

int spira_hip_kmap_search_batch(int n, const spira_hip_kmap_job_t *jobs, int key_bits, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "kmap_search_batch: key_bits must be 32 or 64");
  SPIRA_HIP_REQUIRE(n >= 0 && (n == 0 || jobs != nullptr), "kmap_search_batch: bad job list");
  if (key_bits == 64) return search_batch_impl<uint64_t>(n, jobs, stream);
  return search_batch_impl<uint32_t>(n, jobs, stream);
}

int spira_hip_kmap_scan_workspace(int64_t num_counts, size_t *bytes) {
  *bytes = num_counts <= 0 ? 0 : scan_temp_bytes(num_counts);
  return kOk;
}

int spira_hip_kmap_scan(const int32_t *tile_counts, int rows, int64_t ntiles, int quantum, int32_t *tile_offsets,
                        int32_t *nbsizes, int32_t *naddrs, int32_t *qnaddrs, int32_t *sizes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(rows >= 0 && rows <= kOffsetsMax, "kmap_scan: rows out of range");
  SPIRA_HIP_REQUIRE(quantum >= 1, "kmap_scan: quantum must be positive");
  const int64_t n = static_cast<int64_t>(rows) * ntiles;
  if (n == 0) {
    // empty: every size is zero
    if (naddrs) { int rc = fill_i32(naddrs, rows + 1, 0, stream); if (rc) return rc; }
    if (qnaddrs) { int rc = fill_i32(qnaddrs, rows + 1, 0, stream); if (rc) return rc; }
    if (nbsizes) { int rc = fill_i32(nbsizes, rows, 0, stream); if (rc) return rc; }
    if (sizes) return fill_i32(sizes, 2, 0, stream);
    return kOk;
  }
  size_t need = scan_temp_bytes(n);
  SPIRA_HIP_REQUIRE(workspace != nullptr && workspace_bytes >= need, "kmap_scan: workspace too small");
  SPIRA_HIP_TRY(rocprim::exclusive_scan(workspace, need, tile_counts, tile_offsets, 0, static_cast<size_t>(n),
                                        rocprim::plus<int32_t>(), stream));
  hipLaunchKernelGGL(row_totals_kernel, dim3(1), dim3(kOffsetsMax), 0, stream, tile_counts, tile_offsets, rows,
                     ntiles, quantum, nbsizes, naddrs, qnaddrs, sizes);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_kmap_emit_pairs(const int32_t *kernel_map, int64_t aligned_targets, int row0, int rows,
                              const int32_t *tile_offsets, int32_t *in_idx, int32_t *out_idx, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(aligned_targets % 128 == 0, "kmap_emit_pairs: aligned_targets must be a multiple of 128");
  const int64_t ntiles = aligned_targets / 64;
  const int64_t waves = static_cast<int64_t>(rows) * ntiles;
  if (waves == 0) return kOk;
  hipLaunchKernelGGL(emit_pairs_kernel, dim3(div_up(waves, 4)), dim3(256), 0, stream, kernel_map, aligned_targets,
                     row0, rows, ntiles, tile_offsets, in_idx, out_idx);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_kmap_emit_masks(const int32_t *kernel_map, int64_t num_sources, int64_t num_targets,
                              int64_t aligned_targets, int row0, int rows, int mask_rows, int half,
                              const int32_t *tile_offsets, int32_t *source_masks, int32_t *target_masks,
                              hipStream_t stream) {
  SPIRA_HIP_REQUIRE(aligned_targets % 128 == 0, "kmap_emit_masks: aligned_targets must be a multiple of 128");
  SPIRA_HIP_REQUIRE(!half || num_sources == num_targets, "kmap_emit_masks: half masks need S == T");
  SPIRA_HIP_REQUIRE(rows <= mask_rows, "kmap_emit_masks: more compacted rows than mask rows");
  int rc = fill_i32(source_masks, static_cast<int64_t>(mask_rows) * num_sources, -1, stream);
  if (rc) return rc;
  rc = fill_i32(target_masks, static_cast<int64_t>(mask_rows) * num_targets, -1, stream);
  if (rc) return rc;
  const int64_t ntiles = aligned_targets / 64;
  const int64_t waves = static_cast<int64_t>(rows) * ntiles;
  if (waves == 0) return kOk;
  hipLaunchKernelGGL(emit_masks_kernel, dim3(div_up(waves, 4)), dim3(256), 0, stream, kernel_map, num_sources,
                     num_targets, aligned_targets, row0, rows, mask_rows, half, ntiles, tile_offsets, source_masks,
                     target_masks);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_convert_transposed_os(const int32_t *out_in_map, int64_t aligned_targets, int num_offsets,
                                    int64_t aligned_sources, int32_t *out, hipStream_t stream) {
  int rc = fill_i32(out, aligned_sources * num_offsets, -1, stream);
  if (rc) return rc;
  const int64_t n = aligned_targets * num_offsets;
  if (n == 0) return kOk;
  hipLaunchKernelGGL(convert_transposed_kernel, dim3(div_up(n, 256)), dim3(256), 0, stream, out_in_map, n,
                     num_offsets, out);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_fill_i32(int32_t *ptr, int64_t n, int32_t value, hipStream_t stream) {
  return fill_i32(ptr, n, value, stream);
}

int spira_hip_convert_transposed_os_partition(const int32_t *out_in_map, int64_t aligned_targets, int num_offsets,
                                              int64_t num_sources, int64_t aligned_sources, int32_t *out,
                                              hipStream_t stream) {
  SPIRA_HIP_REQUIRE(num_offsets >= 1 && num_sources >= 0 && aligned_sources >= num_sources,
                    "convert_transposed_os_partition: bad sizes");
  const int64_t n = aligned_targets * num_offsets, pad = (aligned_sources - num_sources) * num_offsets;
  if (n + pad == 0) return kOk;
  hipLaunchKernelGGL(convert_transposed_partition_kernel, dim3(div_up(n + pad, 256)), dim3(256), 0, stream,
                     out_in_map, n, num_offsets, num_sources, aligned_sources, out);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_convert_transposed_os_partition_order_workspace(int64_t num_coarse, int num_offsets, size_t *bytes) {
  const int64_t ntiles = div_up(std::max<int64_t>(num_coarse, 1), kTpTile);
  *bytes = static_cast<size_t>(num_offsets * ntiles) * sizeof(int32_t);
  return kOk;
}

int spira_hip_convert_transposed_os_partition_order(const int32_t *out_in_map, int64_t num_coarse, int num_offsets,
                                                    int64_t num_sources, int64_t aligned_sources, int32_t *out,
                                                    int32_t *order, int32_t *ordered_map, uint64_t *group_masks,
                                                    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  const int K = num_offsets;
  SPIRA_HIP_REQUIRE(K >= 1 && K <= kTpMaxK, "convert_transposed_os_partition_order: at most 8 offsets");
  SPIRA_HIP_REQUIRE(num_coarse >= 0 && num_sources >= 0 && aligned_sources >= num_sources &&
                        num_sources < (int64_t(1) << 31),
                    "convert_transposed_os_partition_order: bad sizes");
  const int64_t ntiles = div_up(std::max<int64_t>(num_coarse, 1), kTpTile);
  SPIRA_HIP_REQUIRE(K * ntiles <= kTpMaxCounts, "convert_transposed_os_partition_order: too many coarse rows");
  SPIRA_HIP_REQUIRE(workspace != nullptr && workspace_bytes >= static_cast<size_t>(K * ntiles) * sizeof(int32_t),
                    "convert_transposed_os_partition_order: workspace too small");
  if (num_sources == 0 && aligned_sources == 0) return kOk;
  int32_t *cnt = static_cast<int32_t *>(workspace);
  hipLaunchKernelGGL(tp_count_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(kTpTile), 0, stream, out_in_map,
                     num_coarse, K, static_cast<int>(ntiles), cnt, num_sources, aligned_sources, out, ordered_map);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(tp_emit_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(kTpTile), 0, stream, out_in_map,
                     num_coarse, K, static_cast<int>(ntiles), cnt, num_sources, order, ordered_map, out, group_masks);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_kmap_row_order_workspace(int64_t num_targets, size_t *bytes) {
  *bytes = num_targets <= 0 ? 0 : row_order_parts(num_targets, nullptr).total;
  return kOk;
}

int spira_hip_kmap_row_order(const int32_t *out_in_map, int64_t num_targets, int num_offsets, int32_t *order,
                             uint64_t *group_masks, int32_t *ordered_map, void *workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  SPIRA_HIP_REQUIRE(num_targets >= 0 && num_targets < (int64_t(1) << 31), "kmap_row_order: size out of range");
  SPIRA_HIP_REQUIRE(num_offsets >= 1, "kmap_row_order: no offsets");
  SPIRA_HIP_REQUIRE(group_masks == nullptr || num_offsets <= 128, "kmap_row_order: group masks need <= 128 offsets");
  if (num_targets == 0) return kOk;
  SPIRA_HIP_REQUIRE(workspace != nullptr && workspace_bytes >= row_order_parts(num_targets, nullptr).total,
                    "kmap_row_order: workspace too small");
  RowOrderParts w = row_order_parts(num_targets, workspace);
  if (num_offsets <= 8) {
    // counting sort (bucket counts in w.keys, their scan in w.keys_out),
    // then the rows in that order with their 128-row column unions
    const int64_t ntiles = div_up(num_targets, kSmallRowsPerTile);
    int32_t *hist = reinterpret_cast<int32_t *>(w.keys), *offs = reinterpret_cast<int32_t *>(w.keys_out);
    hipLaunchKernelGGL(small_hist_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(256), 0, stream, out_in_map,
                       num_targets, num_offsets, ntiles, hist);
    SPIRA_HIP_LAUNCH_CHECK();
    size_t stb = w.tmp_bytes;
    SPIRA_HIP_TRY(rocprim::exclusive_scan(w.tmp, stb, hist, offs, 0, static_cast<size_t>(256 * ntiles),
                                          rocprim::plus<int32_t>(), stream));
    hipLaunchKernelGGL(small_scatter_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(256), 0, stream, out_in_map,
                       num_targets, num_offsets, ntiles, offs, w.sorted);
    SPIRA_HIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(order_rows_kernel, dim3(div_up(num_targets, 256)), dim3(256), 0, stream, out_in_map, w.sorted,
                       static_cast<const int32_t *>(nullptr), num_targets, num_offsets, order, ordered_map,
                       static_cast<const uint64_t *>(nullptr), group_masks);
    SPIRA_HIP_LAUNCH_CHECK();
    return kOk;
  }
  const int rb = num_offsets <= 32 ? 256 : 64;
  SPIRA_HIP_REQUIRE(static_cast<size_t>(rb) * num_offsets * sizeof(int32_t) <= 64 * 1024,
                    "kmap_row_order: at most 256 offsets");
  // 32-bit sort keys when they fit (kernels of <= 27 offsets): the sort
  // moves half the key bytes
  const int kbits = row_key_bits(num_offsets);
  const bool k32 = kbits <= 32;
  size_t tb = w.tmp_bytes;
  if (k32) {
    uint32_t *keys = reinterpret_cast<uint32_t *>(w.keys), *keys_out = reinterpret_cast<uint32_t *>(w.keys_out);
    hipLaunchKernelGGL(row_mask_kernel<uint32_t>, dim3(div_up(num_targets, rb)), dim3(256),
                       rb * num_offsets * sizeof(int32_t), stream, out_in_map, num_targets, num_offsets, rb, keys,
                       w.iota);
    SPIRA_HIP_LAUNCH_CHECK();
    SPIRA_HIP_TRY(rocprim::radix_sort_pairs(w.tmp, tb, keys, keys_out, w.iota, w.sorted,
                                            static_cast<size_t>(num_targets), 0, kbits, stream));
  } else {
    hipLaunchKernelGGL(row_mask_kernel<uint64_t>, dim3(div_up(num_targets, rb)), dim3(256),
                       rb * num_offsets * sizeof(int32_t), stream, out_in_map, num_targets, num_offsets, rb, w.keys,
                       w.iota);
    SPIRA_HIP_LAUNCH_CHECK();
    SPIRA_HIP_TRY(rocprim::radix_sort_pairs(w.tmp, tb, w.keys, w.keys_out, w.iota, w.sorted,
                                            static_cast<size_t>(num_targets), 0, kbits, stream));
  }
  const int64_t G = div_up(num_targets, 128);
  const int32_t *gperm = nullptr;
  const uint64_t *gm = nullptr;
  if (group_masks) {
    // group unions, then the groups with the most columns first: the
    // longest blocks start first
    const bool from_keys = num_offsets <= 57;  // the sort keys hold the whole column mask
    if (!from_keys) {
      hipLaunchKernelGGL(order_rows_kernel, dim3(div_up(num_targets, 256)), dim3(256), 0, stream, out_in_map,
                         w.sorted, static_cast<const int32_t *>(nullptr), num_targets, num_offsets,
                         static_cast<int32_t *>(nullptr), static_cast<int32_t *>(nullptr),
                         static_cast<const uint64_t *>(nullptr), w.gm);
      SPIRA_HIP_LAUNCH_CHECK();
    }
    if (k32)
      hipLaunchKernelGGL(group_union_keys_kernel<uint32_t>, dim3(div_up(G, 4)), dim3(256), 0, stream,
                         from_keys ? reinterpret_cast<const uint32_t *>(w.keys_out) : nullptr, num_offsets,
                         num_targets, w.gm, w.gkey, w.giota);
    else
      hipLaunchKernelGGL(group_union_keys_kernel<uint64_t>, dim3(div_up(G, 4)), dim3(256), 0, stream,
                         from_keys ? w.keys_out : static_cast<const uint64_t *>(nullptr), num_offsets, num_targets,
                         w.gm, w.gkey, w.giota);
    SPIRA_HIP_LAUNCH_CHECK();
    // (a few thousand groups: one wave beats a device-wide sort's launches)
    if (G <= kGroupOrderMax) {
      hipLaunchKernelGGL(group_order_kernel, dim3(1), dim3(256), 0, stream, w.gkey, static_cast<int>(G), w.gperm);
      SPIRA_HIP_LAUNCH_CHECK();
    } else {
      tb = w.tmp_bytes;
      SPIRA_HIP_TRY(rocprim::radix_sort_pairs(w.tmp, tb, w.gkey, w.gkey_out, w.giota, w.gperm,
                                              static_cast<size_t>(G), 0, 8, stream));
    }
    gperm = w.gperm;
    gm = w.gm;
  }
  hipLaunchKernelGGL(order_rows_kernel, dim3(div_up(num_targets, 256)), dim3(256), 0, stream, out_in_map, w.sorted,
                     gperm, num_targets, num_offsets, order, ordered_map, gm, group_masks);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_kmap_row_order_batch_workspace(int n, const spira_hip_row_order_job_t *jobs, size_t *bytes) {
  RowBatch bt;
  int64_t N = 0, G = 0;
  const int rc = make_row_batch(n, jobs, bt, N, G);
  if (rc) return rc;
  *bytes = row_batch_parts(N, G, n, nullptr).total;
  return kOk;
}

int spira_hip_kmap_row_order_batch(int n, const spira_hip_row_order_job_t *jobs, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  RowBatch bt;
  int64_t N = 0, G = 0;
  const int rc = make_row_batch(n, jobs, bt, N, G);
  if (rc) return rc;
  SPIRA_HIP_REQUIRE(workspace != nullptr && workspace_bytes >= row_batch_parts(N, G, n, nullptr).total,
                    "kmap_row_order_batch: workspace too small");
  RowBatchParts w = row_batch_parts(N, G, n, workspace);
  int kmax = 1;
  for (int m = 0; m < n; ++m) kmax = std::max(kmax, jobs[m].num_offsets);
  hipLaunchKernelGGL(row_mask_batch_kernel, dim3(static_cast<unsigned>(bt.mask_blk[n])), dim3(256),
                     256 * kmax * sizeof(int32_t), stream, bt, w.keys, w.iota);
  SPIRA_HIP_LAUNCH_CHECK();
  const int hi = 32 + (n > 1 ? 32 - __builtin_clz(static_cast<unsigned>(n - 1)) : 0);
  // (rocPRIM: at 438k keys of 34 bits it measured ahead of radix.hip's sort,
  // config-4 step 2.418 against 2.434 ms)
  size_t tb = w.tmp_bytes;
  SPIRA_HIP_TRY(rocprim::radix_sort_pairs(w.tmp, tb, w.keys, w.keys_out, w.iota, w.sorted, static_cast<size_t>(N), 0,
                                          hi, stream));
  hipLaunchKernelGGL(group_union_batch_kernel, dim3(static_cast<unsigned>(bt.group_blk[n])), dim3(256), 0, stream, bt,
                     w.keys_out, w.gm, w.gkey);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(group_order_batch_kernel, dim3(static_cast<unsigned>(n)), dim3(256), 0, stream, bt, w.gkey,
                     w.gperm);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(order_rows_batch_kernel, dim3(static_cast<unsigned>(bt.rows_blk[n])), dim3(256), 0, stream, bt,
                     w.sorted, w.gperm, w.gm);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

}  // extern "C"
