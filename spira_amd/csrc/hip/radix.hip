// Stable LSD radix sort of (key, int32 value) pairs for gfx950, exported as
// spira_hip_radix_sort_pairs.  Measured on MI355X it is slower than
// rocPRIM's merge-path sort at the sizes of the benchmark scenes (200k
// 64-bit keys: ~110 us against ~75 us; every pass is bound by the latency of
// one tile's load -> rank -> look-back -> scatter chain at this size), so
// flatten_sort and the row order keep rocPRIM.
//
// Reference semantics: FlattenSort (arg_sort_coodrinates.cu:36-88) sorts the
// packed keys with their original indices, ascending and stable (CUB
// DeviceRadixSort::SortPairs).  This sort gives the same order.
//
// Design (one digit of 8 bits per pass, keys of 32 or 64 bits):
//   rs_hist_kernel   per 2048-key tile: the histograms of every digit of the
//                    tile (the digit counts do not depend on the key order,
//                    so one read of the keys serves all passes); also clears
//                    the tile's look-back words of every pass;
//   rs_scan_kernel   one block per pass: global digit counts -> digit base
//                    offsets; a pass whose digit is the same for every key is
//                    marked trivial and skipped (the remaining passes
//                    alternate buffers so that the last one writes the
//                    output);
//   rs_pass_kernel   per pass (trivial passes return at once): a block takes
//                    the next tile in ticket order, ranks its keys stably per
//                    digit (wave-level peer masks from 8 ballots, per-wave
//                    running counts in LDS), publishes its digit counts and
//                    finds its offset per digit by a decoupled look-back over
//                    the tiles before it, then scatters.
// The look-back waits only on tiles with smaller tickets, which started
// earlier and are resident or done; the wait is bounded all the same.
#include "common.hpp"
#include "../../../include/spira_hip.h"

namespace spira_hip {

namespace radix {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kItems = 8;                       // keys per thread
constexpr int kTile = kThreads * kItems;        // keys per tile
constexpr int kWaveKeys = kTile / kWaves;       // contiguous keys per wave
constexpr int kBins = 256;
constexpr uint32_t kFlagAgg = 1u << 30;         // look-back word: tile count only
constexpr uint32_t kFlagPrefix = 2u << 30;      // look-back word: inclusive prefix
constexpr uint32_t kCountMask = (1u << 30) - 1;
constexpr int kSpinLimit = 1 << 22;

// device-side control block of one sort
struct Ctrl {
  uint32_t base[8][kBins];  // digit base offsets per pass
  int32_t trivial[8];       // the pass's digit is the same for every key
  uint32_t ticket[8];
  uint32_t stalled;         // a look-back wait ran out (never expected)
};

// Buffers of pass `pass` (0 input, 1 output, 2 temp), or src = -1 for a
// skipped pass: the live passes alternate between output and temp so that
// the last one writes the output; with no live pass, pass 0 copies.
template <int D> __device__ __forceinline__ void pass_buffers(const Ctrl *ctrl, int pass, int &src, int &dst) {
  int live = 0, k = 0;
#pragma unroll
  for (int p = 0; p < D; ++p) live += ctrl->trivial[p] ? 0 : 1;
  const bool none = live == 0;
  if (none) live = 1;
  src = 0;
  dst = -1;
  for (int p = 0; p <= pass; ++p) {
    if (ctrl->trivial[p] && !(none && p == 0)) {
      if (p == pass) src = -1;
      continue;
    }
    ++k;
    const int d = ((live - k) % 2 == 0) ? 1 : 2;
    if (p == pass) dst = d;
    else src = d;
  }
}

template <typename CT> __device__ __forceinline__ uint32_t digit(CT k, int pass) {
  return static_cast<uint32_t>(k >> (8 * pass)) & 0xFFu;
}

template <typename CT>
__global__ __launch_bounds__(kThreads) void rs_hist_kernel(const CT *__restrict__ keys, int64_t n, int ntiles,
                                                           uint32_t *__restrict__ tile_hist,
                                                           uint32_t *__restrict__ status) {
  constexpr int D = sizeof(CT);
  __shared__ uint32_t h[D][kBins];
  const int tid = threadIdx.x;
  for (int i = tid; i < D * kBins; i += kThreads) (&h[0][0])[i] = 0;
  // this tile's look-back words of every pass start cleared
  for (int p = 0; p < D; ++p) status[(static_cast<int64_t>(p) * ntiles + blockIdx.x) * kBins + tid] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  const int lane = tid & 63;
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = base + j * kThreads + tid;
    const bool ok = i < n;
    const CT k = ok ? keys[i] : CT(0);
    const uint64_t valid = __ballot(ok);
#pragma unroll
    for (int p = 0; p < D; ++p) {
      // a digit shared by the whole wave (the common case for the high
      // digits) is one LDS add instead of 64 contending ones
      const uint32_t d = digit(k, p);
      const uint32_t d0 = __builtin_amdgcn_readfirstlane(d);
      if (__ballot(d == d0) == __ballot(true) && valid == __ballot(true)) {
        if (lane == 0) atomicAdd(&h[p][d0], 64u);
      } else if (ok) {
        atomicAdd(&h[p][d], 1u);
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < D * kBins; i += kThreads)
    tile_hist[static_cast<int64_t>(blockIdx.x) * D * kBins + i] = (&h[0][0])[i];
}

// one block per pass: the pass's global digit counts, their exclusive scan,
// and whether the pass is trivial
template <typename CT>
__global__ __launch_bounds__(kThreads) void rs_scan_kernel(const uint32_t *__restrict__ tile_hist, int ntiles,
                                                           int64_t n, Ctrl *__restrict__ ctrl) {
  constexpr int D = sizeof(CT);
  __shared__ uint32_t tot[kBins];
  __shared__ int trivial;
  const int tid = threadIdx.x, p = blockIdx.x;
  // 8 independent loads in flight per thread
  constexpr int kIlp = 8;
  uint32_t acc[kIlp];
#pragma unroll
  for (int q = 0; q < kIlp; ++q) acc[q] = 0;
  int t0 = 0;
  for (; t0 + kIlp <= ntiles; t0 += kIlp)
#pragma unroll
    for (int q = 0; q < kIlp; ++q) acc[q] += tile_hist[(static_cast<int64_t>(t0 + q) * D + p) * kBins + tid];
  for (; t0 < ntiles; ++t0) acc[0] += tile_hist[(static_cast<int64_t>(t0) * D + p) * kBins + tid];
  uint32_t c = 0;
#pragma unroll
  for (int q = 0; q < kIlp; ++q) c += acc[q];
  tot[tid] = c;
  if (tid == 0) trivial = 0;
  __syncthreads();
  if (c == static_cast<uint32_t>(n)) trivial = 1;  // every key has this digit
  // exclusive scan of the 256 counts (Hillis-Steele in LDS)
  for (int off = 1; off < kBins; off <<= 1) {
    const uint32_t v = tid >= off ? tot[tid - off] : 0u;
    __syncthreads();
    tot[tid] += v;
    __syncthreads();
  }
  ctrl->base[p][tid] = tot[tid] - c;
  if (tid == 0) {
    ctrl->trivial[p] = trivial;
    ctrl->ticket[p] = 0;
    if (p == 0) ctrl->stalled = 0;
  }
}

// the three buffers of a sort: 0 input, 1 output, 2 temporary
template <typename CT> struct Bufs {
  const CT *k0;
  CT *k1, *k2;
  const int32_t *v0;
  int32_t *v1, *v2;
};

template <typename CT>
__global__ __launch_bounds__(kThreads) void rs_pass_kernel(int pass, int64_t n, int ntiles, Bufs<CT> b,
                                                           uint32_t *__restrict__ status, Ctrl *__restrict__ ctrl) {
  int src, dst;
  pass_buffers<sizeof(CT)>(ctrl, pass, src, dst);
  if (src < 0) return;  // trivial pass (block-uniform)
  __shared__ uint32_t wcnt[kWaves][kBins];
  __shared__ uint32_t excl[kBins];
  __shared__ int s_tile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Tiles in ticket order, so that every tile a look-back waits on has
  // started, whatever order the hardware dispatches the blocks in.
  if (tid == 0) s_tile = static_cast<int>(atomicAdd(&ctrl->ticket[pass], 1u));
  for (int i = tid; i < kWaves * kBins; i += kThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  const int tile = s_tile;
  const CT *__restrict__ kin = src == 0 ? b.k0 : (src == 1 ? b.k1 : b.k2);
  const int32_t *__restrict__ vin = src == 0 ? b.v0 : (src == 1 ? b.v1 : b.v2);
  CT *__restrict__ kout = dst == 1 ? b.k1 : b.k2;
  int32_t *__restrict__ vout = dst == 1 ? b.v1 : b.v2;
  // wave w ranks the contiguous keys [w * kWaveKeys, (w + 1) * kWaveKeys) of
  // the tile in rounds of 64, in order: stable within the tile
  const int64_t wbase = static_cast<int64_t>(tile) * kTile + wave * kWaveKeys;
  CT key[kItems];
  int32_t val[kItems];
  uint32_t rank[kItems];
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    const bool ok = i < n;
    key[j] = ok ? kin[i] : CT(0);
    val[j] = ok ? vin[i] : 0;
  }
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    const bool ok = i < n;
    const uint32_t d = digit(key[j], pass);
    uint64_t peers = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t m = __ballot((d >> bit) & 1u);
      peers &= ((d >> bit) & 1u) ? m : ~m;
    }
    const uint32_t before = wcnt[wave][d];
    rank[j] = before + static_cast<uint32_t>(__builtin_popcountll(peers & lt));
    // the group's first lane advances the wave's count of the digit
    const bool leader = ok && (peers & lt) == 0;
    __builtin_amdgcn_wave_barrier();
    if (leader) wcnt[wave][d] = before + static_cast<uint32_t>(__builtin_popcountll(peers));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __syncthreads();
  // the tile's count of digit tid, and the waves' exclusive prefixes
  {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t v = wcnt[w][tid];
      wcnt[w][tid] = c;
      c += v;
    }
    uint32_t *st = status + (static_cast<int64_t>(pass) * ntiles) * kBins + tid;
    if (tile == 0) {
      __hip_atomic_store(st, kFlagPrefix | c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      excl[tid] = 0;
    } else {
      __hip_atomic_store(st + static_cast<int64_t>(tile) * kBins, kFlagAgg | c, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      // look back over up to kWindow tiles at a time (independent loads):
      // add tile counts until an inclusive prefix; a tile that has not
      // published yet is waited for
      constexpr int kWindow = 32;
      uint32_t e = 0;
      int t = tile - 1, spins = 0;
      bool done = false;
      while (!done && t >= 0) {
        uint32_t w[kWindow];
#pragma unroll
        for (int q = 0; q < kWindow; ++q)
          w[q] = t - q >= 0 ? __hip_atomic_load(st + static_cast<int64_t>(t - q) * kBins, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0u;
        int q = 0;
        for (; q < kWindow && t - q >= 0; ++q) {
          if ((w[q] & ~kCountMask) == 0) break;  // not published yet: wait from here
          e += w[q] & kCountMask;
          if (w[q] & kFlagPrefix) {
            done = true;
            break;
          }
        }
        if (done) break;
        t -= q;
        if (q < kWindow && t >= 0) {
          if (++spins > kSpinLimit) {  // bounded: never expected (earlier tickets are running)
            atomicOr(&ctrl->stalled, 1u);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __hip_atomic_store(st + static_cast<int64_t>(tile) * kBins, kFlagPrefix | (e + c), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      excl[tid] = e;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    if (i < n) {
      const uint32_t d = digit(key[j], pass);
      const uint32_t pos = ctrl->base[pass][d] + excl[d] + wcnt[wave][d] + rank[j];
      if (pos < static_cast<uint64_t>(n)) {  // always, unless a look-back wait ran out
        kout[pos] = key[j];
        vout[pos] = val[j];
      }
    }
  }
}

}  // namespace radix

static inline size_t rs_align(size_t b) { return (b + 255) / 256 * 256; }

template <typename CT> size_t radix_sort_bytes(int64_t n) {
  constexpr int D = sizeof(CT);
  const int64_t ntiles = div_up(std::max<int64_t>(n, 1), radix::kTile);
  return rs_align(n * sizeof(CT)) + rs_align(n * sizeof(int32_t)) +
         rs_align(ntiles * D * radix::kBins * sizeof(uint32_t)) * 2 + rs_align(sizeof(radix::Ctrl));
}

// Stable ascending sort of (keys_in, vals_in) into (keys_out, vals_out); the
// inputs are left unchanged.  n < 2^30.
template <typename CT>
int radix_sort_pairs(const CT *keys_in, const int32_t *vals_in, CT *keys_out, int32_t *vals_out, int64_t n, void *ws,
                     size_t ws_bytes, hipStream_t s) {
  constexpr int D = sizeof(CT);
  SPIRA_HIP_REQUIRE(n >= 0 && n < (int64_t(1) << 30), "radix_sort: n out of range");
  if (n == 0) return kOk;
  SPIRA_HIP_REQUIRE(ws != nullptr && ws_bytes >= radix_sort_bytes<CT>(n), "radix_sort: workspace too small");
  const int ntiles = static_cast<int>(div_up(n, radix::kTile));
  char *p = static_cast<char *>(ws);
  CT *ktmp = reinterpret_cast<CT *>(p);
  p += rs_align(n * sizeof(CT));
  int32_t *vtmp = reinterpret_cast<int32_t *>(p);
  p += rs_align(n * sizeof(int32_t));
  uint32_t *tile_hist = reinterpret_cast<uint32_t *>(p);
  p += rs_align(static_cast<size_t>(ntiles) * D * radix::kBins * sizeof(uint32_t));
  uint32_t *status = reinterpret_cast<uint32_t *>(p);
  p += rs_align(static_cast<size_t>(ntiles) * D * radix::kBins * sizeof(uint32_t));
  radix::Ctrl *ctrl = reinterpret_cast<radix::Ctrl *>(p);
  const radix::Bufs<CT> bufs{keys_in, keys_out, ktmp, vals_in, vals_out, vtmp};
  hipLaunchKernelGGL(radix::rs_hist_kernel<CT>, dim3(ntiles), dim3(radix::kThreads), 0, s, keys_in, n, ntiles,
                     tile_hist, status);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(radix::rs_scan_kernel<CT>, dim3(D), dim3(radix::kThreads), 0, s, tile_hist, ntiles, n, ctrl);
  SPIRA_HIP_LAUNCH_CHECK();
  for (int pass = 0; pass < D; ++pass) {
    hipLaunchKernelGGL(radix::rs_pass_kernel<CT>, dim3(ntiles), dim3(radix::kThreads), 0, s, pass, n, ntiles, bufs,
                       status, ctrl);
    SPIRA_HIP_LAUNCH_CHECK();
  }
  return kOk;
}

template size_t radix_sort_bytes<uint64_t>(int64_t);
template size_t radix_sort_bytes<uint32_t>(int64_t);
template int radix_sort_pairs<uint64_t>(const uint64_t *, const int32_t *, uint64_t *, int32_t *, int64_t, void *,
                                        size_t, hipStream_t);
template int radix_sort_pairs<uint32_t>(const uint32_t *, const int32_t *, uint32_t *, int32_t *, int64_t, void *,
                                        size_t, hipStream_t);

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_radix_sort_workspace(int64_t n, int key_bits, size_t *bytes) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  *bytes = n <= 0 ? 0 : (key_bits == 64 ? radix_sort_bytes<uint64_t>(n) : radix_sort_bytes<uint32_t>(n));
  return kOk;
}

int spira_hip_radix_sort_status(const void *workspace, int64_t n, int key_bits, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  if (n <= 0) return kOk;
  SPIRA_HIP_REQUIRE(workspace != nullptr, "radix_sort_status: null workspace");
  const size_t bytes = key_bits == 64 ? radix_sort_bytes<uint64_t>(n) : radix_sort_bytes<uint32_t>(n);
  const auto *ctrl = reinterpret_cast<const radix::Ctrl *>(static_cast<const char *>(workspace) + bytes -
                                                           rs_align(sizeof(radix::Ctrl)));
  uint32_t stalled = 0;
  SPIRA_HIP_REQUIRE(hipMemcpyAsync(&stalled, &ctrl->stalled, sizeof(stalled), hipMemcpyDeviceToHost, stream) ==
                            hipSuccess &&
                        hipStreamSynchronize(stream) == hipSuccess,
                    "radix_sort_status: read failed");
  SPIRA_HIP_REQUIRE(stalled == 0, "radix_sort: a look-back wait ran out; the output is incomplete");
  return kOk;
}

int spira_hip_radix_sort_pairs(const void *keys_in, const int32_t *vals_in, void *keys_out, int32_t *vals_out,
                               int64_t n, int key_bits, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  if (key_bits == 64)
    return radix_sort_pairs<uint64_t>(static_cast<const uint64_t *>(keys_in), vals_in,
                                      static_cast<uint64_t *>(keys_out), vals_out, n, workspace, workspace_bytes,
                                      stream);
  return radix_sort_pairs<uint32_t>(static_cast<const uint32_t *>(keys_in), vals_in, static_cast<uint32_t *>(keys_out),
                                    vals_out, n, workspace, workspace_bytes, stream);
}

}  // extern "C"
