// Stable LSD radix sort of (key, int32 value) pairs for gfx950, exported as
// spira_hip_radix_sort_pairs.
//
// Reference semantics: FlattenSort (arg_sort_coodrinates.cu:36-88) sorts the
// packed keys with their original indices, ascending and stable (CUB
// DeviceRadixSort::SortPairs).  This sort gives the same order.
//
// Design:
//   * Digits follow the bits in which the keys differ.  A first launch ORs
//     every key's difference from the first key per 4096-key tile; the digit
//     plan takes runs of at most 9 of those bits, lowest first, each digit
//     ending at its highest varying bit.  Packed voxel keys (x, y, z fields of
//     ~9 varying bits each) then take 3 passes, 32-bit keys 4.
//   * sk_hist_kernel: per tile, the histogram of every pass's digit (the
//     digit counts do not depend on the key order, so one read of the keys
//     serves every pass); block 0 publishes the plan.
//   * sk_pass_kernel, one launch per pass (passes beyond the plan return at
//     once), thread t owning digit t: a block takes the next tile in ticket
//     order, sums the tiles' histograms of its digit for the global digit
//     base (these loads overlap the ticket and key loads), ranks its keys
//     stably (wave-level peer masks from one ballot per digit bit, per-wave
//     running counts in LDS), publishes its digit counts and finds its offset
//     per digit by a decoupled look-back over the tiles before it (16 tiles
//     per round of independent loads), then stages the tile in digit order in
//     LDS and writes each digit's run with consecutive threads.
//   * The look-back waits only on tiles with smaller tickets, which started
//     earlier and are running or done; the wait is bounded all the same, and
//     a wait that runs out sets a flag that spira_hip_radix_sort_status
//     reports.
// The look-back words of a pass alternate between two buffers: the reduce
// launch clears the first for pass 0, and pass p clears its own tile's words
// in the other buffer for pass p + 1 (pass p - 1, the last user of that
// buffer, has completed).
//
// Measured on MI355X at 200k keys it is slower than rocPRIM's sorts (32-bit
// keys ~96 us against ~69 us; packed 64-bit voxel keys ~85 us against ~42 us
// for rocPRIM's radix path).  In-kernel clock stamps put a pass at ~14 us:
// ~4 us ranking (with the key loads), ~5 us look-back and ~3.5 us staged
// scatter; the look-back's device-coherent loads grow with tiles x digits,
// and each exchange between blocks costs a device-scope round trip of
// ~1.5 us.  flatten_sort and the row order therefore keep rocPRIM.
#include "common.hpp"
#include "radix.hpp"
#include "../../../include/spira_hip.h"

namespace spira_hip {

namespace sortk {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kItems = 8;                       // keys per thread
constexpr int kWaveKeys = kItems * 64;          // contiguous keys per wave
constexpr int kTile = kThreads * kItems;        // keys per tile
constexpr int kMaxWidth = 9;                    // digit bits (one digit per thread)
constexpr int kMaxBins = 1 << kMaxWidth;
constexpr int kMaxPasses = 8;                   // 8 x 9 >= 64
constexpr uint32_t kFlagAgg = 1u << 30;         // look-back word: tile count only
constexpr uint32_t kFlagPrefix = 2u << 30;      // look-back word: inclusive prefix
constexpr uint32_t kCountMask = (1u << 30) - 1;
constexpr int kWindow = 16;                     // tiles per look-back round
constexpr int kSpinLimit = 1 << 22;

static_assert(kMaxBins == kThreads, "one digit per thread");



// device-side control block of one sort
struct Plan {
  int npasses;
  int shift[kMaxPasses], width[kMaxPasses];
  uint32_t ticket[kMaxPasses];
  uint32_t stalled;  // a look-back wait ran out (never expected)
};

template <typename CT> __device__ __forceinline__ uint32_t digit(CT k, int shift, int width) {
  return static_cast<uint32_t>(k >> shift) & ((1u << width) - 1u);
}

// The digit plan of a mask of varying bits (identical in every block).
__device__ inline Plan make_plan(uint64_t mask) {
  Plan pl{};
  int np = 0;
  while (mask != 0 && np < kMaxPasses) {
    const int lo = __builtin_ctzll(mask);
    const uint64_t win = (mask >> lo) & ((uint64_t(1) << kMaxWidth) - 1);
    const int w = 64 - __builtin_clzll(win);  // up to the highest varying bit in the window
    pl.shift[np] = lo;
    pl.width[np] = w;
    mask &= ~(((uint64_t(1) << w) - 1) << lo);
    ++np;
  }
  if (np == 0) {  // every key equal: one pass of a 0-bit digit (a stable copy)
    pl.shift[0] = 0;
    pl.width[0] = 0;
    np = 1;
  }
  pl.npasses = np;
  return pl;
}

__device__ __forceinline__ uint64_t block_or(uint64_t v, uint64_t *red) {
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int q = 0; q < static_cast<int>(blockDim.x >> 6); ++q) r |= red[q];
  return r;
}

// Per tile: the OR of every key's difference from the first key; clears the
// tile's look-back words of pass 0.
template <typename CT>
__global__ __launch_bounds__(kThreads) void sk_reduce_kernel(const CT *__restrict__ keys, int64_t n,
                                                             uint64_t *__restrict__ tile_or,
                                                             uint32_t *__restrict__ status0) {
  __shared__ uint64_t red[kWaves];
  const int tid = threadIdx.x;
  const CT k0 = keys[0];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  uint64_t acc = 0;
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = base + j * kThreads + tid;
    if (i < n) acc |= static_cast<uint64_t>(keys[i] ^ k0);
  }
  const uint64_t r = block_or(acc, red);
  if (tid == 0) tile_or[blockIdx.x] = r;
  for (int d = tid; d < kMaxBins; d += kThreads) status0[static_cast<int64_t>(blockIdx.x) * kMaxBins + d] = 0;
}

// Per tile: the histogram of every pass's digit; block 0 publishes the plan.
template <typename CT>
__global__ __launch_bounds__(kThreads) void sk_hist_kernel(const CT *__restrict__ keys, int64_t n, int ntiles,
                                                           const uint64_t *__restrict__ tile_or,
                                                           uint32_t *__restrict__ hist, Plan *__restrict__ plan) {
  __shared__ uint32_t h[kMaxPasses * kMaxBins];
  __shared__ uint64_t red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63;
  uint64_t m = 0;
  for (int t = tid; t < ntiles; t += kThreads) m |= tile_or[t];
  const uint64_t mask = block_or(m, red);
  const Plan pl = make_plan(mask);
  if (blockIdx.x == 0 && tid == 0) *plan = pl;  // (tickets 0, no stall)
  for (int i = tid; i < pl.npasses * kMaxBins; i += kThreads) h[i] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = base + j * kThreads + tid;
    const bool ok = i < n;
    const CT k = ok ? keys[i] : CT(0);
    const uint64_t all = __ballot(true), valid = __ballot(ok);
    for (int p = 0; p < pl.npasses; ++p) {
      const uint32_t d = digit(k, pl.shift[p], pl.width[p]);
      // a digit shared by the whole wave is one LDS add instead of 64
      const uint32_t d0 = __builtin_amdgcn_readfirstlane(d);
      if (__ballot(d == d0) == all && valid == all) {
        if (lane == 0) atomicAdd(&h[p * kMaxBins + d0], 64u);
      } else if (ok) {
        atomicAdd(&h[p * kMaxBins + d], 1u);
      }
    }
  }
  __syncthreads();
  for (int p = 0; p < pl.npasses; ++p) {
    const int bins = 1 << pl.width[p];
    for (int d = tid; d < bins; d += kThreads)
      hist[(static_cast<int64_t>(blockIdx.x) * kMaxPasses + p) * kMaxBins + d] = h[p * kMaxBins + d];
  }
}

// The buffers of a sort: 0 input, 1 output, 2 temporary.
template <typename CT> struct Bufs {
  const CT *k0;
  CT *k1, *k2;
  const int32_t *v0;  // null: the values are the input indices
  int32_t *v1, *v2;   // null v1: keys only
};

// VALS: 0 keys only, 1 key-value pairs.  Thread t owns digit t.
template <typename CT, int VALS>
__global__ __launch_bounds__(kThreads) void sk_pass_kernel(int pass, int64_t n, int ntiles, Bufs<CT> b,
                                                           const uint32_t *__restrict__ hist,
                                                           uint32_t *__restrict__ status, Plan *__restrict__ plan) {
  const int np = plan->npasses;
  if (pass >= np) return;  // (block-uniform)
  const int shift = plan->shift[pass], width = plan->width[pass], bins = 1 << width;
  __shared__ uint16_t wcnt[kWaves][kMaxBins];  // per-wave running counts, then wave prefixes
  __shared__ uint32_t toff[kMaxBins];          // the tile's exclusive digit offsets
  __shared__ uint32_t gpos[kMaxBins];          // global position of the tile's first key of each digit
  __shared__ uint32_t wsum[2][kWaves];
  __shared__ int s_tile;
  __shared__ CT skey[kTile];                   // the tile in digit order
  __shared__ int32_t sval[VALS ? kTile : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Tiles in ticket order: every tile a look-back waits on has started.
  if (tid == 0) s_tile = static_cast<int>(atomicAdd(&plan->ticket[pass], 1u));
  // the global total of this thread's digit (loads overlap the ticket's)
  const bool live = tid < bins;
  uint32_t tot = 0;
  if (live) {
#pragma unroll 8
    for (int t = 0; t < ntiles; ++t) tot += hist[(static_cast<int64_t>(t) * kMaxPasses + pass) * kMaxBins + tid];
  }
  for (int i = tid; i < kWaves * kMaxBins / 2; i += kThreads) reinterpret_cast<uint32_t *>(&wcnt[0][0])[i] = 0;
  __syncthreads();
  const int tile = s_tile;
  // source / destination buffers: the passes alternate between output and
  // temporary so that the last one writes the output
  const int dst = ((np - 1 - pass) % 2 == 0) ? 1 : 2;
  const int src = pass == 0 ? 0 : 3 - dst;
  const CT *__restrict__ kin = src == 0 ? b.k0 : (src == 1 ? b.k1 : b.k2);
  const int32_t *__restrict__ vin = src == 0 ? b.v0 : (src == 1 ? b.v1 : b.v2);
  CT *__restrict__ kout = dst == 1 ? b.k1 : b.k2;
  int32_t *__restrict__ vout = dst == 1 ? b.v1 : b.v2;
  const int64_t tbase = static_cast<int64_t>(tile) * kTile;
  const int64_t wbase = tbase + wave * kWaveKeys;
  CT key[kItems];
  int32_t val[kItems];
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    const bool ok = i < n;
    key[j] = ok ? kin[i] : CT(0);
    if constexpr (VALS) val[j] = ok ? (vin ? vin[i] : static_cast<int32_t>(i)) : 0;
  }
  // block-wide exclusive scan of one value per thread (digit order)
  auto block_scan = [&](uint32_t v, int slot) {
    uint32_t inc = v;
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t u = __shfl_up(inc, o, 64);
      if (lane >= o) inc += u;
    }
    if (lane == 63) wsum[slot][wave] = inc;
    __syncthreads();
    uint32_t run = inc - v;
    for (int w = 0; w < wave; ++w) run += wsum[slot][w];
    return run;
  };
  const uint32_t gbase = block_scan(live ? tot : 0u, 0);  // the digit's first global position
  // stable ranks: wave w holds the contiguous keys [w * kWaveKeys, (w + 1) *
  // kWaveKeys) of the tile, in rounds of 64, in order
  uint32_t rank[kItems];
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    const bool ok = i < n;
    const uint32_t d = digit(key[j], shift, width);
    uint64_t peers = __ballot(ok);
    for (int bit = 0; bit < width; ++bit) {
      const bool on = (d >> bit) & 1u;
      const uint64_t mb = __ballot(on);
      peers &= on ? mb : ~mb;
    }
    const uint32_t before = wcnt[wave][d];
    rank[j] = before + static_cast<uint32_t>(__builtin_popcountll(peers & lt));
    // the group's first lane advances the wave's count of the digit
    const bool leader = ok && (peers & lt) == 0;
    __builtin_amdgcn_wave_barrier();
    if (leader) wcnt[wave][d] = static_cast<uint16_t>(before + __builtin_popcountll(peers));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __syncthreads();
  // the tile's count of this thread's digit and the waves' exclusive prefixes
  uint32_t cnt = 0;
  if (live) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t v = wcnt[w][tid];
      wcnt[w][tid] = static_cast<uint16_t>(cnt);
      cnt += v;
    }
  }
  uint32_t *st = status + static_cast<int64_t>(pass & 1) * ntiles * kMaxBins + tid;
  if (live)
    __hip_atomic_store(st + static_cast<int64_t>(tile) * kMaxBins, (tile == 0 ? kFlagPrefix : kFlagAgg) | cnt,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  toff[tid] = block_scan(cnt, 1);
  // decoupled look-back: the counts of this digit in the tiles before this
  // one, kWindow tiles per round of independent loads
  uint32_t excl = 0;
  if (live && tile > 0) {
    int cur = tile - 1, spins = 0;
    while (cur >= 0) {
      uint32_t w[kWindow];
#pragma unroll
      for (int k = 0; k < kWindow; ++k)
        w[k] = cur - k >= 0 ? __hip_atomic_load(st + static_cast<int64_t>(cur - k) * kMaxBins, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0u;
      int k = 0;
      bool found = false;
      for (; k < kWindow && cur - k >= 0; ++k) {
        if ((w[k] & ~kCountMask) == 0) break;  // not published yet: read again from here
        excl += w[k] & kCountMask;
        if (w[k] & kFlagPrefix) {
          found = true;
          break;
        }
      }
      if (found) break;
      cur -= k;
      if (k < kWindow && cur >= 0) {
        if (++spins > kSpinLimit) {  // bounded: never expected (earlier tickets are running)
          atomicOr(&plan->stalled, 1u);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __hip_atomic_store(st + static_cast<int64_t>(tile) * kMaxBins, kFlagPrefix | (excl + cnt), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  gpos[tid] = gbase + excl;
  // this tile's look-back words of the next pass start cleared
  status[(static_cast<int64_t>((pass + 1) & 1) * ntiles + tile) * kMaxBins + tid] = 0;
  __syncthreads();  // (toff)
  // the tile in digit order in LDS, then out with consecutive threads on
  // consecutive positions of each digit's run
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = wbase + j * 64 + lane;
    if (i < n) {
      const uint32_t d = digit(key[j], shift, width);
      const uint32_t l = toff[d] + wcnt[wave][d] + rank[j];
      skey[l] = key[j];
      if constexpr (VALS) sval[l] = val[j];
    }
  }
  __syncthreads();
  const int cnt_tile = static_cast<int>(n - tbase < kTile ? n - tbase : kTile);
#pragma unroll 4
  for (int l = tid; l < cnt_tile; l += kThreads) {
    const CT k = skey[l];
    const uint32_t d = digit(k, shift, width);
    const uint32_t pos = gpos[d] + (static_cast<uint32_t>(l) - toff[d]);
    if (pos < static_cast<uint64_t>(n)) {  // always, unless a look-back wait ran out
      kout[pos] = k;
      if constexpr (VALS) vout[pos] = sval[l];
    }
  }
}

static inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

struct Parts {
  void *ktmp;
  int32_t *vtmp;
  uint64_t *tile_or;
  uint32_t *hist, *status;
  Plan *plan;
  size_t total;
};
template <typename CT> static Parts parts(int64_t n, bool vals, void *ws) {
  const int64_t ntiles = div_up(std::max<int64_t>(n, 1), kTile);
  char *p = static_cast<char *>(ws);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = p ? p + off : nullptr;
    off += align256(bytes);
    return q;
  };
  Parts r{};
  r.ktmp = take(n * sizeof(CT));
  r.vtmp = reinterpret_cast<int32_t *>(vals ? take(n * sizeof(int32_t)) : nullptr);
  r.tile_or = reinterpret_cast<uint64_t *>(take(ntiles * sizeof(uint64_t)));
  r.hist = reinterpret_cast<uint32_t *>(take(static_cast<size_t>(ntiles) * kMaxPasses * kMaxBins * 4));
  r.status = reinterpret_cast<uint32_t *>(take(static_cast<size_t>(ntiles) * 2 * kMaxBins * 4));
  r.plan = reinterpret_cast<Plan *>(take(sizeof(Plan)));
  r.total = off;
  return r;
}

}  // namespace sortk

template <typename CT> size_t sort_bytes(int64_t n, bool with_values) {
  return n <= 0 ? 0 : sortk::parts<CT>(n, with_values, nullptr).total;
}

template <typename CT>
int sort_keys_values(const CT *keys_in, const int32_t *vals_in, CT *keys_out, int32_t *vals_out, int64_t n,
                     void *ws, size_t ws_bytes, hipStream_t s) {
  using namespace sortk;
  SPIRA_HIP_REQUIRE(n >= 0 && n < (int64_t(1) << 30), "radix_sort: n out of range");
  if (n == 0) return kOk;
  const bool vals = vals_out != nullptr;
  SPIRA_HIP_REQUIRE(ws != nullptr && ws_bytes >= sort_bytes<CT>(n, vals), "radix_sort: workspace too small");
  const Parts w = parts<CT>(n, vals, ws);
  const int ntiles = static_cast<int>(div_up(n, kTile));
  const Bufs<CT> bufs{keys_in, keys_out, static_cast<CT *>(w.ktmp), vals_in, vals_out, w.vtmp};
  hipLaunchKernelGGL(sk_reduce_kernel<CT>, dim3(ntiles), dim3(kThreads), 0, s, keys_in, n, w.tile_or, w.status);
  SPIRA_HIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(sk_hist_kernel<CT>, dim3(ntiles), dim3(kThreads), 0, s, keys_in, n, ntiles, w.tile_or, w.hist,
                     w.plan);
  SPIRA_HIP_LAUNCH_CHECK();
  // the most passes any key set of this width can need (the later ones
  // return at once when the plan has fewer)
  const int maxp = static_cast<int>((8 * sizeof(CT) + kMaxWidth - 1) / kMaxWidth);
  for (int pass = 0; pass < maxp; ++pass) {
    if (vals)
      hipLaunchKernelGGL(HIP_KERNEL_NAME(sk_pass_kernel<CT, 1>), dim3(ntiles), dim3(kThreads), 0, s, pass, n, ntiles,
                         bufs, w.hist, w.status, w.plan);
    else
      hipLaunchKernelGGL(HIP_KERNEL_NAME(sk_pass_kernel<CT, 0>), dim3(ntiles), dim3(kThreads), 0, s, pass, n, ntiles,
                         bufs, w.hist, w.status, w.plan);
    SPIRA_HIP_LAUNCH_CHECK();
  }
  return kOk;
}

template <typename CT> int sort_status(const void *ws, int64_t n, bool with_values, hipStream_t s) {
  if (n <= 0) return kOk;
  SPIRA_HIP_REQUIRE(ws != nullptr, "radix_sort_status: null workspace");
  const sortk::Parts w = sortk::parts<CT>(n, with_values, const_cast<void *>(ws));
  uint32_t stalled = 0;
  SPIRA_HIP_TRY(hipMemcpyAsync(&stalled, &w.plan->stalled, sizeof(stalled), hipMemcpyDeviceToHost, s));
  SPIRA_HIP_TRY(hipStreamSynchronize(s));
  SPIRA_HIP_REQUIRE(stalled == 0, "radix_sort: a look-back wait ran out; the output is incomplete");
  return kOk;
}

template size_t sort_bytes<uint64_t>(int64_t, bool);
template size_t sort_bytes<uint32_t>(int64_t, bool);
template int sort_keys_values<uint64_t>(const uint64_t *, const int32_t *, uint64_t *, int32_t *, int64_t, void *,
                                        size_t, hipStream_t);
template int sort_keys_values<uint32_t>(const uint32_t *, const int32_t *, uint32_t *, int32_t *, int64_t, void *,
                                        size_t, hipStream_t);
template int sort_status<uint64_t>(const void *, int64_t, bool, hipStream_t);
template int sort_status<uint32_t>(const void *, int64_t, bool, hipStream_t);

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_radix_sort_workspace(int64_t n, int key_bits, size_t *bytes) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  *bytes = key_bits == 64 ? sort_bytes<uint64_t>(n, true) : sort_bytes<uint32_t>(n, true);
  return kOk;
}

int spira_hip_radix_sort_pairs(const void *keys_in, const int32_t *vals_in, void *keys_out, int32_t *vals_out,
                               int64_t n, int key_bits, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  SPIRA_HIP_REQUIRE(n == 0 || (keys_in && keys_out && vals_out), "radix_sort: null buffer");
  if (key_bits == 64)
    return sort_keys_values<uint64_t>(static_cast<const uint64_t *>(keys_in), vals_in,
                                      static_cast<uint64_t *>(keys_out), vals_out, n, workspace, workspace_bytes,
                                      stream);
  return sort_keys_values<uint32_t>(static_cast<const uint32_t *>(keys_in), vals_in,
                                    static_cast<uint32_t *>(keys_out), vals_out, n, workspace, workspace_bytes,
                                    stream);
}

int spira_hip_radix_sort_status(const void *workspace, int64_t n, int key_bits, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "radix_sort: key_bits must be 32 or 64");
  return key_bits == 64 ? sort_status<uint64_t>(workspace, n, true, stream)
                        : sort_status<uint32_t>(workspace, n, true, stream);
}

}  // extern "C"
