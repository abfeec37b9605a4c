// Sparse-convolution feature kernels for gfx950.
//
// Dataflows (reference semantics):
//  * output-stationary implicit GEMM, Y[t] = sum_j X[map[t, j]] @ W[j]
//    (output_stat.cuh:20-1031, sparse_convolution.cu:1354-1393);
//  * fused weight-stationary over compacted pair lists with mirrored offsets
//    (weight_stat.cuh:33-1221, sparse_convolution.cu:16-167, 1267-1350);
//  * gather -> grouped GEMM -> scatter over per-offset masks
//    (padded_gather/scatter_warp_optimized.cuh, sparse_convolution.cu:488-1124).
//
// MI355X design: fp16 operands on v_mfma_f32_32x32x16_f16 with fp32
// accumulation.  A block is 4 waves; a wave owns 32 output rows x 32*WN
// columns (WN accumulators of 16 floats).  A-operand rows are gathered
// straight from HBM/L2 into registers (each lane loads the 16 bytes its MFMA
// slot needs, so no LDS round trip for the irregular side); the offset's
// weight slice is staged once per block in LDS, pre-transposed to
// [Cout, Cin] so that B operands are 16-byte LDS reads.  Waves whose 32 rows
// have no neighbour at an offset skip its MFMAs.
#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <algorithm>
#include <vector>

namespace spira_hip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kRowsPerBlock = 128;  // 4 waves x 32 rows
constexpr int kChunk = 64;          // Cin staged per LDS round
constexpr int kBStride = kChunk + 8;  // halves per staged weight row (bank spread)
constexpr int kMaxGroups = 128;

enum OutMode { kStoreNative = 0, kStoreF32 = 1, kAddF32 = 2, kAtomicF32 = 3 };

__device__ __forceinline__ half8 zero_h8() {
  half8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = static_cast<_Float16>(0.f);
  return z;
}

// Stage WT[wrow][n0:n0+BN][kc:kc+kChunk] (transposed weights [K, Cout, Cin])
// into LDS, zero outside Cout / Cin.
template <int BN>
__device__ __forceinline__ void stage_weights(_Float16 *Bs, const _Float16 *__restrict__ WT, int64_t wrow, int n0,
                                              int Cout, int kc, int Cin) {
  constexpr int VPR = kChunk / 8;  // 16-byte vectors per row
  for (int v = threadIdx.x; v < BN * VPR; v += 256) {
    const int n = v / VPR, kk = (v % VPR) * 8;
    half8 w = zero_h8();
    if (n0 + n < Cout && kc + kk < Cin)
      w = *reinterpret_cast<const half8 *>(WT + (wrow * Cout + n0 + n) * Cin + kc + kk);
    *reinterpret_cast<half8 *>(Bs + n * kBStride + kk) = w;
  }
}

// One staged chunk: acc[wn] += A(rows of this wave) x Bs.
template <int WN>
__device__ __forceinline__ void mma_chunk(floatx16 *acc, const _Float16 *Bs, const _Float16 *xrow, bool has_row,
                                          int kc, int Cin, int r, int kh) {
#pragma unroll
  for (int ks = 0; ks < kChunk / 16; ++ks) {
    const int k = kc + ks * 16 + kh * 8;
    if (kc + ks * 16 >= Cin) break;  // wave-uniform
    half8 a = zero_h8();
    if (has_row && k < Cin) a = *reinterpret_cast<const half8 *>(xrow + k);
#pragma unroll
    for (int wn = 0; wn < WN; ++wn) {
      const half8 b = *reinterpret_cast<const half8 *>(Bs + (wn * 32 + r) * kBStride + ks * 16 + kh * 8);
      acc[wn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[wn], 0, 0, 0);
    }
  }
}

// Write one wave's 32 x (32*WN) accumulator tile.  row_of(i) maps the tile row
// to an output row (or -1).
template <int WN, int MODE>
__device__ __forceinline__ void store_tile(const floatx16 *acc, const int64_t *orow, int n0, int Cout, int r, int kh,
                                           void *Yv) {
#pragma unroll
  for (int wn = 0; wn < WN; ++wn) {
    const int col = n0 + wn * 32 + r;
    if (col >= Cout) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i / 4) * 8 + kh * 4 + (i % 4);
      const int64_t o = orow[row];
      if (o < 0) continue;
      const float v = acc[wn][i];
      if constexpr (MODE == kStoreNative) {
        static_cast<_Float16 *>(Yv)[o * Cout + col] = static_cast<_Float16>(v);
      } else if constexpr (MODE == kStoreF32) {
        static_cast<float *>(Yv)[o * Cout + col] = v;
      } else if constexpr (MODE == kAddF32) {
        static_cast<float *>(Yv)[o * Cout + col] += v;
      } else {
        atomicAdd(static_cast<float *>(Yv) + o * Cout + col, v);
      }
    }
  }
}

// Output-stationary implicit GEMM, fp16 in / fp32 accumulate.
template <int WN, int MODE>
__global__ __launch_bounds__(256) void os_f16_kernel(const int32_t *__restrict__ map, int64_t T, int Kc,
                                                     const _Float16 *__restrict__ X, int Cin,
                                                     const _Float16 *__restrict__ WT, int Cout, void *Y) {
  constexpr int BN = 32 * WN;
  __shared__ __align__(16) _Float16 Bs[BN * kBStride];
  __shared__ int64_t orow_s[4][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, kh = lane >> 5;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + wave * 32;
  const int n0 = blockIdx.y * BN;
  const int64_t t = t0 + r;
  const bool tvalid = t < T;
  floatx16 acc[WN];
#pragma unroll
  for (int wn = 0; wn < WN; ++wn)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[wn][i] = 0.f;

  for (int j = 0; j < Kc; ++j) {
    const int32_t idx = tvalid ? map[t * Kc + j] : -1;
    const bool any = ballot(idx >= 0) != 0;
    const _Float16 *xrow = X + static_cast<int64_t>(idx < 0 ? 0 : idx) * Cin;
    for (int kc = 0; kc < Cin; kc += kChunk) {
      __syncthreads();
      stage_weights<BN>(Bs, WT, j, n0, Cout, kc, Cin);
      __syncthreads();
      if (any) mma_chunk<WN>(acc, Bs, xrow, idx >= 0, kc, Cin, r, kh);
    }
  }
  if (kh == 0) orow_s[wave][r] = tvalid ? t : -1;
  __syncthreads();
  store_tile<WN, MODE>(acc, orow_s[wave], n0, Cout, r, kh, Y);
}

// Fused weight-stationary tile over 128 consecutive pairs of one offset row.
// Tiles [0, nfwd) use (in -> out) with W[woffset + r]; with `mirror`, tiles
// [nfwd, 2 nfwd) use (out -> in) with W[woffset + Kw-1-r], skipping a
// self-mirrored centre row.  Results are atomically added to an fp32 buffer.
template <int WN>
__global__ __launch_bounds__(256) void ws_fused_f16_kernel(const int32_t *__restrict__ in_idx,
                                                           const int32_t *__restrict__ out_idx,
                                                           const int32_t *__restrict__ naddrs,
                                                           const int32_t *__restrict__ qnaddrs, int R, int64_t nfwd,
                                                           int Kw, int woffset, const _Float16 *__restrict__ X,
                                                           int Cin, const _Float16 *__restrict__ WT, int Cout,
                                                           float *__restrict__ Yacc) {
  constexpr int BN = 32 * WN;
  __shared__ __align__(16) _Float16 Bs[BN * kBStride];
  __shared__ int64_t orow_s[4][32];
  int64_t tile = blockIdx.x;
  const bool mir = tile >= nfwd;
  if (mir) tile -= nfwd;
  const int64_t pos = tile * kRowsPerBlock;
  // row r: last r with qnaddrs[r] <= pos
  int lo = 0, hi = R;
  while (hi - lo > 1) {
    int m = (lo + hi) >> 1;
    if (qnaddrs[m] <= pos) lo = m;
    else hi = m;
  }
  const int row = lo;
  if (mir && 2 * row + 1 == Kw) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, kh = lane >> 5;
  const int64_t local = pos - qnaddrs[row] + wave * 32 + r;
  const int64_t nrow = naddrs[row + 1] - naddrs[row];
  const bool valid = local < nrow;
  const int64_t p = naddrs[row] + local;
  const int32_t src = valid ? (mir ? out_idx[p] : in_idx[p]) : -1;
  const int32_t dst = valid ? (mir ? in_idx[p] : out_idx[p]) : -1;
  const int64_t wrow = woffset + (mir ? Kw - 1 - row : row);
  const int n0 = blockIdx.y * BN;
  floatx16 acc[WN];
#pragma unroll
  for (int wn = 0; wn < WN; ++wn)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[wn][i] = 0.f;
  const bool any = ballot(src >= 0) != 0;
  const _Float16 *xrow = X + static_cast<int64_t>(src < 0 ? 0 : src) * Cin;
  for (int kc = 0; kc < Cin; kc += kChunk) {
    __syncthreads();
    stage_weights<BN>(Bs, WT, wrow, n0, Cout, kc, Cin);
    __syncthreads();
    if (any) mma_chunk<WN>(acc, Bs, xrow, src >= 0, kc, Cin, r, kh);
  }
  if (kh == 0) orow_s[wave][r] = dst;
  __syncthreads();
  store_tile<WN, kAtomicF32>(acc, orow_s[wave], n0, Cout, r, kh, Yacc);
}

struct GroupTable {
  int n;                          // groups
  int64_t tile_start[kMaxGroups + 1];  // prefix of 128-row tiles
  int64_t row_off[kMaxGroups];    // first buffer row of the group
  int32_t rows[kMaxGroups];       // valid rows of the group
};

// Grouped GEMM over the padded gather buffer: Ybuf[g rows] = Xbuf[g rows] @ W[g].
template <int WN>
__global__ __launch_bounds__(256) void group_gemm_f16_kernel(const GroupTable gt, const _Float16 *__restrict__ Xb,
                                                             int Cin, const _Float16 *__restrict__ WT, int Cout,
                                                             float *__restrict__ Yb) {
  constexpr int BN = 32 * WN;
  __shared__ __align__(16) _Float16 Bs[BN * kBStride];
  __shared__ int64_t orow_s[4][32];
  const int64_t tile = blockIdx.x;
  int g = 0;
  while (g + 1 < gt.n && gt.tile_start[g + 1] <= tile) ++g;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, kh = lane >> 5;
  const int64_t local = (tile - gt.tile_start[g]) * kRowsPerBlock + wave * 32 + r;
  const bool valid = local < gt.rows[g];
  const int64_t brow = gt.row_off[g] + local;
  const int n0 = blockIdx.y * BN;
  floatx16 acc[WN];
#pragma unroll
  for (int wn = 0; wn < WN; ++wn)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[wn][i] = 0.f;
  const bool any = ballot(valid) != 0;
  const _Float16 *xrow = Xb + (valid ? brow : 0) * Cin;
  for (int kc = 0; kc < Cin; kc += kChunk) {
    __syncthreads();
    stage_weights<BN>(Bs, WT, g, n0, Cout, kc, Cin);
    __syncthreads();
    if (any) mma_chunk<WN>(acc, Bs, xrow, valid, kc, Cin, r, kh);
  }
  if (kh == 0) orow_s[wave][r] = valid ? brow : -1;
  __syncthreads();
  store_tile<WN, kStoreF32>(acc, orow_s[wave], n0, Cout, r, kh, Yb);
}

// ---------------------------------------------------------------------------
// generic (any channel count, fp32 or fp16 storage) kernels, fp32 accumulate
// ---------------------------------------------------------------------------
template <typename FT> __device__ __forceinline__ float ld(const FT *p) { return static_cast<float>(*p); }

template <typename FT, int MODE>
__device__ __forceinline__ void put(void *Y, int64_t i, float v) {
  if constexpr (MODE == kStoreNative) static_cast<FT *>(Y)[i] = static_cast<FT>(v);
  else if constexpr (MODE == kStoreF32) static_cast<float *>(Y)[i] = v;
  else if constexpr (MODE == kAddF32) static_cast<float *>(Y)[i] += v;
  else atomicAdd(static_cast<float *>(Y) + i, v);
}

template <typename FT, int MODE>
__global__ __launch_bounds__(256) void os_generic_kernel(const int32_t *__restrict__ map, int64_t T, int Kc,
                                                         const FT *__restrict__ X, int Cin,
                                                         const FT *__restrict__ W, int Cout, void *Y) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * Cout) return;
  const int64_t t = i / Cout;
  const int c = static_cast<int>(i % Cout);
  float acc = 0.f;
  for (int j = 0; j < Kc; ++j) {
    const int32_t s = map[t * Kc + j];
    if (s < 0) continue;
    const FT *x = X + static_cast<int64_t>(s) * Cin;
    const FT *w = W + (static_cast<int64_t>(j) * Cin) * Cout + c;
    for (int ci = 0; ci < Cin; ++ci) acc += ld(x + ci) * ld(w + static_cast<int64_t>(ci) * Cout);
  }
  put<FT, MODE>(Y, i, acc);
}

template <typename FT>
__global__ __launch_bounds__(256) void ws_fused_generic_kernel(const int32_t *__restrict__ in_idx,
                                                               const int32_t *__restrict__ out_idx,
                                                               const int32_t *__restrict__ naddrs, int R, int Kw,
                                                               int woffset, int mirror, int64_t P,
                                                               const FT *__restrict__ X, int Cin,
                                                               const FT *__restrict__ W, int Cout,
                                                               float *__restrict__ Yacc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t passes = mirror ? 2 : 1;
  if (i >= passes * P * Cout) return;
  int64_t p = i / Cout;
  const int c = static_cast<int>(i % Cout);
  const bool mir = p >= P;
  if (mir) p -= P;
  int lo = 0, hi = R;
  while (hi - lo > 1) {
    int m = (lo + hi) >> 1;
    if (naddrs[m] <= p) lo = m;
    else hi = m;
  }
  const int row = lo;
  if (mir && 2 * row + 1 == Kw) return;
  const int32_t s = mir ? out_idx[p] : in_idx[p];
  const int32_t d = mir ? in_idx[p] : out_idx[p];
  const int64_t wrow = woffset + (mir ? Kw - 1 - row : row);
  const FT *x = X + static_cast<int64_t>(s) * Cin;
  const FT *w = W + wrow * Cin * Cout + c;
  float acc = 0.f;
  for (int ci = 0; ci < Cin; ++ci) acc += ld(x + ci) * ld(w + static_cast<int64_t>(ci) * Cout);
  atomicAdd(Yacc + static_cast<int64_t>(d) * Cout + c, acc);
}

template <typename FT>
__global__ __launch_bounds__(256) void group_gemm_generic_kernel(const GroupTable gt, int64_t total_rows,
                                                                 const FT *__restrict__ Xb, int Cin,
                                                                 const FT *__restrict__ W, int Cout,
                                                                 float *__restrict__ Yb) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total_rows * Cout) return;
  const int64_t brow = i / Cout;
  const int c = static_cast<int>(i % Cout);
  int g = 0;
  while (g + 1 < gt.n && gt.row_off[g + 1] <= brow) ++g;
  if (brow - gt.row_off[g] >= gt.rows[g]) return;
  const FT *x = Xb + brow * Cin;
  const FT *w = W + static_cast<int64_t>(g) * Cin * Cout + c;
  float acc = 0.f;
  for (int ci = 0; ci < Cin; ++ci) acc += ld(x + ci) * ld(w + static_cast<int64_t>(ci) * Cout);
  Yb[i] = acc;
}

struct OffsetTable {
  int n;
  int64_t off[kMaxGroups];  // first padded buffer row of each offset
};

// gather: buf[off[k] + mask[k, s]] = X[s] for every mask entry >= 0
template <typename FT>
__global__ __launch_bounds__(256) void gather_kernel(const OffsetTable ot, int64_t S, int Cin,
                                                     const int32_t *__restrict__ smask, const FT *__restrict__ X,
                                                     FT *__restrict__ buf) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= S * Cin) return;
  const int64_t s = i / Cin;
  const int c = static_cast<int>(i % Cin);
  const FT v = X[i];
  for (int k = 0; k < ot.n; ++k) {
    const int32_t m = smask[k * S + s];
    if (m >= 0) buf[(ot.off[k] + m) * Cin + c] = v;
  }
}

// vectorised fp16 gather for Cin % 8 == 0
__global__ __launch_bounds__(256) void gather_h8_kernel(const OffsetTable ot, int64_t S, int Cin,
                                                        const int32_t *__restrict__ smask,
                                                        const _Float16 *__restrict__ X, _Float16 *__restrict__ buf) {
  const int nv = Cin / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= S * nv) return;
  const int64_t s = i / nv;
  const int c = static_cast<int>(i % nv) * 8;
  const half8 v = *reinterpret_cast<const half8 *>(X + s * Cin + c);
  for (int k = 0; k < ot.n; ++k) {
    const int32_t m = smask[k * S + s];
    if (m >= 0) *reinterpret_cast<half8 *>(buf + (ot.off[k] + m) * Cin + c) = v;
  }
}

// scatter: Y[t] (+)= sum_k buf[off[k] + mask[k, t]]
template <typename FT>
__global__ __launch_bounds__(256) void scatter_kernel(const OffsetTable ot, int64_t T, int Cout,
                                                      const int32_t *__restrict__ tmask,
                                                      const float *__restrict__ buf, FT *__restrict__ Y,
                                                      const float *__restrict__ base) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * Cout) return;
  const int64_t t = i / Cout;
  const int c = static_cast<int>(i % Cout);
  float acc = base ? base[i] : 0.f;
  for (int k = 0; k < ot.n; ++k) {
    const int32_t m = tmask[k * T + t];
    if (m >= 0) acc += buf[(ot.off[k] + m) * Cout + c];
  }
  Y[i] = static_cast<FT>(acc);
}

template <typename FT>
__global__ void cast_f32_kernel(const float *__restrict__ src, int64_t n, FT *__restrict__ dst) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = static_cast<FT>(src[i]);
}

// [K, Cin, Cout] -> [K, Cout, Cin]
__global__ void transpose_w_kernel(const _Float16 *__restrict__ W, int K, int Cin, int Cout,
                                   _Float16 *__restrict__ WT) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = static_cast<int64_t>(K) * Cin * Cout;
  if (i >= n) return;
  const int64_t k = i / (static_cast<int64_t>(Cin) * Cout);
  const int64_t rem = i % (static_cast<int64_t>(Cin) * Cout);
  const int ci = static_cast<int>(rem / Cout), co = static_cast<int>(rem % Cout);
  WT[(k * Cout + co) * Cin + ci] = W[i];
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
static inline bool mfma_ok(int dtype, int Cin) { return dtype == SPIRA_F16 && Cin % 8 == 0; }

static inline int wn_for(int Cout) { return Cout <= 32 ? 1 : (Cout <= 64 ? 2 : 4); }

static size_t wt_bytes(int K, int Cin, int Cout) { return static_cast<size_t>(K) * Cin * Cout * sizeof(_Float16); }

static int transpose_weights(const void *W, int K, int Cin, int Cout, void *WT, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(K) * Cin * Cout;
  if (n == 0) return kOk;
  hipLaunchKernelGGL(transpose_w_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, static_cast<const _Float16 *>(W), K,
                     Cin, Cout, static_cast<_Float16 *>(WT));
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

template <int MODE>
static void launch_os_f16(int wn, dim3 grid, hipStream_t s, const int32_t *map, int64_t T, int Kc, const void *X,
                          int Cin, const void *WT, int Cout, void *Y) {
  auto x = static_cast<const _Float16 *>(X);
  auto wt = static_cast<const _Float16 *>(WT);
  if (wn == 1) hipLaunchKernelGGL((os_f16_kernel<1, MODE>), grid, dim3(256), 0, s, map, T, Kc, x, Cin, wt, Cout, Y);
  else if (wn == 2) hipLaunchKernelGGL((os_f16_kernel<2, MODE>), grid, dim3(256), 0, s, map, T, Kc, x, Cin, wt, Cout, Y);
  else hipLaunchKernelGGL((os_f16_kernel<4, MODE>), grid, dim3(256), 0, s, map, T, Kc, x, Cin, wt, Cout, Y);
}

template <typename FT, int MODE>
static void launch_os_generic(hipStream_t s, const int32_t *map, int64_t T, int Kc, const void *X, int Cin,
                              const void *W, int Cout, void *Y) {
  const int64_t n = T * Cout;
  hipLaunchKernelGGL((os_generic_kernel<FT, MODE>), dim3(div_up(n, 256)), dim3(256), 0, s, map, T, Kc,
                     static_cast<const FT *>(X), Cin, static_cast<const FT *>(W), Cout, Y);
}

static int fill_groups(GroupTable &gt, int K, const int32_t *rows, const int64_t *row_off) {
  SPIRA_HIP_REQUIRE(K <= kMaxGroups, "at most 128 kernel offsets are supported");
  gt.n = K;
  gt.tile_start[0] = 0;
  for (int k = 0; k < K; ++k) {
    gt.rows[k] = rows[k];
    gt.row_off[k] = row_off[k];
    gt.tile_start[k + 1] = gt.tile_start[k] + div_up(rows[k], kRowsPerBlock);
  }
  return kOk;
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_conv_workspace(int num_offsets, int c_in, int c_out, int dtype, size_t *bytes) {
  *bytes = mfma_ok(dtype, c_in) ? wt_bytes(num_offsets, c_in, c_out) : 0;
  return kOk;
}

int spira_hip_conv_os(int64_t num_targets, int num_offsets, const int32_t *out_in_map, const void *sources,
                      int64_t num_sources, int c_in, const void *weights, int c_out, int dtype, void *targets,
                      int out_mode, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  (void)num_sources;
  SPIRA_HIP_REQUIRE(dtype == SPIRA_F16 || dtype == SPIRA_F32, "conv_os: dtype must be fp16 or fp32");
  SPIRA_HIP_REQUIRE(out_mode >= SPIRA_OUT_STORE && out_mode <= SPIRA_OUT_ADD_F32, "conv_os: bad out_mode");
  SPIRA_HIP_REQUIRE(c_in > 0 && c_out > 0 && num_offsets > 0, "conv_os: empty channel / offset dimension");
  if (num_targets <= 0) return kOk;
  // out_mode: 0 = store in dtype, 1 = store fp32, 2 = add into fp32
  if (mfma_ok(dtype, c_in)) {
    SPIRA_HIP_REQUIRE(workspace && workspace_bytes >= wt_bytes(num_offsets, c_in, c_out),
                      "conv_os: workspace too small");
    int rc = transpose_weights(weights, num_offsets, c_in, c_out, workspace, stream);
    if (rc) return rc;
    const int wn = wn_for(c_out);
    dim3 grid(static_cast<unsigned>(div_up(num_targets, kRowsPerBlock)), static_cast<unsigned>(div_up(c_out, 32 * wn)));
    if (out_mode == SPIRA_OUT_STORE)
      launch_os_f16<kStoreNative>(wn, grid, stream, out_in_map, num_targets, num_offsets, sources, c_in, workspace,
                                c_out, targets);
    else if (out_mode == SPIRA_OUT_STORE_F32)
      launch_os_f16<kStoreF32>(wn, grid, stream, out_in_map, num_targets, num_offsets, sources, c_in, workspace,
                               c_out, targets);
    else
      launch_os_f16<kAddF32>(wn, grid, stream, out_in_map, num_targets, num_offsets, sources, c_in, workspace,
                             c_out, targets);
  } else if (dtype == SPIRA_F16) {
    if (out_mode == SPIRA_OUT_STORE)
      launch_os_generic<_Float16, kStoreNative>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights,
                                              c_out, targets);
    else if (out_mode == SPIRA_OUT_STORE_F32)
      launch_os_generic<_Float16, kStoreF32>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights,
                                             c_out, targets);
    else
      launch_os_generic<_Float16, kAddF32>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights,
                                           c_out, targets);
  } else {
    if (out_mode == SPIRA_OUT_ADD_F32)
      launch_os_generic<float, kAddF32>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights, c_out,
                                        targets);
    else
      launch_os_generic<float, kStoreNative>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights,
                                           c_out, targets);
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_conv_ws_fused(int64_t num_sources, int64_t num_targets, const int32_t *in_idx, const int32_t *out_idx,
                            int rows, const int32_t *naddrs, const int32_t *qnaddrs, int64_t num_pairs,
                            int64_t quantized_pairs, int weight_offset, int mirror_rows, const void *sources,
                            int c_in, const void *weights, int num_weights, int c_out, int dtype, float *target_acc,
                            void *workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  (void)num_sources;
  (void)num_targets;
  SPIRA_HIP_REQUIRE(dtype == SPIRA_F16 || dtype == SPIRA_F32, "conv_ws_fused: dtype must be fp16 or fp32");
  SPIRA_HIP_REQUIRE(rows >= 1 || num_pairs == 0, "conv_ws_fused: rows must be positive");
  if (num_pairs <= 0) return kOk;
  // mirror_rows = Kw > 0 enables the mirrored pass over Kw offsets; 0 disables it
  const int Kw = mirror_rows;
  if (mfma_ok(dtype, c_in)) {
    const int K = num_weights;
    SPIRA_HIP_REQUIRE(weight_offset + std::max(Kw, rows) <= K, "conv_ws_fused: weight rows out of range");
    SPIRA_HIP_REQUIRE(workspace && workspace_bytes >= wt_bytes(K, c_in, c_out), "conv_ws_fused: workspace too small");
    int rc = transpose_weights(weights, K, c_in, c_out, workspace, stream);
    if (rc) return rc;
    const int wn = wn_for(c_out);
    const int64_t nfwd = quantized_pairs / kRowsPerBlock;
    dim3 grid(static_cast<unsigned>(Kw > 0 ? 2 * nfwd : nfwd), static_cast<unsigned>(div_up(c_out, 32 * wn)));
    auto x = static_cast<const _Float16 *>(sources);
    auto wt = static_cast<const _Float16 *>(workspace);
    if (wn == 1)
      hipLaunchKernelGGL((ws_fused_f16_kernel<1>), grid, dim3(256), 0, stream, in_idx, out_idx, naddrs, qnaddrs, rows,
                         nfwd, Kw, weight_offset, x, c_in, wt, c_out, target_acc);
    else if (wn == 2)
      hipLaunchKernelGGL((ws_fused_f16_kernel<2>), grid, dim3(256), 0, stream, in_idx, out_idx, naddrs, qnaddrs, rows,
                         nfwd, Kw, weight_offset, x, c_in, wt, c_out, target_acc);
    else
      hipLaunchKernelGGL((ws_fused_f16_kernel<4>), grid, dim3(256), 0, stream, in_idx, out_idx, naddrs, qnaddrs, rows,
                         nfwd, Kw, weight_offset, x, c_in, wt, c_out, target_acc);
  } else {
    const int64_t n = (Kw > 0 ? 2 : 1) * num_pairs * c_out;
    if (dtype == SPIRA_F16)
      hipLaunchKernelGGL(ws_fused_generic_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, in_idx,
                         out_idx, naddrs, rows, Kw, weight_offset, Kw > 0 ? 1 : 0, num_pairs,
                         static_cast<const _Float16 *>(sources), c_in, static_cast<const _Float16 *>(weights), c_out,
                         target_acc);
    else
      hipLaunchKernelGGL(ws_fused_generic_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, in_idx, out_idx,
                         naddrs, rows, Kw, weight_offset, Kw > 0 ? 1 : 0, num_pairs,
                         static_cast<const float *>(sources), c_in, static_cast<const float *>(weights), c_out,
                         target_acc);
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_ws_gather(int64_t num_sources, int c_in, int num_offsets, int dtype, const void *sources,
                        const int32_t *source_masks, const int64_t *padded_offsets, void *buffer, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(num_offsets <= kMaxGroups, "ws_gather: at most 128 offsets");
  if (num_sources <= 0 || num_offsets <= 0) return kOk;
  OffsetTable ot{};
  ot.n = num_offsets;
  for (int k = 0; k < num_offsets; ++k) ot.off[k] = padded_offsets[k];
  if (dtype == SPIRA_F16 && c_in % 8 == 0) {
    const int64_t n = num_sources * (c_in / 8);
    hipLaunchKernelGGL(gather_h8_kernel, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_sources, c_in,
                       source_masks, static_cast<const _Float16 *>(sources), static_cast<_Float16 *>(buffer));
  } else if (dtype == SPIRA_F16) {
    const int64_t n = num_sources * c_in;
    hipLaunchKernelGGL(gather_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_sources, c_in,
                       source_masks, static_cast<const _Float16 *>(sources), static_cast<_Float16 *>(buffer));
  } else {
    const int64_t n = num_sources * c_in;
    hipLaunchKernelGGL(gather_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_sources, c_in,
                       source_masks, static_cast<const float *>(sources), static_cast<float *>(buffer));
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_ws_gemm(int num_offsets, const int32_t *rows, const int64_t *padded_offsets, int c_in, int c_out,
                      int dtype, const void *buffer_in, const void *weights, float *buffer_out, void *workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  GroupTable gt{};
  int rc = fill_groups(gt, num_offsets, rows, padded_offsets);
  if (rc) return rc;
  if (num_offsets <= 0) return kOk;
  if (mfma_ok(dtype, c_in)) {
    SPIRA_HIP_REQUIRE(workspace && workspace_bytes >= wt_bytes(num_offsets, c_in, c_out),
                      "ws_gemm: workspace too small");
    rc = transpose_weights(weights, num_offsets, c_in, c_out, workspace, stream);
    if (rc) return rc;
    const int64_t tiles = gt.tile_start[num_offsets];
    if (tiles == 0) return kOk;
    const int wn = wn_for(c_out);
    dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(div_up(c_out, 32 * wn)));
    auto x = static_cast<const _Float16 *>(buffer_in);
    auto wt = static_cast<const _Float16 *>(workspace);
    if (wn == 1)
      hipLaunchKernelGGL((group_gemm_f16_kernel<1>), grid, dim3(256), 0, stream, gt, x, c_in, wt, c_out, buffer_out);
    else if (wn == 2)
      hipLaunchKernelGGL((group_gemm_f16_kernel<2>), grid, dim3(256), 0, stream, gt, x, c_in, wt, c_out, buffer_out);
    else
      hipLaunchKernelGGL((group_gemm_f16_kernel<4>), grid, dim3(256), 0, stream, gt, x, c_in, wt, c_out, buffer_out);
  } else {
    int64_t total = 0;
    for (int k = 0; k < num_offsets; ++k) total = std::max<int64_t>(total, padded_offsets[k] + rows[k]);
    const int64_t n = total * c_out;
    if (n == 0) return kOk;
    if (dtype == SPIRA_F16)
      hipLaunchKernelGGL(group_gemm_generic_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, gt, total,
                         static_cast<const _Float16 *>(buffer_in), c_in, static_cast<const _Float16 *>(weights),
                         c_out, buffer_out);
    else
      hipLaunchKernelGGL(group_gemm_generic_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, gt, total,
                         static_cast<const float *>(buffer_in), c_in, static_cast<const float *>(weights), c_out,
                         buffer_out);
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_ws_scatter(int64_t num_targets, int c_out, int num_offsets, int dtype, const int32_t *target_masks,
                         const int64_t *padded_offsets, const float *buffer, const float *base, void *targets,
                         hipStream_t stream) {
  SPIRA_HIP_REQUIRE(num_offsets <= kMaxGroups, "ws_scatter: at most 128 offsets");
  if (num_targets <= 0) return kOk;
  OffsetTable ot{};
  ot.n = num_offsets;
  for (int k = 0; k < num_offsets; ++k) ot.off[k] = padded_offsets[k];
  const int64_t n = num_targets * c_out;
  if (dtype == SPIRA_F16)
    hipLaunchKernelGGL(scatter_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_targets, c_out,
                       target_masks, buffer, static_cast<_Float16 *>(targets), base);
  else
    hipLaunchKernelGGL(scatter_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_targets, c_out,
                       target_masks, buffer, static_cast<float *>(targets), base);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_cast_f32(const float *src, int64_t n, int dtype, void *dst, hipStream_t stream) {
  if (n <= 0) return kOk;
  if (dtype == SPIRA_F16)
    hipLaunchKernelGGL(cast_f32_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, src, n,
                       static_cast<_Float16 *>(dst));
  else
    hipLaunchKernelGGL(cast_f32_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, src, n,
                       static_cast<float *>(dst));
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

}  // extern "C"
