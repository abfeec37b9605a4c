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
// MI355X design (fp16 storage, fp32 accumulation on v_mfma_f32_16x16x32_f16).
// All three dataflows share one MMA core:
//  * a block is 4 waves; a wave owns a tile of 32 rows (two 16-row MFMA
//    tiles) x 32*WN columns; WN = 1, 2, 3 or 4 (wider layers take several
//    128-column tiles), so that 96-channel layers do not pad to a power of
//    two.  The tiles are small on purpose: the kernels are bound by the
//    latency of their gathers, not by any one unit, and small tiles let 2-4
//    waves share each SIMD;
//  * the K dimension is walked in steps of 32, 64 or 128 input channels of
//    one kernel offset.  The offset's weight chunk (shared by the four waves)
//    lands in a 2-4 stage LDS ring through buffer_load ... lds (direct
//    HBM/L2 -> LDS) with an XOR swizzle that makes the B reads
//    conflict-free; the gathered rows (private to a wave) are loaded straight
//    into the registers of the MFMA A operand (lane L fetches exactly the 16
//    bytes its A slot needs: one load covers 16 rows x 64 bytes).  Loads run
//    NS - 1 steps ahead of the MFMAs and are issued slice by slice between
//    the current step's weight reads and MFMAs; a step costs one workgroup
//    barrier and one vmcnt wait, and rows without a neighbour read a 16-byte
//    zero block instead of branching;
//  * weights are prepared once per weight tensor into [K, CoutP, CinP]
//    (transposed, zero-padded to 32 output / 16 input channels), so odd
//    channel counts (the 3-channel stem) take the same path;
//  * the output-stationary kernel can walk its rows in neighbour-mask order
//    (rows with the same neighbour pattern together) and visits only the
//    offsets some row of the block uses; small layers split the offsets over
//    blocks (fp32 atomics into a workspace that stays zeroed + finalize);
//  * an optional epilogue folds a per-channel scale / shift (eval-mode batch
//    norm), a residual add and ReLU into the output write.
#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace spira_hip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uint32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

constexpr int kMaxGroups = 128;

enum OutMode { kStoreNative = 0, kStoreF32 = 1, kAddF32 = 2, kAtomicF32 = 3 };

// Work balance of the output-stationary kernel (storage-dtype outputs).
// A row-ordered map puts rows with many neighbours together, so its row
// tiles need from a few to all of the kernel's offsets, and the launch lasts
// as long as its longest tile.  With offsets > 0 a row tile with more than
// that many valid offsets (its group mask) is split over up to zmax
// blocks, ceil(valid / offsets) of them.  split_items_kernel lists the launch's work items
// (row tile t, part p) in row-tile order, items[0 .. *total); grid x walks
// them (blocks past the list exit), so that a tile's parts run together and
// no block waits behind empty ones.  Part p of z takes the tile's valid
// offsets of rank [p n / z, (p + 1) n / z) and writes its fp32 partial tile
// to part[(tile * zmax + p) * BM * BN ...] (tile = row tile * gy + column
// tile); a tile that is not split is stored by its one block.
// split_finalize_kernel then sums each split tile's parts in order
// 0 .. z - 1 and writes the output with the epilogue.  (Summing in the last
// part to finish instead needs device-coherent partial tiles: an L2
// writeback per block, or stores and loads that bypass the L2s, both
// measured 1.5-5x slower than the separate pass.)  The list and the partial
// tiles live in the workspace, which arrives zeroed and is left zeroed.
struct TileSplit {
  int offsets;  // 0: off
  int zmax;
  float *part;
  int32_t *items;  // (t << 3) | p
  int32_t *total;
};

// The number of parts of a row tile whose group mask is (lo, hi).
__host__ __device__ __forceinline__ int split_parts(uint64_t lo, uint64_t hi, int Kc, int offsets, int zmax) {
  const uint64_t klo = Kc >= 64 ? ~uint64_t(0) : (uint64_t(1) << Kc) - 1;
  const uint64_t khi = Kc >= 128 ? ~uint64_t(0) : (Kc > 64 ? (uint64_t(1) << (Kc - 64)) - 1 : 0);
  const int nact = __builtin_popcountll(lo & klo) + __builtin_popcountll(hi & khi);
  const int want = (nact + offsets - 1) / offsets;
  return want < 1 ? 1 : (want > zmax ? zmax : want);
}

struct Epilogue {
  const float *scale;    // [Cout] or null
  const float *shift;    // [Cout] or null
  const void *residual;  // [T, Cout] in the storage dtype, or null
  int relu;
  TileSplit split;       // (os_kernel with storage-dtype outputs only)
};

// Gathered operands of the MMA core.  Both are addressed through buffer
// resources with 32-bit byte offsets: a lane whose row is missing (or whose
// channels lie in the padding) uses an offset past the end, and the buffer
// unit then returns zeros instead of reading memory.
struct Operands {
  const _Float16 *X;  // [rows, C1] gathered rows: input channels 0 .. C1-1
  uint32_t xbytes;
  const _Float16 *X2;  // [rows, Cin - C1]: channels C1 .. Cin-1 (a channel concatenation), or null
  uint32_t x2bytes;
  int C1;  // channels held by X (Cin without X2; a multiple of 32 with it)
  int Cin, CinP;
  const _Float16 *WT;  // prepared weights [K, CoutP, CinP]
  uint32_t wbytes;
  int Cout, CoutP;
};
constexpr uint32_t kOutOfRange = 0x80000000u;  // > every buffer size (sizes are < 2^31)
constexpr int kRsrcWord3 = 0x00020000;         // raw (untyped) buffer, 32-bit data format
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, static_cast<int>(bytes), kRsrcWord3);
}
// The same descriptor as four words (base address, stride 0, size, flags),
// for the inline-assembly loads of load16.
__device__ __forceinline__ uint32x4 rsrc_words(const void *p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  uint32x4 r;
  r[0] = static_cast<uint32_t>(a);
  r[1] = static_cast<uint32_t>(a >> 32) & 0xffffu;
  r[2] = bytes;
  r[3] = static_cast<uint32_t>(kRsrcWord3);
  return r;
}
// 16 bytes at byte offset `off` of buffer `r` into v, in place: the
// register is v's own (tied operand), so the compiler neither waits for the
// load nor moves the value while it is in flight.  The caller waits
// (vmcnt) before reading v and ties the value after the wait with pin().
// (With the compiler's own buffer loads, its register allocation reused the
// registers of loads still in flight and the inserted waits drained every
// load of the pipeline at the start of 4 of the 6 unrolled steps.)
__device__ __forceinline__ void load16(half8 &v, uint32x4 r, uint32_t off) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "+v"(v) : "v"(off), "s"(r) : "memory");
}


namespace ring {

// Ring layout: stage s at byte s * STAGE holds the step's weight chunk
// (BN rows x ROWB = KC * 2 bytes, 16-byte chunks XOR-swizzled per row),
// shared by the block's four waves.  The gathered rows are private to a wave
// and go straight into registers (one 16-byte buffer load per lane, 16-row
// tile and 32-channel block: the MFMA A layout), so they cost no LDS
// bandwidth.  A step covers KC = 16 * NKS input channels of one kernel
// offset: NKS = 2, 4 or 8 (32, 64 or 128 channels: fewer steps and so less
// per-step synchronisation for wide layers).
constexpr int kMapTileK = 27;  // map columns held in LDS (kernels of <= 27 offsets)
template <int WN, int MT, int NS_, int NKS_> struct Cfg {
  static constexpr int NS = NS_;  // ring depth: NS - 1 steps load while one computes
  static constexpr int NKS = NKS_;
  static constexpr int KC = 16 * NKS;  // input channels per step
  static constexpr int ROWB = KC * 2;  // bytes of a weight row per step
  static constexpr int CPR = ROWB / 16;  // 16-byte chunks per weight row
  static constexpr int BN = 32 * WN;
  static constexpr int BM = 128 * MT;
  static constexpr int BVEC = (BN * CPR + 255) / 256;  // 16-byte weight vectors per thread and step
  static constexpr int B_BYTES = BVEC * 4096;
  static constexpr int STAGE = B_BYTES;
  static constexpr int RING = NS * STAGE;
  static constexpr int OUT_STAGE = BM * (BN + 8) * 2;  // fp16 output tile staged by the epilogue
  static constexpr int MAP_TILE_K = kMapTileK;
  static constexpr int MAP_TILE = BM * MAP_TILE_K * 4;  // the block's map rows, after the ring
  static constexpr int LDS = RING + MAP_TILE > OUT_STAGE ? RING + MAP_TILE : OUT_STAGE;
  static constexpr int LPS = MT * NKS + BVEC;  // vector-memory loads per wave and step
  static_assert(NKS == 2 || NKS == 4 || NKS == 8, "a step is 32, 64 or 128 channels");
  static_assert(MT == 1, "a wave owns 32 rows: two 16-row MFMA tiles");
  // every LDS read offset of a stage is an instruction immediate (< 64 KiB)
  static_assert((NS - 1) * STAGE + (WN - 1) * 32 * ROWB < 65536, "weight read offset exceeds 16 bits");
  static_assert((NS - 2) * LPS + (NS - 1) < 64, "vmcnt range");
  // physical chunk of logical chunk c of weight row n: a 16-byte LDS read
  // serves 16 lanes (16 rows at one logical chunk) per cycle, and they are
  // conflict-free when their byte addresses differ mod 256 (64 banks): rows
  // of ROWB = 64 (128) bytes take 4 (2) positions from n, the swizzle the
  // other 4 (8) from n >> 2 (n >> 1)
  __host__ __device__ static constexpr int swz(int n) {
    return NKS == 2 ? (n >> 2) & 3 : (NKS == 4 ? (n >> 1) & 7 : n & 15);
  }
};

// Tile shape per column-tile width and step: one 32-row tile per wave (the
// kernels are latency-bound: more resident waves beat larger wave tiles),
// the ring depth, and the blocks per CU the launch planning counts on
// (WAVES: 4 for up to 96 columns, 3 for 128).  The compiler's occupancy
// target (OCC) is the most waves per SIMD that each tile reaches without
// spilling inside the step loop: 4 for 32-column tiles, 3 for 64 and 96
// columns and 2 for 128 with 32- and 64-channel steps; 2 for the tiles
// wider than 32 columns with 128-channel steps, whose weight fragments are
// double-buffered (compute).  The DA = 2 build of the two-step-gather kernel targets
// one wave per SIMD (its accumulators then sit in AGPRs and its loop is
// scheduled with room to spare), for launches of about one block per CU.
// (Measured, kernel only: s8 256 -> 256 row-ordered, 128-column tiles and
// 128-channel steps, 84.7 -> 66.3 us; s8 384 -> 256 124.9 -> 95.8 us; the
// 529-block s4 128 -> 128 layer at the same tile went 51.1 -> 58.5 us, as
// it needs two blocks per CU.)
// (32-column tiles of 32-channel steps take 3 stages, not 4: measured on the
// config-4 32 -> 32 layers, s1 18.0 -> 17.4 us, s2 20.2 -> 18.9 us.)
// DS = 1: one more ring stage for 64-channel steps of wide tiles (chosen
// where the larger blocks still fit the grid in one round, os_deep_ring).
template <int WN, int NKS = 2, int DS = 0> struct TileOf {
  static constexpr int MT = 1;
  static_assert(DS == 0 || NKS == 4 || (NKS == 8 && WN <= 2), "no room for an extra ring stage");
  static constexpr int NS = (NKS == 2 ? (WN == 2 ? 4 : 3) : (NKS == 8 || WN >= 3 ? 2 : 3)) + DS;
  static constexpr int WAVES = WN <= 3 ? 4 : 3;
  // (only 128-channel steps double-buffer their weight fragments)
  static constexpr int OCC = NKS == 8 ? (WN == 1 ? (DS == 1 ? 3 : 4) : 2) : (WN == 1 ? 4 : (WN <= 3 ? 3 : 2));
  using C = Cfg<WN, MT, NS, NKS>;
};

// compile-time loop: f(std::integral_constant<int, I>) for I in [0, N)
template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F> __device__ __forceinline__ void unroll(F &&f) {
  unroll_seq(f, std::make_integer_sequence<int, N>{});
}

// 4 bytes per lane from buffer `r` at byte offset `off` into
// lds_wave_base + lane * 4; the LDS base must be wave-uniform.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t off, void *lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(lds_wave_base), 4, off, 0, 0, 0);
}

// wait until at most N vector-memory operations of this wave are in flight
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS reads of the ring are inline assembly with immediate offsets from a
// few per-lane base registers.  The compiler then inserts no waits of its own
// for them (its LDS-DMA tracking loses precision at the loop header and
// would drain the whole ring there) and cannot hoist one address register per
// read and stage out of the loop; the ring's explicit vmcnt wait + barrier
// orders them after the DMA writes, lds_wait() after their own completion.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t *)(const_cast<void *>(p))));
}
template <int OFF> __device__ __forceinline__ half8 rd16(uint32_t base) {
  half8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(OFF) : "memory");
  return v;
}
template <int OFF> __device__ __forceinline__ int32_t rd4(uint32_t base) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(OFF) : "memory");
  return v;
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// ties a value read by rd16 / rd4 to a point after lds_wait()
template <class V> __device__ __forceinline__ void pin(V &v) { asm volatile("" : "+v"(v)); }

// per-lane LDS read bases of the ring: the weight fragment of 32-channel
// block kq (v_mfma_f32_16x16x32_f16 B layout: lane l holds column l % 16,
// channels 8 (l / 16) .. + 7 of the block), + s * STAGE + nb * 16 * ROWB for
// stage s and 16-column tile nb (the swizzle depends on l % 16 only)
template <int NKS> struct ReadBase {
  uint32_t b[NKS / 2];
};
template <class C> __device__ __forceinline__ ReadBase<C::NKS> read_base(const char *ring) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lq = lane >> 4;
  const uint32_t base = lds_addr(ring);
  ReadBase<C::NKS> rb;
#pragma unroll
  for (int kq = 0; kq < C::NKS / 2; ++kq) rb.b[kq] = base + (l16 * C::CPR + ((4 * kq + lq) ^ C::swz(l16))) * 16;
  return rb;
}

// Per-lane constants of a pipeline's loads, computed once per block so that
// a step's issue is a few adds and selects per load (the step loop is bound
// by instruction issue, not by the memory system).
template <class C> struct IssueCtx {
  uint32_t wlane[C::BVEC];  // byte offset of the lane's weight chunk in an (offset, kb = 0) block, or kOutOfRange
  int c8[C::BVEC];          // first input channel of that chunk (OP > 1: the step's offset part it belongs to)
  uint32_t ldsw;            // LDS address of the wave's DMA slot in stage 0 (wave-uniform)
  uint32_t kh16;            // byte offset of the lane's quarter of a 32-channel block
  int kh8;                  // its first channel
};
// OP > 1 (OP kernel offsets per step, KC = OP CinP): channel c of a step is
// channel c % CinP of the step's offset c / CinP.
template <class C, int OP = 1>
__device__ __forceinline__ IssueCtx<C> issue_ctx(const char *ring, int wave, int n0, const Operands &op) {
  IssueCtx<C> cx;
  const int tid = threadIdx.x & 255;
#pragma unroll
  for (int i = 0; i < C::BVEC; ++i) {
    const int v = i * 256 + tid;
    const int n = v / C::CPR;
    const int c8 = ((v % C::CPR) ^ C::swz(n)) * 8;
    const int part = OP > 1 ? c8 / op.CinP : 0;
    const int ch = c8 - part * op.CinP;
    // (columns past C_out: their prepared weights are zero padding, and the
    // out-of-range DMA writes the same zeros without reading them)
    cx.wlane[i] = (n < C::BN && n0 + n < op.Cout) ? static_cast<uint32_t>(((n0 + n) * op.CinP + ch) * 2)
                                                    : kOutOfRange;
    cx.c8[i] = OP > 1 ? part : c8;
  }
  cx.ldsw = __builtin_amdgcn_readfirstlane(lds_addr(ring) + wave * 64 * 16);
  cx.kh8 = ((threadIdx.x & 63) >> 4) * 8;
  cx.kh16 = static_cast<uint32_t>(cx.kh8 * 2);
  return cx;
}

// The operands of one step: the gathered row of the lane in each of the
// wave's two 16-row tiles, idx[rt] (source row of tile row l % 16, or -1),
// weight row wrow, first input channel kb; !live: a step past the end (every
// load out of range, so that each wave issues the same number of loads in
// every step).
// OP > 1 (offset packing): idxp / wrowp / livep[p - 1] describe the step's
// offset p = 1 .. OP - 1.
struct StepIn {
  bool live;
  int32_t idx[2];
  int wrow, kb;
  bool livep[3];
  int32_t idxp[3][2];
  int wrowp[3];
};

// The value of offset part p of a packed step (OP = 2 or 4).
template <int OP, class T> __device__ __forceinline__ T part_sel(int p, T v0, T v1, T v2, T v3) {
  if constexpr (OP == 2) return p ? v1 : v0;
  else return p < 2 ? (p ? v1 : v0) : (p == 2 ? v2 : v3);
}

// Issue the loads of slice KS of a step into ring stage S: the A fragment
// of row tile rt = KS % 2 and 32-channel block kq = KS / 2 (lane l: its row
// idx[rt], channels kb + 32 kq + 8 (l / 16) .. + 7, the
// v_mfma_f32_16x16x32_f16 A layout: one instruction reads 16 rows x 64
// bytes) into a[0][KS], and the weight DMAs i = KS, KS + NKS, ... (a step's
// slices together issue every load of the step, in slice order).  CAT: the
// input is a channel concatenation [X | X2] (each 32-channel block lies
// wholly in one part, C1 % 32 == 0).  The offsets use 32-bit arithmetic:
// every operand is below 2 GiB.
//
// OP = 2 or 4 (offset packing for 16- and 32-channel inputs, KC = OP CinP,
// one channel chunk per offset): channels [p CinP, (p + 1) CinP) of the step
// belong to its offset p; the lane picks its row and each weight DMA its
// weight row by the part its channels fall in.
template <class C, bool ALIGNED, bool CAT, int S, int KS, int OP = 1>
__device__ __forceinline__ void issue_slice(const IssueCtx<C> &cx, const StepIn &st, const Operands &op,
                                            __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t xr2,
                                            __amdgpu_buffer_rsrc_t wr, half8 (&a)[1][C::NKS]) {
  constexpr int rt = KS & 1;
  const int k0 = st.kb + (KS >> 1) * 32;
  if constexpr (OP > 1) {
    static_assert(ALIGNED && !CAT, "offset packing: aligned rows of one source");
    constexpr int CP = C::KC / OP;          // channels per offset (16 or 32)
    const int k = (KS >> 1) * 32 + cx.kh8;  // the lane's channel within the step
    const int part = k / CP;
    const int ch = k - part * CP;
    const int32_t ix = part_sel<OP>(part, st.idx[rt], st.idxp[0][rt], st.idxp[1][rt], st.idxp[2][rt]);
    const bool lv = part_sel<OP>(part, st.live, st.livep[0], st.livep[1], st.livep[2]);
    const bool ok = lv & (ix >= 0) & (ch < op.Cin);
    const uint32_t at = static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.Cin * 2) + static_cast<uint32_t>(ch * 2);
    a[0][KS] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? at : kOutOfRange, 0, 0));
    const uint32_t wb = static_cast<uint32_t>(op.CoutP * op.CinP * 2);
    // (a part past the step's last offset: out of range)
    const uint32_t w0 = st.live ? static_cast<uint32_t>(st.wrow) * wb : kOutOfRange;
    uint32_t wp[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) wp[q] = st.livep[q] ? static_cast<uint32_t>(st.wrowp[q]) * wb : kOutOfRange;
#pragma unroll
    for (int i = KS; i < C::BVEC; i += C::NKS) {
      const uint32_t ws = part_sel<OP>(cx.c8[i], w0, wp[0], wp[1], wp[2]);
      const uint32_t off = (ws == kOutOfRange || cx.wlane[i] == kOutOfRange) ? kOutOfRange : cx.wlane[i] + ws;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void_t *)(cx.ldsw + S * C::STAGE + i * 4096), 16, off, 0, 0,
                                               0);
    }
    return;
  }
  {
    constexpr int m = 0;
    // branch-free selects: a divergent branch here would make both sides
    // write the destination registers, and the second write would have to
    // wait for every load in flight
    const int32_t ix = st.idx[rt];
    const bool rv = st.live & (ix >= 0);
    if constexpr (!ALIGNED) {
      // rows that are not 16-byte aligned: element loads (still one
      // vector-memory op per k-half in the count, the first element's)
      const int k = k0 + cx.kh8;
      const uint32_t off = (rv & (k < op.Cin)) ? (static_cast<uint32_t>(ix) * op.Cin + k) * 2u : kOutOfRange;
      half8 v;
      v[0] = __builtin_bit_cast(_Float16, static_cast<unsigned short>(
                                              __builtin_amdgcn_raw_buffer_load_b16(xr, off, 0, 0)));
#pragma unroll
      for (int e = 1; e < 8; ++e)
        v[e] = (rv && k + e < op.Cin) ? op.X[static_cast<int64_t>(ix) * op.Cin + k + e]
                                      : static_cast<_Float16>(0.f);
      a[m][KS] = v;
    } else {
      const bool ok = rv & (cx.kh8 < op.Cin - k0);
      if constexpr (CAT) {
        const bool second = k0 >= op.C1;  // block-uniform
        const uint32_t at = second ? static_cast<uint32_t>(ix) * static_cast<uint32_t>((op.Cin - op.C1) * 2) +
                                         static_cast<uint32_t>((k0 - op.C1) * 2)
                                   : static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.C1 * 2) +
                                         static_cast<uint32_t>(k0 * 2);
        a[m][KS] = __builtin_bit_cast(
            half8, __builtin_amdgcn_raw_buffer_load_b128(second ? xr2 : xr, ok ? at + cx.kh16 : kOutOfRange, 0, 0));
      } else {
        const uint32_t rb1 = static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.C1 * 2);
        a[m][KS] = __builtin_bit_cast(
            half8, __builtin_amdgcn_raw_buffer_load_b128(
                       xr, ok ? rb1 + static_cast<uint32_t>(k0 * 2) + cx.kh16 : kOutOfRange, 0, 0));
      }
    }
  }
  // weights: chunk c8 of the lane's row holds input channels while c8 <
  // Cin - kb (the chunks past it are zero padding, which the out-of-range
  // DMA writes without reading); an out-of-range lane offset stays out of
  // range after adding the step's (wstep < wbytes < 2^31)
  const uint32_t wstep = static_cast<uint32_t>((st.wrow * op.CoutP * op.CinP + st.kb) * 2);
  const int wlim = st.live ? op.Cin - st.kb : 0;
#pragma unroll
  for (int i = KS; i < C::BVEC; i += C::NKS) {
    const uint32_t off = cx.c8[i] < wlim ? cx.wlane[i] + wstep : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void_t *)(cx.ldsw + S * C::STAGE + i * 4096), 16, off, 0, 0, 0);
  }
}

// Every load of a step, slice after slice (the prologue's steps).
template <class C, bool ALIGNED, bool CAT, int S, int OP = 1>
__device__ __forceinline__ void issue(const IssueCtx<C> &cx, const StepIn &st, const Operands &op,
                                      __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t xr2,
                                      __amdgpu_buffer_rsrc_t wr, half8 (&a)[1][C::NKS]) {
  unroll<C::NKS>(
      [&](auto KS) { issue_slice<C, ALIGNED, CAT, S, decltype(KS)::value, OP>(cx, st, op, xr, xr2, wr, a); });
}

// MFMAs of stage S (rows without a neighbour hold zeros): per 32-channel
// block kq, the weight fragments of the BN / 16 column tiles, then
// v_mfma_f32_16x16x32_f16 for both row tiles.  Wide tiles take their weight
// fragments in two halves (fewer live registers), so a step is a sequence
// of phases (kq, half).  With 128-channel steps the fragments are
// double-buffered: a phase's LDS reads are issued before the previous
// phase's MFMAs, and each phase waits only for its own reads (lgkmcnt = the
// reads issued after them; LDS reads complete in order), so that a wave's
// LDS reads overlap its MFMAs instead of alternating with them.  (Shorter
// steps keep one buffer: the second cost them a wave per SIMD.)  between(KQ) runs after block kq's first weight
// reads are issued: the next step's loads issued there overlap the LDS
// latency and the MFMAs, instead of all waves of the block issuing them in
// one burst after the barrier.  acc[rt][nb]: lane l holds rows 4 (l / 16) +
// i (i < 4) of row tile rt, column l % 16 of column tile nb.
template <int N> __device__ __forceinline__ void lds_wait_n() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
template <class C, int S, class Between>
__device__ __forceinline__ void compute(floatx4 (&acc)[2][C::BN / 16], const ReadBase<C::NKS> &rb,
                                        const half8 (&a)[1][C::NKS], Between between) {
  constexpr int NB = C::BN / 16;
  constexpr int NH = NB > 4 ? 2 : 1, NBH = NB / NH;
  constexpr int NP = (C::NKS / 2) * NH;  // phases (kq, half)
  constexpr bool DB = C::NKS == 8;        // double-buffered fragments
  static_assert(NB % NH == 0, "column tiles split evenly");
  half8 b[DB ? 2 : 1][NBH];
  auto rd = [&](auto P) {
    constexpr int p = decltype(P)::value, kq = p / NH, h = p % NH;
    unroll<NBH>([&](auto B) {
      constexpr int nb = decltype(B)::value;
      b[DB ? (p & 1) : 0][nb] = rd16<S * C::STAGE + (h * NBH + nb) * 16 * C::ROWB>(rb.b[kq]);
    });
  };
  if constexpr (DB) rd(std::integral_constant<int, 0>{});
  unroll<NP>([&](auto P) {
    constexpr int p = decltype(P)::value, kq = p / NH, h = p % NH;
    constexpr int cur = DB ? (p & 1) : 0;
    if constexpr (!DB) rd(P);
    else if constexpr (p + 1 < NP) rd(std::integral_constant<int, p + 1>{});
    if constexpr (h == 0) between(std::integral_constant<int, kq>{});
    if constexpr (DB && p + 1 < NP) lds_wait_n<NBH>();
    else lds_wait();
#pragma unroll
    for (int nb = 0; nb < NBH; ++nb) pin(b[cur][nb]);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int nb = 0; nb < NBH; ++nb)
        acc[rt][h * NBH + nb] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0][2 * kq + rt], b[cur][nb], acc[rt][h * NBH + nb], 0, 0, 0);
  });
}

// The pipelined step loop over nsteps steps; stage u % NS of the ring holds
// step u.  Two callbacks describe the steps (S = the stage, a
// std::integral_constant):
//  * fetch(u, S) issues exactly PL LDS-DMA loads per wave that bring step
//    u's row indices into the caller's index slot S (also for u >= nsteps,
//    so that the vmcnt arithmetic is the same in every wave);
//  * resolve(u, S, st) turns them into step u's operands st (the lane's
//    gathered rows idx[rt] (or -1), the weight row and the first input
//    channel; OP = 2 also the second offset's).
// Both are called with u = 0, 1, 2, ... in order (fetch NS steps ahead of
// resolve).  Issue order: F(0..NS-1), then per step u: D(u) F(u+NS)
// (D = the LPS LDS-DMA loads of a step, F = a fetch).  Before step s
// computes, D(s) must be complete while F(s+NS) and D/F of the NS-2 younger
// steps may still be in flight: vmcnt((NS-2) LPS + (NS-1) PL).  F(s+NS-1),
// which step s+NS-1's issue reads, is older than D(s) and covered by the
// same wait.  F(u+NS) overwrites the index slot that step u's issue has
// just read (each wave reads only its own slot).  Steps past nsteps (at most
// NS-1) compute on all-zero stages, so the trip is uniform and the
// accumulators stay in place.
template <class C, bool ALIGNED, bool CAT, int PL, int OP = 1, class Fetch, class Resolve>
__device__ __forceinline__ void run(floatx4 (&acc)[2][C::BN / 16], int nsteps, Fetch fetch,
                                    Resolve resolve, const Operands &op, int n0, char *ring) {
  constexpr int MT = C::BM / 128, NS = C::NS;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(op.X, op.xbytes);
  const __amdgpu_buffer_rsrc_t xr2 = make_rsrc(op.X2 ? op.X2 : op.X, op.X2 ? op.x2bytes : 0u);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(op.WT, op.wbytes);
  const ReadBase<C::NKS> rb = read_base<C>(ring);
  const IssueCtx<C> cx = issue_ctx<C, OP>(ring, wave, n0, op);
  half8 areg[NS][MT][C::NKS];  // gathered rows per stage
  auto prepare = [&](int u, auto St) {
    StepIn st;
    st.wrow = 0;
    st.kb = 0;
    st.live = u < nsteps;
    st.idx[0] = st.idx[1] = -1;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      st.livep[q] = false;
      st.wrowp[q] = 0;
      st.idxp[q][0] = st.idxp[q][1] = -1;
    }
    if (st.live) resolve(u, St, st);
    return st;
  };
  auto put = [&](int u, auto St) {
    const StepIn st = prepare(u, St);
    issue<C, ALIGNED, CAT, decltype(St)::value, OP>(cx, st, op, xr, xr2, wr, areg[decltype(St)::value]);
  };
  unroll<NS>([&](auto I) { fetch(decltype(I)::value, I); });
  unroll<NS - 1>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if constexpr (PL > 0) wait_vm<(NS - 1) * PL + i * C::LPS>();  // F(i) is older than these
    put(i, I);
    fetch(i + NS, I);
  });
  for (int s = 0; s < nsteps; s += NS) {
    unroll<NS>([&](auto I) {
      constexpr int i = decltype(I)::value;
      constexpr int slot = (i + NS - 1) % NS;
      wait_vm<(NS - 2) * C::LPS + (NS - 1) * PL>();
      __builtin_amdgcn_s_barrier();
      const StepIn nx = prepare(s + i + NS - 1, std::integral_constant<int, slot>{});
      compute<C, i>(acc, rb, areg[i], [&](auto KQ) {
        issue_slice<C, ALIGNED, CAT, slot, 2 * decltype(KQ)::value, OP>(cx, nx, op, xr, xr2, wr, areg[slot]);
        issue_slice<C, ALIGNED, CAT, slot, 2 * decltype(KQ)::value + 1, OP>(cx, nx, op, xr, xr2, wr, areg[slot]);
      });
      fetch(s + i + 2 * NS - 1, std::integral_constant<int, slot>{});
    });
  }
  wait_vm<0>();
}

// The A loads (gathered rows, slice KS) of a step, as issue_slice issues
// them (OP = 1).
template <class C, bool ALIGNED, bool CAT, int KS>
__device__ __forceinline__ void issue_a(const IssueCtx<C> &cx, const StepIn &st, const Operands &op,
                                        __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t xr2,
                                        half8 (&a)[1][C::NKS]) {
  constexpr int rt = KS & 1;
  const int k0 = st.kb + (KS >> 1) * 32;
  const int32_t ix = st.idx[rt];
  const bool rv = st.live & (ix >= 0);
  if constexpr (!ALIGNED) {
    const int k = k0 + cx.kh8;
    const uint32_t off = (rv & (k < op.Cin)) ? (static_cast<uint32_t>(ix) * op.Cin + k) * 2u : kOutOfRange;
    half8 v;
    v[0] = __builtin_bit_cast(_Float16, static_cast<unsigned short>(
                                            __builtin_amdgcn_raw_buffer_load_b16(xr, off, 0, 0)));
#pragma unroll
    for (int e = 1; e < 8; ++e)
      v[e] = (rv && k + e < op.Cin) ? op.X[static_cast<int64_t>(ix) * op.Cin + k + e] : static_cast<_Float16>(0.f);
    a[0][KS] = v;
  } else {
    const bool ok = rv & (cx.kh8 < op.Cin - k0);
    if constexpr (CAT) {
      const bool second = k0 >= op.C1;
      const uint32_t at = second ? static_cast<uint32_t>(ix) * static_cast<uint32_t>((op.Cin - op.C1) * 2) +
                                       static_cast<uint32_t>((k0 - op.C1) * 2)
                                 : static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.C1 * 2) +
                                       static_cast<uint32_t>(k0 * 2);
      a[0][KS] = __builtin_bit_cast(
          half8, __builtin_amdgcn_raw_buffer_load_b128(second ? xr2 : xr, ok ? at + cx.kh16 : kOutOfRange, 0, 0));
    } else {
      const uint32_t rb1 = static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.C1 * 2);
      a[0][KS] = __builtin_bit_cast(
          half8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? rb1 + static_cast<uint32_t>(k0 * 2) + cx.kh16
                                                              : kOutOfRange,
                                                       0, 0));
    }
  }
}

// Every weight DMA of a step into ring stage S (OP = 1).
template <class C, int S>
__device__ __forceinline__ void issue_b(const IssueCtx<C> &cx, const StepIn &st, const Operands &op,
                                        __amdgpu_buffer_rsrc_t wr) {
  const uint32_t wstep = static_cast<uint32_t>((st.wrow * op.CoutP * op.CinP + st.kb) * 2);
  const int wlim = st.live ? op.Cin - st.kb : 0;  // (chunks past C_in: zero padding)
#pragma unroll
  for (int i = 0; i < C::BVEC; ++i) {
    const uint32_t off = cx.c8[i] < wlim ? cx.wlane[i] + wstep : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void_t *)(cx.ldsw + S * C::STAGE + i * 4096), 16, off, 0, 0, 0);
  }
}

// The step loop with the gathered rows two steps ahead (a ring of three
// register stages) and the weights one step ahead (the two-stage LDS ring),
// for maps held in LDS (no index fetches) and one offset per step.  Per
// step v: wait for the loads of step v (the only younger loads are step
// v + 1's gathers, issued after step v's weights), barrier, then the
// weights of step v + 1 and the gathers of step v + 2 are issued between
// the MFMAs of step v.  The weights' LDS stage (v + 1) % 2 was last read by
// step v - 1, which every wave finished before the barrier.  resolve() runs
// for steps 0, 1, 2, ... in order (two steps ahead); a step's weight row and
// channel offset are kept one step for its weights.  The loop's unrolled
// period is 6 (stage v % 2, register slot v % 3); steps past nsteps are
// skipped (block-uniform).
// The A loads (gathered rows, slice KS) of a step for aligned rows of one
// source, as issue_a issues them, through load16.
template <class C, int KS>
__device__ __forceinline__ void issue_a16(const IssueCtx<C> &cx, const StepIn &st, const Operands &op, uint32x4 xw,
                                          half8 (&a)[1][C::NKS]) {
  constexpr int rt = KS & 1;
  const int k0 = st.kb + (KS >> 1) * 32;
  const int32_t ix = st.idx[rt];
  const bool ok = st.live & (ix >= 0) & (cx.kh8 < op.Cin - k0);
  const uint32_t rb1 = static_cast<uint32_t>(ix) * static_cast<uint32_t>(op.C1 * 2);
  load16(a[0][KS], xw, ok ? rb1 + static_cast<uint32_t>(k0 * 2) + cx.kh16 : kOutOfRange);
}

template <class C, bool ALIGNED, bool CAT, class Resolve>
__device__ __forceinline__ void run_da(floatx4 (&acc)[2][C::BN / 16], int nsteps, Resolve resolve,
                                       const Operands &op, int n0, char *ring) {
  static_assert(C::NS == 2 && C::BM == 128, "two LDS stages, one row tile per wave");
  constexpr int LA = C::NKS;  // gathered-row loads per wave and step
  constexpr bool A16 = ALIGNED && !CAT;  // gathers through load16
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const uint32x4 xw = rsrc_words(op.X, op.xbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(op.X, op.xbytes);
  const __amdgpu_buffer_rsrc_t xr2 = make_rsrc(op.X2 ? op.X2 : op.X, op.X2 ? op.x2bytes : 0u);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(op.WT, op.wbytes);
  const ReadBase<C::NKS> rb = read_base<C>(ring);
  const IssueCtx<C> cx = issue_ctx<C, 1>(ring, wave, n0, op);
  half8 areg[3][1][C::NKS];
  auto prepare = [&](int u) {
    StepIn st;
    st.wrow = 0;
    st.kb = 0;
    st.live = u < nsteps;
    st.idx[0] = st.idx[1] = -1;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      st.livep[q] = false;
      st.wrowp[q] = 0;
      st.idxp[q][0] = st.idxp[q][1] = -1;
    }
    if (st.live) resolve(u, std::integral_constant<int, 0>{}, st);
    return st;
  };
  auto gather = [&](auto KS, const StepIn &st, half8(&a)[1][C::NKS]) {
    if constexpr (A16) issue_a16<C, decltype(KS)::value>(cx, st, op, xw, a);
    else issue_a<C, ALIGNED, CAT, decltype(KS)::value>(cx, st, op, xr, xr2, a);
  };
  if constexpr (A16) {
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int k = 0; k < C::NKS; ++k) areg[q][0][k] = half8{};
  }
  // prologue: A(0), B(0), A(1)
  StepIn st0 = prepare(0);
  unroll<C::NKS>([&](auto KS) { gather(KS, st0, areg[0]); });
  issue_b<C, 0>(cx, st0, op, wr);
  StepIn nb = prepare(1);  // step v + 1: its weights are issued in step v
  // (the map-tile read that resolve(2) takes was issued by resolve(1), with
  // no compute, and so no LDS wait, in between)
  lds_wait();
  unroll<C::NKS>([&](auto KS) { gather(KS, nb, areg[1]); });
  for (int s = 0; s < nsteps; s += 6) {
    unroll<6>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (s + i < nsteps) {
        wait_vm<LA>();
        __builtin_amdgcn_s_barrier();
        if constexpr (A16) {
#pragma unroll
          for (int k = 0; k < C::NKS; ++k) pin(areg[i % 3][0][k]);  // (loaded: the wait covers them)
        }
        const StepIn na = prepare(s + i + 2);
        compute<C, i % 2>(acc, rb, areg[i % 3], [&](auto KQ) {
          constexpr int kq = decltype(KQ)::value;
          if constexpr (kq == 0) issue_b<C, (i + 1) % 2>(cx, nb, op, wr);
          gather(std::integral_constant<int, 2 * kq>{}, na, areg[(i + 2) % 3]);
          gather(std::integral_constant<int, 2 * kq + 1>{}, na, areg[(i + 2) % 3]);
        });
        nb = na;
      }
    });
  }
  wait_vm<0>();
  if constexpr (A16) {
    // the last steps' loads (past nsteps) land in their registers only now:
    // the registers stay reserved until this wait
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int k = 0; k < C::NKS; ++k) pin(areg[q][0][k]);
  }
}

// Scalar iterator over the set bits of a 128-bit offset set, nch channel
// chunks per offset: step() moves to the next (offset, chunk).
struct StepIter {
  uint64_t lo, hi;  // offsets not yet started (relative to j0)
  int j;            // current offset (relative)
  int chunk;
  __device__ __forceinline__ static int first(uint64_t lo, uint64_t hi) {
    return lo ? __builtin_ctzll(lo) : (hi ? 64 + __builtin_ctzll(hi) : 0);
  }
  __device__ __forceinline__ void init(uint64_t l, uint64_t h) {
    lo = l;
    hi = h;
    j = first(lo, hi);
    drop();
    chunk = 0;
  }
  __device__ __forceinline__ void drop() {
    if (j < 64) lo &= ~(uint64_t(1) << j);
    else hi &= ~(uint64_t(1) << (j - 64));
  }
  __device__ __forceinline__ void step(int nch) {
    if (++chunk == nch) {
      chunk = 0;
      j = first(lo, hi);
      drop();
    }
  }
};

// OP offsets per step (offset packing, one channel chunk per offset): j,
// jp[0 .. OP - 2] (-1 when the set has run out).
template <int OP> struct GroupIter {
  uint64_t lo, hi;
  int j, jp[OP - 1];
  static constexpr int chunk = 0;
  __device__ __forceinline__ void take(int &x) {
    if (!(lo | hi)) {
      x = -1;
      return;
    }
    x = StepIter::first(lo, hi);
    if (x < 64) lo &= ~(uint64_t(1) << x);
    else hi &= ~(uint64_t(1) << (x - 64));
  }
  __device__ __forceinline__ void step(int) {
    take(j);
#pragma unroll
    for (int q = 0; q < OP - 1; ++q) take(jp[q]);
  }
  __device__ __forceinline__ void init(uint64_t l, uint64_t h) {
    lo = l;
    hi = h;
    step(1);
  }
};

}  // namespace ring

// A wave's accumulators: 32 rows x 32 WN columns as 2 x 2 WN tiles of
// 16 x 16 (v_mfma_f32_16x16x32_f16 layout: acc[rt][nb][i] of lane l is row
// 16 rt + 4 (l / 16) + i, column 16 nb + l % 16).
template <int WN> __device__ __forceinline__ void zero_acc(floatx4 (&acc)[2][2 * WN]) {
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int nb = 0; nb < 2 * WN; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[rt][nb][i] = 0.f;
}

// Write a wave's 32-row tile; orow[row] is the output row or -1.
template <int WN, int MODE>
__device__ __forceinline__ void store_tile(const floatx4 (&acc)[2][2 * WN], const int32_t *orow, int n0, int Cout,
                                           void *Yv, const Epilogue &epi) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int nb = 0; nb < 2 * WN; ++nb) {
    const int col = n0 + nb * 16 + l16;
    if (col >= Cout) continue;
    float sc = 1.f, sh = 0.f;
    if constexpr (MODE == kStoreNative) {
      if (epi.scale) sc = epi.scale[col];
      if (epi.shift) sh = epi.shift[col];
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t o = orow[rt * 16 + lq * 4 + i];
        if (o < 0) continue;
        float v = acc[rt][nb][i];
        const int64_t at = static_cast<int64_t>(o) * Cout + col;
        if constexpr (MODE == kStoreNative) {
          v = v * sc + sh;
          if (epi.residual) v += static_cast<float>(static_cast<const _Float16 *>(epi.residual)[at]);
          if (epi.relu) v = v > 0.f ? v : 0.f;
          static_cast<_Float16 *>(Yv)[at] = static_cast<_Float16>(v);
        } else if constexpr (MODE == kStoreF32) {
          static_cast<float *>(Yv)[at] = v;
        } else if constexpr (MODE == kAddF32) {
          static_cast<float *>(Yv)[at] += v;
        } else {
          atomicAdd(static_cast<float *>(Yv) + at, v);
        }
      }
  }
}

// Storage-dtype output of a wave's 32 x BN tile through LDS: the
// accumulators (times scale, plus shift) are staged as fp16 rows, then every
// lane writes 16-byte chunks of output rows (adding the residual and
// applying ReLU), so that the output rows are written with full-width
// vector stores.  Needs Cout % 8 == 0 (16-byte aligned rows) and a staging
// area of 32 x (BN + 8) halves per wave.
template <int WN>
__device__ __forceinline__ void store_tile_vec(const floatx4 (&acc)[2][2 * WN], const int32_t *orow, int n0, int Cout,
                                               _Float16 *stage, void *Yv, const Epilogue &epi) {
  constexpr int BN = 32 * WN, BNP = BN + 8, ROWS = 32;
  const int lane = threadIdx.x & 63, l16 = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int nb = 0; nb < 2 * WN; ++nb) {
    const int col = n0 + nb * 16 + l16;
    float sc = 1.f, sh = 0.f;
    if (col < Cout) {
      if (epi.scale) sc = epi.scale[col];
      if (epi.shift) sh = epi.shift[col];
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rt * 16 + lq * 4 + i;
        stage[row * BNP + nb * 16 + l16] = static_cast<_Float16>(acc[rt][nb][i] * sc + sh);
      }
  }
  // the staging rows are private to the wave: LDS keeps its accesses in order
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  constexpr int CPR = BN / 8;  // 16-byte chunks per row
  _Float16 *Y = static_cast<_Float16 *>(Yv);
  const _Float16 *R = static_cast<const _Float16 *>(epi.residual);
  for (int q = lane; q < ROWS * CPR; q += 64) {
    const int row = q / CPR, ch = q - row * CPR;
    const int col = n0 + ch * 8;
    const int32_t o = orow[row];
    if (o < 0 || col >= Cout) continue;
    half8 v = *reinterpret_cast<const half8 *>(stage + row * BNP + ch * 8);
    const int64_t at = static_cast<int64_t>(o) * Cout + col;
    if (R || epi.relu) {
      half8 rv = {};
      if (R) rv = *reinterpret_cast<const half8 *>(R + at);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float f = static_cast<float>(v[e]) + static_cast<float>(rv[e]);
        if (epi.relu) f = f > 0.f ? f : 0.f;
        v[e] = static_cast<_Float16>(f);
      }
    }
    *reinterpret_cast<half8 *>(Y + at) = v;
  }
}


// XCD-contiguous block order: the hardware hands workgroup w (in x, y, z
// dispatch order) to XCD w % 8; remapped, the workgroups of XCD x take one
// contiguous range of the logical (row tile, column tile, split) order,
// column tiles innermost, so that the XCD's L2 serves one slab of rows (and
// the column tiles of a row tile run on one XCD, close in time).
// order >= 2: runs of c = 2^order consecutive blocks per XCD, dealt to the
// XCDs in turn.  Hardware ids [8cs, 8c(s + 1)) (round s) give each XCD c
// blocks; XCD x's k-th block of round s is logical block 8cs + cx + k.  The
// last, partial round keeps its ids.  Consecutive blocks (a row tile's
// column tiles, then neighbouring row tiles) share an L2 while every XCD
// still gets its share of each part of the grid (row-ordered maps put the
// longest blocks first, so one contiguous range per XCD is unbalanced).
__device__ __forceinline__ void xcd_block(int64_t &bx, int &by, int &bz, int order) {
  constexpr int64_t kXcds = 8;
  const int64_t X = gridDim.x, Y = gridDim.y, Z = gridDim.z, G = X * Y * Z;
  const int64_t w = blockIdx.x + X * (blockIdx.y + Y * static_cast<int64_t>(blockIdx.z));
  int64_t L;
  if (order == 1) {
    const int64_t q = G / kXcds, r = G % kXcds, x = w % kXcds, i = w / kXcds;
    L = x * q + (x < r ? x : r) + i;  // a bijection of [0, G)
  } else {
    const int64_t c = int64_t(1) << order, round = kXcds * c;
    if (w < G / round * round) {
      const int64_t x = w % kXcds, i = w / kXcds;
      L = (i / c) * round + x * c + i % c;
    } else {
      L = w;
    }
  }
  bz = static_cast<int>(L / (X * Y));
  const int64_t rem = L % (X * Y);
  bx = rem / Y;
  by = static_cast<int>(rem % Y);
}

// Output-stationary implicit GEMM.  A block owns BM = 128 logical rows
// (wave w: rows [32 w, 32 w + 32) as two 16-row MFMA tiles) and BN = 32*WN
// output channels; grid = (row blocks, column blocks, offset splits), split z
// covering offsets [z*jper, min(Kc, (z+1)*jper)), jper <= 128.  With `order`,
// logical row i is target order[i] and `map` holds the rows in logical order;
// `gmask` (2 words per 128 logical rows: the union of their valid columns)
// lets the block skip offsets none of its rows uses.
template <int WN, int MODE, bool ALIGNED, int NKS, bool CAT, int OP, int DS = 0, int DA = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DA == 2 ? 1 : ring::TileOf<WN, NKS, DS>::OCC))) void os_kernel(const int32_t *__restrict__ map,
                                                    const int32_t *__restrict__ order,
                                                    const uint64_t *__restrict__ gmask, int64_t T, int Kc, int jper,
                                                    Operands op, void *Y, Epilogue epi, int xcd_order) {
  using C = typename ring::TileOf<WN, NKS, DS>::C;
  constexpr int MT = C::BM / 128, NS = C::NS;
  __shared__ __align__(1024) char ring_lds[C::LDS];
  // map entries of a later step, per stage and packed offset (untiled maps;
  // the map tile's place)
  int32_t(*idx_lds)[256] = reinterpret_cast<int32_t(*)[256]>(ring_lds + C::RING);
  static_assert(NS * OP * 256 * 4 <= C::MAP_TILE, "index slots exceed the map tile");
  static_assert(OP == 1 || ((OP == 2 || OP == 4) && ALIGNED && !CAT && MODE == kStoreNative),
                "offset packing: plain stores");
  // output row per tile row (epilogue); 64 per wave so that during the
  // step loop a wave's dummy map fetches (tiled maps) can land here
  __shared__ int32_t orow_s[4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, kh = lane >> 5;
  int64_t bx = blockIdx.x;
  int by = blockIdx.y, bz = blockIdx.z;
  if (xcd_order) xcd_block(bx, by, bz, xcd_order);
  // work balance: block x takes work item x (row tile, part)
  const bool balance = MODE == kStoreNative && OP == 1 && epi.split.offsets > 0;
  if (balance) {
    const int total = *epi.split.total;
    const int item = epi.split.items[bx < total ? bx : 0];
    if (bx >= total) return;  // (block-uniform, before any barrier)
    bz = item & 7;
    bx = item >> 3;
  }
  const int64_t row0 = bx * C::BM;
  const int n0 = by * C::BN;
  const int j0 = balance ? 0 : bz * jper;
  const int jn = ((j0 + jper) < Kc ? (j0 + jper) : Kc) - j0;
  // offsets [j0, j0 + jn) used by some row of the block, relative to j0
  uint64_t ulo = jn >= 64 ? ~uint64_t(0) : (uint64_t(1) << jn) - 1;
  uint64_t uhi = jn >= 128 ? ~uint64_t(0) : (jn > 64 ? (uint64_t(1) << (jn - 64)) - 1 : 0);
  if (gmask) {
    uint64_t glo = 0, ghi = 0;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int64_t g = row0 / 128 + m;
      if (g * 128 < T) {
        glo |= gmask[g * 2];
        ghi |= gmask[g * 2 + 1];
      }
    }
    // shift the 128-bit union right by j0 (0 <= j0 < 128)
    const uint64_t slo = j0 == 0 ? glo : (j0 < 64 ? (glo >> j0) | (ghi << (64 - j0)) : ghi >> (j0 - 64));
    const uint64_t shi = j0 == 0 ? ghi : (j0 < 64 ? ghi >> j0 : 0);
    ulo &= slo;
    uhi &= shi;
  }
  int nact = __builtin_popcountll(ulo) + __builtin_popcountll(uhi);
  const int nch = (op.CinP + C::KC - 1) / C::KC;
  // work balance: this block is part bz of its tile's nparts
  int nparts = 1;
  if (balance) {
    // (split_items_kernel counted the same parts from the same mask)
    nparts = split_parts(ulo, uhi, Kc, epi.split.offsets, epi.split.zmax);
    if (nparts > 1) {
      // keep the valid offsets of rank [a0, a1)
      const int a0 = nact * bz / nparts, a1 = nact * (bz + 1) / nparts;
      uint64_t lo = ulo, hi = uhi, klo = 0, khi = 0;
      for (int rk = 0; rk < a1; ++rk) {
        const bool inlo = lo != 0;
        const int j = inlo ? __builtin_ctzll(lo) : __builtin_ctzll(hi);
        if (rk >= a0) {
          if (inlo) klo |= uint64_t(1) << j;
          else khi |= uint64_t(1) << j;
        }
        if (inlo) lo &= lo - 1;
        else hi &= hi - 1;
      }
      ulo = klo;
      uhi = khi;
      nact = a1 - a0;
    }
  }
  // OP > 1: OP offsets per step (one channel chunk each)
  const int nsteps = OP > 1 ? (nact + OP - 1) / OP : nact * nch;

  floatx4 acc[2][2 * WN];
  zero_acc<WN>(acc);
  // the lane's rows in the wave's two 16-row tiles: 32 wave + 16 rt + l % 16
  const int l16 = lane & 15;
  bool mvalid[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) mvalid[rt] = row0 + wave * 32 + rt * 16 + l16 < T;
  // Map entries.  Kernels of at most 27 offsets: the block's BM map rows are
  // copied into LDS once (row stride KP = Kc | 1 words, odd, so that the
  // per-row reads of one column are conflict-free) and every step reads its
  // column there.  Larger kernels: lane L of a wave fetches the entry of row
  // L % 32 of the wave's rows for step u into the stage's index slot, NS
  // steps ahead (lane l then reads the entries of rows l % 16 and 16 + l % 16);
  // with offset packing each fetch serves two offsets of the step, one per
  // half-wave, so a step costs OP / 2 fetch loads (measured on the 125-offset
  // layers of 16 to 64 channels: the map fetches cost as much as the gathers'
  // request slots).  Rows past T read nothing (out of range) and are masked
  // when resolved.  No map: the identity (logical row
  // i reads source i); the fetches then load nothing (out of range) but keep
  // the vmcnt arithmetic.
  const bool ident = map == nullptr;
  const bool tiled = !ident && Kc <= C::MAP_TILE_K;
  const int frow = MT == 2 ? lane : r;
  const int64_t flr = row0 + wave * 32 * MT + frow;
  const uint32_t fbase = (flr < T && !ident) ? static_cast<uint32_t>(flr * Kc + j0) * 4u : kOutOfRange;
  const __amdgpu_buffer_rsrc_t mr = make_rsrc(map, static_cast<uint32_t>(T * Kc * 4));
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t ibase = ring::lds_addr(&idx_lds[0][0]) + (wave * 64 + l16) * 4;
  using Iter = std::conditional_t<(OP > 1), ring::GroupIter<(OP > 1 ? OP : 2)>, ring::StepIter>;
  Iter fit, pit;  // fetch side (runs NS steps ahead) and issue side
  fit.init(ulo, uhi);
  pit = fit;
  int fu = 0;
  constexpr int kFetchOps = OP > 1 ? OP / 2 : 1;  // map-fetch loads per step
  const int KP = Kc | 1;
  int32_t *tile = reinterpret_cast<int32_t *>(ring_lds + C::RING);
  if (tiled) {
    // slot s = round * 256 + tid holds element (row0 + s / KP, s % KP)
    int rr = tid / KP, cc = tid - rr * KP;
    const int drow = 256 / KP, dcol = 256 - drow * KP;
    const int rounds = (C::BM * KP + 255) / 256;
    for (int i = 0; i < rounds; ++i) {
      const int64_t grow = row0 + rr;
      const uint32_t off = (cc < Kc && grow < T) ? static_cast<uint32_t>(grow * Kc + cc) * 4u : kOutOfRange;
      ring::dma4(mr, off, tile + i * 256 + uwave * 64);
      rr += drow;
      cc += dcol;
      if (cc >= KP) {
        cc -= KP;
        ++rr;
      }
    }
    ring::wait_vm<0>();
    __syncthreads();
  }
  const uint32_t tbase = ring::lds_addr(tile) + ((wave * 32 + l16) * KP + j0) * 4;
  auto fetch = [&](int u, auto St) {
    (void)u;
    // (tiled: out-of-range fetches that only keep the vmcnt arithmetic)
    const bool none = tiled || fbase == kOutOfRange || fu >= nsteps;
    if constexpr (OP == 1) {
      const uint32_t off = none ? kOutOfRange : fbase + fit.j * 4u;
      ring::dma4(mr, off, tiled ? &orow_s[uwave][0] : &idx_lds[decltype(St)::value][uwave * 64]);
    } else {
      // two offset parts per fetch: lanes 0-31 take part 2p, lanes 32-63
      // part 2p + 1 (rows lane % 32), into slots 0-31 / 32-63 of index
      // slot St * OP + 2p
      ring::unroll<OP / 2>([&](auto P) {
        constexpr int p = decltype(P)::value;
        const int ja = p == 0 ? fit.j : fit.jp[2 * p - 1];
        const int jj = kh == 0 ? ja : fit.jp[2 * p];
        const uint32_t off = (none || jj < 0) ? kOutOfRange : fbase + jj * 4u;
        ring::dma4(mr, off, tiled ? &orow_s[uwave][0] : &idx_lds[decltype(St)::value * OP + 2 * p][uwave * 64]);
      });
    }
    ++fu;
    fit.step(nch);
  };
  // Tiled maps: the indices of the next step are read from the tile right
  // after a step's are resolved, so their LDS latency hides behind the
  // following compute (whose B-read wait also covers them); only the
  // prologue's steps (no compute in between) wait for their own read.
  int32_t pre[2], prep[3][2];
  auto read_tile = [&]() {
    // (past the last offset (OP = 2: j = -1) column 0 is read, unused)
    const uint32_t col = static_cast<uint32_t>(pit.j < 0 ? 0 : pit.j) * 4u;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      asm volatile("ds_read_b32 %0, %1" : "=v"(pre[rt]) : "v"(tbase + rt * 16 * KP * 4 + col) : "memory");
    if constexpr (OP > 1) {
      // (a part past the last offset: column 0 is read and discarded when resolved)
#pragma unroll
      for (int q = 0; q < OP - 1; ++q) {
        const uint32_t colq = static_cast<uint32_t>(pit.jp[q] < 0 ? 0 : pit.jp[q]) * 4u;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          asm volatile("ds_read_b32 %0, %1" : "=v"(prep[q][rt]) : "v"(tbase + rt * 16 * KP * 4 + colq) : "memory");
      }
    }
  };
  if (tiled) read_tile();
  auto resolve = [&](int u, auto St, ring::StepIn &st) {
    int32_t(&idx)[2] = st.idx;
    if (tiled) {
      if (u < NS) ring::lds_wait();  // prologue puts: no compute since the read
      idx[0] = pre[0];
      idx[1] = pre[1];
      if constexpr (OP > 1) {
#pragma unroll
        for (int q = 0; q < OP - 1; ++q) {
          st.idxp[q][0] = prep[q][0];
          st.idxp[q][1] = prep[q][1];
        }
      }
    } else {
      // (part m of the step: index slot St * OP + 2 (m / 2), rows from
      // 32 (m % 2); tile rt's rows from 16 rt)
      idx[0] = ring::rd4<decltype(St)::value * OP * 1024>(ibase);
      idx[1] = ring::rd4<decltype(St)::value * OP * 1024 + 64>(ibase);
      if constexpr (OP > 1) {
        ring::unroll<OP - 1>([&](auto Q) {
          constexpr int m = decltype(Q)::value + 1;
          constexpr int at = (decltype(St)::value * OP + 2 * (m / 2)) * 1024 + (m % 2) * 128;
          st.idxp[m - 1][0] = ring::rd4<at>(ibase);
          st.idxp[m - 1][1] = ring::rd4<at + 64>(ibase);
        });
      }
      ring::lds_wait();
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      ring::pin(idx[rt]);
      if (ident) idx[rt] = static_cast<int32_t>(row0 + wave * 32 + rt * 16 + l16);
      if (!mvalid[rt]) idx[rt] = -1;
      if constexpr (OP > 1) {
#pragma unroll
        for (int q = 0; q < OP - 1; ++q) {
          ring::pin(st.idxp[q][rt]);
          if (!mvalid[rt]) st.idxp[q][rt] = -1;
        }
      }
    }
    st.wrow = j0 + pit.j;
    st.kb = pit.chunk * C::KC;
    if constexpr (OP > 1) {
#pragma unroll
      for (int q = 0; q < OP - 1; ++q) {
        st.livep[q] = pit.jp[q] >= 0;
        st.wrowp[q] = j0 + (pit.jp[q] < 0 ? 0 : pit.jp[q]);
      }
    }
    pit.step(nch);
    if (tiled) read_tile();
  };
  if constexpr (DA >= 1) {
    // gathered rows two steps ahead (maps held in LDS only)
    if (tiled) ring::run_da<C, ALIGNED, CAT>(acc, nsteps, resolve, op, n0, ring_lds);
    else ring::run<C, ALIGNED, CAT, kFetchOps, OP>(acc, nsteps, fetch, resolve, op, n0, ring_lds);
  } else {
    ring::run<C, ALIGNED, CAT, kFetchOps, OP>(acc, nsteps, fetch, resolve, op, n0, ring_lds);
  }
  if (balance && nparts > 1) {
    // the partial tile to the part's slot (lane layout of the accumulators:
    // row 32 wave + 16 rt + 4 (lane / 16) + i, column 16 nb + lane % 16);
    // split_finalize_kernel writes the output
    const int64_t tile = bx * static_cast<int64_t>(gridDim.y) + by;
    const int lq = lane >> 4;
    float *slot = epi.split.part + (tile * epi.split.zmax + bz) * (C::BM * C::BN);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int nb = 0; nb < 2 * WN; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          slot[(wave * 32 + rt * 16 + lq * 4 + i) * C::BN + nb * 16 + l16] = acc[rt][nb][i];
    return;
  }
  if (kh == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int64_t lr = row0 + wave * 32 * MT + m * 32 + r;
      orow_s[wave][m * 32 + r] = lr < T ? (order ? order[lr] : static_cast<int32_t>(lr)) : -1;
    }
  }
  __syncthreads();  // every wave is done with the ring: it becomes the staging area
  if constexpr (MODE == kStoreNative) {
    if (op.Cout % 8 == 0) {
      store_tile_vec<WN>(acc, orow_s[wave], n0, op.Cout,
                         reinterpret_cast<_Float16 *>(ring_lds) + wave * 32 * (C::BN + 8), Y, epi);
      return;
    }
  }
  store_tile<WN, MODE>(acc, orow_s[wave], n0, op.Cout, Y, epi);
}

// The work list of a balanced launch (TileSplit): one block of 1024
// threads, each counting the parts of a contiguous run of row tiles; a
// block-wide exclusive scan of the counts places each run's items.
__global__ __launch_bounds__(1024) void split_items_kernel(const uint64_t *__restrict__ gmask, int64_t gx, int Kc,
                                                           TileSplit ts) {
  __shared__ int wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t per = (gx + 1023) / 1024;
  const int64_t t0 = tid * per, t1 = t0 + per < gx ? t0 + per : gx;
  int cnt = 0;
  for (int64_t t = t0; t < t1; ++t) cnt += split_parts(gmask[2 * t], gmask[2 * t + 1], Kc, ts.offsets, ts.zmax);
  int incl = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int pos = incl - cnt;
  for (int q = 0; q < w; ++q) pos += wsum[q];
  if (tid == 1023) *ts.total = pos + cnt;
  for (int64_t t = t0; t < t1; ++t) {
    const int np = split_parts(gmask[2 * t], gmask[2 * t + 1], Kc, ts.offsets, ts.zmax);
    for (int p = 0; p < np; ++p) ts.items[pos++] = static_cast<int32_t>((t << 3) | p);
  }
}

// The outputs of the work-balanced tiles (TileSplit): kFinSubs blocks per
// (row tile, column tile) of BM = 128 rows x BN columns, block q taking rows
// [32 q, 32 q + 32); a tile split into z > 1 parts (split_parts of its
// group mask) sums its z partial tiles in order, re-zeroes them, and writes
// rows order[row0 + r] (or row0 + r) with the epilogue, rounded like
// store_tile_vec (scale and shift, fp16, then the residual and ReLU).
constexpr int kFinSubs = 4;
template <int BN>
__global__ __launch_bounds__(256) void split_finalize_kernel(const uint64_t *__restrict__ gmask,
                                                             const int32_t *__restrict__ order, int64_t T, int Kc,
                                                             int Cout, int gy, _Float16 *__restrict__ Y,
                                                             Epilogue epi) {
  const int64_t tile = blockIdx.x / kFinSubs;
  const int q = blockIdx.x % kFinSubs;
  const int64_t t = tile / gy;
  // (the work list back to zeros: the os_kernel launch has read it)
  if (q == 0 && tile % gy == 0 && threadIdx.x < epi.split.zmax) epi.split.items[t * epi.split.zmax + threadIdx.x] = 0;
  if (tile == 0 && q == 0 && threadIdx.x == 0) *epi.split.total = 0;
  const int z = split_parts(gmask[2 * t], gmask[2 * t + 1], Kc, epi.split.offsets, epi.split.zmax);
  if (z < 2) return;
  const int64_t row0 = t * 128;
  const int n0 = static_cast<int>(tile % gy) * BN;
  constexpr int N4 = 128 * BN / 4;         // float4 per partial tile
  constexpr int IT = N4 / kFinSubs / 256;  // per thread: 1, 2, 3 or 4
  floatx4 *__restrict__ base = reinterpret_cast<floatx4 *>(epi.split.part + tile * epi.split.zmax * (128 * BN));
  const _Float16 *R = static_cast<const _Float16 *>(epi.residual);
  // every load first (partial tiles, output rows, scale and shift), then
  // the residual rows, so that the block waits on memory twice
  floatx4 pv[IT][8], sc[IT], sh[IT];
  int64_t o[IT];
  int cbase[IT];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int e4 = (q * IT + k) * 256 + threadIdx.x;
#pragma unroll
    for (int p = 0; p < 8; ++p)
      if (p < z) pv[k][p] = base[p * N4 + e4];
    const int row = (e4 * 4) / BN;
    cbase[k] = n0 + (e4 * 4) % BN;
    const int64_t lr = row0 + row;
    o[k] = lr < T ? (order ? order[lr] : lr) : -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = cbase[k] + i < Cout ? cbase[k] + i : 0;
      sc[k][i] = epi.scale ? epi.scale[col] : 1.f;
      sh[k][i] = epi.shift ? epi.shift[col] : 0.f;
    }
  }
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int e4 = (q * IT + k) * 256 + threadIdx.x;
    floatx4 v = pv[k][0];
#pragma unroll
    for (int p = 1; p < 8; ++p)
      if (p < z) v += pv[k][p];  // parts in order 0 .. z - 1
#pragma unroll
    for (int p = 0; p < 8; ++p)
      if (p < z) base[p * N4 + e4] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (o[k] < 0) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = cbase[k] + i;
      if (col >= Cout) break;
      float f = static_cast<float>(static_cast<_Float16>(v[i] * sc[k][i] + sh[k][i]));
      if (R) f += static_cast<float>(R[o[k] * Cout + col]);
      if (epi.relu) f = f > 0.f ? f : 0.f;
      Y[o[k] * Cout + col] = static_cast<_Float16>(f);
    }
  }
}

// Fused weight-stationary pass.  Rows of the pair list are tiled per
// compacted offset row in blocks of BM pairs (the tile table is rebuilt in
// LDS from naddrs); tiles [0, nfwd) apply (in -> out) with W[woffset + r],
// with Kw > 0 tiles [nfwd, 2 nfwd) apply the mirrored pass (out -> in) with
// W[woffset + Kw-1-r] except for a self-mirrored centre row.  Results are
// atomically added to an fp32 buffer.
template <int WN, bool ALIGNED>
__global__ __launch_bounds__(256, 2) void ws_kernel(const int32_t *__restrict__ in_idx,
                                                    const int32_t *__restrict__ out_idx,
                                                    const int32_t *__restrict__ naddrs, int R, int64_t nfwd, int Kw,
                                                    int woffset, Operands op, float *__restrict__ Yacc) {
  using C = typename ring::TileOf<WN>::C;
  constexpr int MT = C::BM / 128;
  __shared__ __align__(1024) char ring_lds[C::RING];
  __shared__ int32_t tstart[kMaxGroups + 1];
  __shared__ int32_t orow_s[4][32 * MT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, kh = lane >> 5;
  // tile starts per compacted row: exclusive scan of ceil(rows / BM), R <= 128
  {
    int cnt = 0;
    if (tid < R) cnt = (naddrs[tid + 1] - naddrs[tid] + C::BM - 1) / C::BM;
    if (tid < kMaxGroups + 1) tstart[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < kMaxGroups + 1; off <<= 1) {
      const int v = (tid < kMaxGroups + 1 && tid >= off) ? tstart[tid - off] : 0;
      __syncthreads();
      if (tid < kMaxGroups + 1) tstart[tid] += v;
      __syncthreads();
    }
    const int incl = tid < kMaxGroups + 1 ? tstart[tid] : 0;
    __syncthreads();
    if (tid < kMaxGroups + 1) tstart[tid] = incl - (tid < R ? cnt : 0);
    __syncthreads();
  }
  int64_t tile = blockIdx.x;
  const bool mir = tile >= nfwd;
  if (mir) tile -= nfwd;
  int lo = 0, hi = R;  // last row with tstart[row] <= tile
  while (hi - lo > 1) {
    const int md = (lo + hi) >> 1;
    if (tstart[md] <= tile) lo = md;
    else hi = md;
  }
  const int row = lo;
  if (tile >= tstart[R] || (mir && 2 * row + 1 == Kw)) return;  // block-uniform
  const int64_t nrow = naddrs[row + 1] - naddrs[row];
  // the lane's source rows in the wave's two 16-row tiles (MFMA A layout)
  // and the destination of wave row r (epilogue)
  const int64_t base = (tile - tstart[row]) * C::BM + wave * 32;
  int32_t src[2], dst = -1;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int64_t local = base + rt * 16 + (lane & 15);
    src[rt] = local < nrow ? (mir ? out_idx[naddrs[row] + local] : in_idx[naddrs[row] + local]) : -1;
  }
  if (base + r < nrow) dst = mir ? in_idx[naddrs[row] + base + r] : out_idx[naddrs[row] + base + r];
  const int wrow0 = woffset + (mir ? Kw - 1 - row : row);
  const int n0 = blockIdx.y * C::BN;
  floatx4 acc[2][2 * WN];
  zero_acc<WN>(acc);
  auto fetch = [](int, auto) {};
  auto resolve = [&](int u, auto, ring::StepIn &st) {
    st.idx[0] = src[0];
    st.idx[1] = src[1];
    st.wrow = wrow0;
    st.kb = u * C::KC;
  };
  const int nch = (op.CinP + C::KC - 1) / C::KC;
  ring::run<C, ALIGNED, false, 0>(acc, nch, fetch, resolve, op, n0, ring_lds);
  if (kh == 0) orow_s[wave][r] = dst;
  __syncthreads();
  store_tile<WN, kAtomicF32>(acc, orow_s[wave], n0, op.Cout, Yacc, Epilogue{});
}

struct GroupTable {
  int n;                               // groups
  int64_t tile_start[kMaxGroups + 1];  // prefix of row tiles
  int64_t row_off[kMaxGroups];         // first buffer row of the group
  int32_t rows[kMaxGroups];            // valid rows of the group
};

// Grouped GEMM over the padded gather buffer: Ybuf[rows of g] = Xbuf[rows of g] @ W[g].
template <int WN, bool ALIGNED>
__global__ __launch_bounds__(256, 2) void gg_kernel(const GroupTable gt, Operands op, float *__restrict__ Yb) {
  using C = typename ring::TileOf<WN>::C;
  constexpr int MT = C::BM / 128;
  __shared__ __align__(1024) char ring_lds[C::RING];
  __shared__ int32_t orow_s[4][32 * MT];
  const int64_t tile = blockIdx.x;
  int g = 0, ghi = gt.n;  // last group with tile_start[g] <= tile
  while (ghi - g > 1) {
    const int md = (g + ghi) >> 1;
    if (gt.tile_start[md] <= tile) g = md;
    else ghi = md;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, kh = lane >> 5;
  const int64_t base = (tile - gt.tile_start[g]) * C::BM + wave * 32;
  auto row_of = [&](int64_t local) {
    return local < gt.rows[g] ? static_cast<int32_t>(gt.row_off[g] + local) : -1;
  };
  const int32_t src[2] = {row_of(base + (lane & 15)), row_of(base + 16 + (lane & 15))};
  const int n0 = blockIdx.y * C::BN;
  floatx4 acc[2][2 * WN];
  zero_acc<WN>(acc);
  auto fetch = [](int, auto) {};
  auto resolve = [&](int u, auto, ring::StepIn &st) {
    st.idx[0] = src[0];
    st.idx[1] = src[1];
    st.wrow = g;
    st.kb = u * C::KC;
  };
  const int nch = (op.CinP + C::KC - 1) / C::KC;
  ring::run<C, ALIGNED, false, 0>(acc, nch, fetch, resolve, op, n0, ring_lds);
  if (kh == 0) orow_s[wave][r] = row_of(base + r);
  __syncthreads();
  store_tile<WN, kStoreF32>(acc, orow_s[wave], n0, op.Cout, Yb, Epilogue{});
}

// ---------------------------------------------------------------------------
// // element-wise helpers
template <typename FT> __device__ __forceinline__ float ld(const FT *p) { return static_cast<float>(*p); }

// [K, Cin, Cout] -> zero-padded [K, CoutP, CinP]
__global__ void prepare_w_kernel(const _Float16 *__restrict__ W, int K, int Cin, int Cout, int CinP, int CoutP,
                                 _Float16 *__restrict__ WT) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n = static_cast<int64_t>(K) * CoutP * CinP;
  if (i >= n) return;
  const int64_t k = i / (static_cast<int64_t>(CoutP) * CinP);
  const int64_t rem = i % (static_cast<int64_t>(CoutP) * CinP);
  const int co = static_cast<int>(rem / CinP), ci = static_cast<int>(rem % CinP);
  WT[i] = (co < Cout && ci < Cin) ? W[(k * Cin + ci) * Cout + co] : static_cast<_Float16>(0.f);
}

// fp32 partial sums -> storage dtype, with the optional epilogue
template <typename FT>
__global__ void finalize_kernel(float *__restrict__ acc, int64_t T, int Cout, FT *__restrict__ Y,
                                Epilogue epi, int clear) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * Cout) return;
  const int c = static_cast<int>(i % Cout);
  float v = acc[i];
  if (clear) acc[i] = 0.f;
  if (epi.scale) v *= epi.scale[c];
  if (epi.shift) v += epi.shift[c];
  if (epi.residual) v += ld(static_cast<const FT *>(epi.residual) + i);
  if (epi.relu) v = v > 0.f ? v : 0.f;
  Y[i] = static_cast<FT>(v);
}

__global__ void fill_f32_kernel(float *__restrict__ p, int64_t n, float v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// generic (fp32 storage) kernels, fp32 accumulate
template <typename FT, int MODE>
__device__ __forceinline__ void put(void *Y, int64_t i, float v) {
  if constexpr (MODE == kStoreNative) static_cast<FT *>(Y)[i] = static_cast<FT>(v);
  else if constexpr (MODE == kStoreF32) static_cast<float *>(Y)[i] = v;
  else if constexpr (MODE == kAddF32) static_cast<float *>(Y)[i] += v;
  else atomicAdd(static_cast<float *>(Y) + i, v);
}

// Output-stationary layer in fp32 storage on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32): a block owns 64 target rows x 16 NB output
// channels, one 16-row tile per wave, and reads its 64 map rows into LDS
// once.  The K dimension is walked in steps of
// (one offset, 32 input channels).  Each lane gathers the 8 channels of its
// row that its MFMA lane group needs (channels 4 (l / 16) + i and
// 16 + 4 (l / 16) + i for the step's two 16-channel halves) straight into
// registers, one step ahead; the step's 32 x BN weight chunk is shared by the
// four waves through a double-buffered LDS tile whose row pitch (BN + 4
// floats) keeps the four lane groups on distinct banks.  A wave whose 16 rows
// have no neighbour at the step's offset skips its MFMAs.  Sums are fp32; each
// offset's partial sum is added to the total at the end of the offset, as
// the per-offset sums of the reference's fp32 kernels.
template <int NB, int MODE>
__global__ __launch_bounds__(256) void os_f32_kernel(const int32_t *__restrict__ map, int64_t T, int Kc,
                                                     const float *__restrict__ X, int Cin,
                                                     const float *__restrict__ W, int Cout, void *Y, Epilogue epi) {
  constexpr int KC = 32;                                           // input channels per step
  constexpr int BN = 16 * NB, BS = BN + 4, BPT = KC * BN / 256;  // weight floats per thread and step
  constexpr int kMapK = 128;                                       // map columns held in LDS
  __shared__ float Bs[2][KC * BS];
  __shared__ int32_t Ms[64 * kMapK];  // the block's map rows (kernels of <= 128 offsets)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, kk = lane >> 4;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int n0 = blockIdx.y * BN;
  const int64_t arow = row0 + 16 * w + l16;  // the row this lane gathers
  const bool rvalid = arow < T;
  const int nchunk = (Cin + KC - 1) / KC;
  const int nsteps = Kc * nchunk;
  const bool map_lds = map && Kc <= kMapK;
  if (map_lds) {  // one coalesced read of the block's map rows: the gathers then wait on one load, not two
    const int64_t rows = T - row0 < 64 ? T - row0 : 64;
    for (int e = tid; e < rows * Kc; e += 256) Ms[e] = map[row0 * Kc + e];
    __syncthreads();
  }
  // returns whether any row of the wave's tile has a neighbour at the step's offset
  auto load_a = [&](int step, float (&a)[8]) {
    const int k = step / nchunk, c0 = (step - k * nchunk) * KC + 4 * kk;
    int32_t src = -1;
    if (rvalid)  // (no map: the identity)
      src = map_lds ? Ms[(16 * w + l16) * Kc + k] : (map ? map[arow * Kc + k] : static_cast<int32_t>(arow));
    const bool any = __ballot(src >= 0) != 0;
    const float *x = X + static_cast<int64_t>(src) * Cin;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + 16 * h + i;
        a[4 * h + i] = (src >= 0 && c < Cin) ? x[c] : 0.f;
      }
    return any;
  };
  auto load_b = [&](int step, float (&r)[BPT]) {
    const int k = step / nchunk, c0 = (step - k * nchunk) * KC;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int e = q * 256 + tid, cr = e / BN, cn = e - cr * BN;
      const int c = c0 + cr, n = n0 + cn;
      r[q] = (c < Cin && n < Cout) ? W[(static_cast<int64_t>(k) * Cin + c) * Cout + n] : 0.f;
    }
  };
  auto store_b = [&](int buf, const float (&r)[BPT]) {
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int e = q * 256 + tid, cr = e / BN, cn = e - cr * BN;
      Bs[buf][cr * BS + cn] = r[q];
    }
  };
  floatx4 acc[NB], part[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = part[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ra[8], rbv[BPT];
  bool act = load_a(0, ra);
  load_b(0, rbv);
  store_b(0, rbv);
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const bool more = step + 1 < nsteps;
    float na[8], nbv[BPT];
    bool nact = false;
    if (more) {
      nact = load_a(step + 1, na);
      load_b(step + 1, nbv);
    }
    const float *bs = Bs[step & 1];
    // (a tile with no neighbour at this offset adds zeros: skipped)
    if (act)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          part[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[4 * h + i],
                                                          bs[(16 * h + 4 * kk + i) * BS + nb * 16 + l16], part[nb],
                                                          0, 0, 0);
    if ((step + 1) % nchunk == 0) {  // the offset's partial sum into the total
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[nb] += part[nb];
        part[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if (more) store_b((step + 1) & 1, nbv);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int i = 0; i < 8; ++i) ra[i] = na[i];
      act = nact;
    }
  }
  // lane l holds rows 4 (l / 16) + i of the wave's tile, column l % 16
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int c = n0 + nb * 16 + l16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t t = row0 + 16 * w + 4 * kk + i;
      if (t >= T || c >= Cout) continue;
      float v = acc[nb][i];
      const int64_t o = t * Cout + c;
      if constexpr (MODE == kStoreNative) {
        if (epi.scale) v *= epi.scale[c];
        if (epi.shift) v += epi.shift[c];
        if (epi.residual) v += static_cast<const float *>(epi.residual)[o];
        if (epi.relu) v = v > 0.f ? v : 0.f;
      }
      put<float, MODE>(Y, o, v);
    }
  }
}

template <typename FT>
__global__ __launch_bounds__(256) void ws_fused_generic_kernel(const int32_t *__restrict__ in_idx,
                                                               const int32_t *__restrict__ out_idx,
                                                               const int32_t *__restrict__ naddrs, int R, int Kw,
                                                               int woffset, int64_t P, const FT *__restrict__ X,
                                                               int Cin, const FT *__restrict__ W, int Cout,
                                                               float *__restrict__ Yacc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t passes = Kw > 0 ? 2 : 1;
  if (i >= passes * P * Cout) return;
  int64_t p = i / Cout;
  const int c = static_cast<int>(i % Cout);
  const bool mir = p >= P;
  if (mir) p -= P;
  int lo = 0, hi = R;
  while (hi - lo > 1) {
    const int m = (lo + hi) >> 1;
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
  for (int ci = 0; ci < Cin; ++ci) acc = fmaf(ld(x + ci), ld(w + static_cast<int64_t>(ci) * Cout), acc);
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
  for (int ci = 0; ci < Cin; ++ci) acc = fmaf(ld(x + ci), ld(w + static_cast<int64_t>(ci) * Cout), acc);
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

// scatter: Y[t] = base[t] + sum_k buf[off[k] + mask[k, t]]
template <typename FT>
__global__ __launch_bounds__(256) void scatter_kernel(const OffsetTable ot, int64_t T, int Cout,
                                                      const int32_t *__restrict__ tmask,
                                                      const float *__restrict__ buf, FT *__restrict__ Y,
                                                      const float *__restrict__ base, Epilogue epi) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * Cout) return;
  const int64_t t = i / Cout;
  const int c = static_cast<int>(i % Cout);
  float acc = base ? base[i] : 0.f;
  for (int k = 0; k < ot.n; ++k) {
    const int32_t m = tmask[k * T + t];
    if (m >= 0) acc += buf[(ot.off[k] + m) * Cout + c];
  }
  if (epi.scale) acc *= epi.scale[c];
  if (epi.shift) acc += epi.shift[c];
  if (epi.residual) acc += static_cast<float>(static_cast<const FT *>(epi.residual)[i]);
  if (epi.relu) acc = acc > 0.f ? acc : 0.f;
  Y[i] = static_cast<FT>(acc);
}

// ---------------------------------------------------------------------------
// Per-target walk for few input channels (fp16, C_in <= 16): with a large,
// sparse kernel (125 offsets, ~10 valid per target) the MMA tiles spend
// most of their steps on missing neighbours; here every target sums only
// its valid (offset, source) pairs, on the vector ALU (v_dot2_f32_f16).
//
// Block: 256 threads, a slice of 16 output columns (gridDim.y slices).  The
// slice's weights [K][16][CIN] (C_in zero-padded to CIN) sit in LDS for the
// whole block, which then walks 16-target chunks (persistent grid).  Wave w
// takes targets 4w .. 4w+3 of a chunk; the 16 lanes of a target take the
// offsets j = lane, lane + 16, ... (coalesced 64-byte map loads), sum their
// pairs into 16 fp32 column sums, and a 16-lane butterfly adds the lanes'
// sums; lane q then writes column q (with the epilogue).
// ---------------------------------------------------------------------------
constexpr int kWalkOffsetsMax = 128;
template <int CIN> struct WalkShape {
  static constexpr int ROW = 16 * CIN + 8;  // halves per offset in LDS (+16 bytes: bank spread)
  static constexpr int JPL = kWalkOffsetsMax / 16;  // offsets per lane
};

template <int CIN>
__global__ __launch_bounds__(256) void os_walk_kernel(const int32_t *__restrict__ map, int64_t T, int K,
                                                      const _Float16 *__restrict__ X, int Cin,
                                                      const _Float16 *__restrict__ W, int Cout,
                                                      _Float16 *__restrict__ Y, Epilogue epi) {
  using Sh = WalkShape<CIN>;
  __shared__ __align__(16) _Float16 wl[kWalkOffsetsMax * Sh::ROW];
  const int n0 = blockIdx.y * 16;
  // weights of the slice: wl[k][o][c] = W[k][c][n0 + o] (zero past C_in / C_out)
  for (int e = threadIdx.x; e < K * 16 * CIN; e += 256) {
    const int k = e / (16 * CIN), r = e - k * 16 * CIN, o = r / CIN, c = r - o * CIN;
    const int col = n0 + o;
    wl[k * Sh::ROW + o * CIN + c] =
        (c < Cin && col < Cout) ? W[(static_cast<int64_t>(k) * Cin + c) * Cout + col] : static_cast<_Float16>(0.f);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 15;
  const int col = n0 + q;
  float sc = 1.f, sh = 0.f;
  if (col < Cout) {
    if (epi.scale) sc = epi.scale[col];
    if (epi.shift) sh = epi.shift[col];
  }
  const int64_t nchunks = (T + 15) / 16;
  for (int64_t chunk = blockIdx.x; chunk < nchunks; chunk += gridDim.x) {
    const int64_t t = chunk * 16 + wave * 4 + (lane >> 4);
    const bool live = t < T;
    int32_t s[Sh::JPL];
#pragma unroll
    for (int i = 0; i < Sh::JPL; ++i) {
      const int j = q + 16 * i;
      s[i] = (live && j < K) ? map[t * K + j] : -1;
    }
    // every source row of the lane first (their loads overlap), then the sums
    _Float16 x[Sh::JPL][CIN];
#pragma unroll
    for (int i = 0; i < Sh::JPL; ++i) {
      const _Float16 *xr = X + static_cast<int64_t>(s[i] < 0 ? 0 : s[i]) * Cin;
      if (Cin == CIN && (CIN % 8) == 0) {
#pragma unroll
        for (int c = 0; c < CIN; c += 8) {
          half8 v = {};
          if (s[i] >= 0) v = *reinterpret_cast<const half8 *>(xr + c);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[i][c + e] = v[e];
        }
      } else {
#pragma unroll
        for (int c = 0; c < CIN; ++c) x[i][c] = (s[i] >= 0 && c < Cin) ? xr[c] : static_cast<_Float16>(0.f);
      }
    }
    float acc[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) acc[o] = 0.f;
#pragma unroll
    for (int i = 0; i < Sh::JPL; ++i) {
      if (s[i] < 0) continue;
      const _Float16 *w = wl + (q + 16 * i) * Sh::ROW;
#pragma unroll
      for (int o = 0; o < 16; ++o) {
        // the column's CIN weights: 16-byte LDS reads (8-byte ones for CIN = 4)
#pragma unroll
        for (int c0 = 0; c0 < CIN; c0 += (CIN >= 8 ? 8 : 4)) {
          _Float16 wv[8];
          if constexpr (CIN >= 8) {
            const half8 v = *reinterpret_cast<const half8 *>(w + o * CIN + c0);
#pragma unroll
            for (int e = 0; e < 8; ++e) wv[e] = v[e];
          } else {
            const half4 v = *reinterpret_cast<const half4 *>(w + o * CIN + c0);
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[e] = v[e];
          }
#pragma unroll
          for (int c = 0; c < (CIN >= 8 ? 8 : 4); c += 2) {
            const half2 a = {x[i][c0 + c], x[i][c0 + c + 1]};
            const half2 b = {wv[c], wv[c + 1]};
            acc[o] = __builtin_amdgcn_fdot2(a, b, acc[o], false);
          }
        }
      }
    }
    // add the 16 lanes' sums of every column (butterfly inside the 16-lane group)
#pragma unroll
    for (int o = 0; o < 16; ++o)
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) acc[o] += __shfl_xor(acc[o], m, 64);
    float v = 0.f;
#pragma unroll
    for (int o = 0; o < 16; ++o) v = (o == q) ? acc[o] : v;
    if (live && col < Cout) {
      v = v * sc + sh;
      const int64_t at = t * Cout + col;
      if (epi.residual) v += static_cast<float>(static_cast<const _Float16 *>(epi.residual)[at]);
      if (epi.relu) v = v > 0.f ? v : 0.f;
      Y[at] = static_cast<_Float16>(v);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static inline bool mfma_path(int dtype) { return dtype == SPIRA_F16; }
static inline int pad_in(int c) { return static_cast<int>(round_up(c, 16)); }
static inline int pad_out(int c) { return static_cast<int>(round_up(c, 32)); }

// column-tile width (x 32 columns): wider layers take several 128-column
// tiles (more, shorter blocks; a 256-column tile would halve the resident
// waves for the same work)
static inline int wn_for(int Cout) {
  if (Cout <= 32) return 1;
  if (Cout <= 64) return 2;
  if (Cout <= 96) return 3;
  return 4;
}
// rows per block of the MMA kernels for a column-tile width
static inline int bm_for(int wn) {
  switch (wn) {
    case 1: return ring::TileOf<1>::C::BM;
    case 2: return ring::TileOf<2>::C::BM;
    case 3: return ring::TileOf<3>::C::BM;
    default: return ring::TileOf<4>::C::BM;
  }
}

// offsets per split: small layers split their offsets so that the grid
// covers the chip; a split never exceeds 128 offsets (the block's 128-bit
// active-offset set).  splits > 0: that many splits, as asked.
static int choose_jper(int64_t blocks_xy, int Kc, int cus, int splits = 0) {
  int jper = Kc;
  if (splits > 0) {
    jper = static_cast<int>(div_up(Kc, std::min(splits, Kc)));
  } else if (blocks_xy < cus && Kc > 1) {
    const int64_t n = std::min<int64_t>(Kc, div_up(cus, blocks_xy));
    jper = static_cast<int>(div_up(Kc, n));
  }
  return std::min(jper, 128);
}

// Operands of the MMA core; byte sizes must fit the 31-bit buffer offsets
// (X2 / C2: the second half of a channel concatenation, or null / 0)
static int make_operands(Operands &op, const void *X, int64_t xrows, int Cin, const void *WT, int K, int Cout,
                         const void *X2 = nullptr, int C2 = 0) {
  op.Cin = Cin + C2;
  op.C1 = Cin;
  op.CinP = pad_in(op.Cin);
  op.Cout = Cout;
  op.CoutP = pad_out(Cout);
  const int64_t xb = xrows * Cin * 2, x2b = xrows * C2 * 2,
                wb = static_cast<int64_t>(K) * op.CoutP * op.CinP * 2;
  SPIRA_HIP_REQUIRE(xb < (int64_t(1) << 31) && x2b < (int64_t(1) << 31) && wb < (int64_t(1) << 31),
                    "fp16 features / weights of one layer must stay below 2 GiB");
  op.X = static_cast<const _Float16 *>(X);
  op.xbytes = static_cast<uint32_t>(xb);
  op.X2 = static_cast<const _Float16 *>(X2);
  op.x2bytes = static_cast<uint32_t>(x2b);
  op.WT = static_cast<const _Float16 *>(WT);
  op.wbytes = static_cast<uint32_t>(wb);
  return kOk;
}

// Dynamic LDS that caps a launch at `bpc` resident blocks per CU (0: no
// cap): the hardware places the blocks of a small grid unevenly, several on
// some CUs while others idle, and a row-ordered map's blocks past the first
// round are its short ones.  The kernel's static LDS is read once per kernel.
static size_t os_lds_pad(const void *fn, int bpc) {
  if (bpc <= 0) return 0;
  static std::mutex mu;
  static std::unordered_map<const void *, long> lds;
  long st;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = lds.find(fn);
    if (it == lds.end()) {
      hipFuncAttributes at;
      st = hipFuncGetAttributes(&at, fn) == hipSuccess ? static_cast<long>(at.sharedSizeBytes) : -1;
      lds.emplace(fn, st);
    } else {
      st = it->second;
    }
  }
  if (st < 0) return 0;
  constexpr long kLdsPerCu = 160 * 1024;
  const long need = kLdsPerCu / (bpc + 1) - st + 256;  // bpc + 1 blocks no longer fit
  const long room = kLdsPerCu / bpc - st - 256;        // bpc blocks still do
  return (need > 0 && need <= room) ? static_cast<size_t>(need) : 0;
}

// launch `K<WN, ...>` for the column-tile width chosen at run time
#define SPIRA_WN_SWITCH(wn, CALL) \
  switch (wn) {                   \
    case 1: CALL(1); break;       \
    case 2: CALL(2); break;       \
    case 3: CALL(3); break;       \
    default: CALL(4); break;      \
  }

template <int MODE, bool AL, int NKS, bool CAT = false, int OP = 1, int DS = 0, int DA = 0>
static void launch_os(int wn, dim3 grid, hipStream_t s, const int32_t *map, const int32_t *order,
                      const uint64_t *rowmask, int64_t T, int Kc, int jper, const Operands &op,
                      void *Y, const Epilogue &epi, int xcd = 0) {
  // (xcd: the block order in bits 0-7, the blocks-per-CU cap above them)
#define SPIRA_OS_CALL(W)                                                                                       \
  hipLaunchKernelGGL((os_kernel<W, MODE, AL, NKS, CAT, OP, DS, DA>), grid, dim3(256),                           \
                     os_lds_pad(reinterpret_cast<const void *>(&os_kernel<W, MODE, AL, NKS, CAT, OP, DS, DA>), \
                                xcd >> 8),                                                                   \
                     s, map, order, rowmask, T, Kc, jper, op, Y, epi, xcd & 0xff)
  if constexpr (DA == 2) {  // (128-column tiles only)
    SPIRA_OS_CALL(4);
  } else if constexpr ((DS == 1 && NKS == 4) || DA == 1) {  // (96- and 128-column tiles only)
    if (wn == 3) SPIRA_OS_CALL(3);
    else SPIRA_OS_CALL(4);
  } else if constexpr (DS == 1) {  // (32- and 64-column tiles only)
    if (wn == 1) SPIRA_OS_CALL(1);
    else SPIRA_OS_CALL(2);
  } else {
    SPIRA_WN_SWITCH(wn, SPIRA_OS_CALL)
  }
#undef SPIRA_OS_CALL
}

// 16-channel slices per step of the output-stationary kernel: 64-channel
// steps once the (padded) input has 64 channels or more, else 32; and
// 128-channel steps (one step per offset for 96 and 128 channels) when the
// padded input is 96 or a multiple of 128 channels (no half-empty step), and
// either the column tile is at most 96 wide or the grid has at most 1.5
// blocks per CU: the widest tile's 128-channel weight stages hold a block at
// 80 KiB of LDS, which costs more occupancy than the halved steps save on
// larger grids.  (Measured on the config-4 layers: 96 -> 96 at 200k voxels
// 52.3 -> 46.6 us, 256 -> 256 at stride 8 111.6 -> 101.7 us; 128 -> 128 at
// stride 4, 529 blocks of the widest tile, 79.7 -> 92.7 us, so it keeps
// 64-channel steps.)  A tuning's step_channels (32, 64, 128) overrides.
static int os_nks(int CinP, int wn, int64_t blocks, int cus, int step_channels) {
  if (step_channels == 32) return 2;
  if (step_channels == 64) return CinP >= 64 ? 4 : 2;
  if (step_channels == 128) return CinP >= 96 ? 8 : (CinP >= 64 ? 4 : 2);
  if ((CinP == 96 || CinP % 128 == 0) && CinP >= 96 && (wn <= 3 || 2 * blocks <= 3 * static_cast<int64_t>(cus)))
    return 8;
  return CinP >= 64 ? 4 : 2;
}

// Column-tile width of the output-stationary kernel: the widest tile, made
// narrower once (more column blocks, each re-gathering its rows) when the
// grid has fewer than SPIRA_OS_MIN_BLOCKS (default 1) blocks per CU; a grid
// still short of the CUs then splits its offsets (choose_jper).  (Measured
// on the config-4 layers: s8 128 -> 128, 134 row blocks, is fastest with
// one halving (42.9 us, 46.7 us without); s16 256 -> 256, 32 row blocks,
// took 53.0 us narrowed down to 32-column tiles against 34.8 us without,
// as every narrowing multiplies the gathered rows.  More than one block per
// CU this way, or by more offset splits, costs more in re-gathered rows /
// atomics than the added occupancy returns.)
static int os_wn(int64_t num_targets, int c_out, int cus, int col_tile) {
  if (col_tile == 32 || col_tile == 64 || col_tile == 96 || col_tile == 128) return col_tile / 32;
  int wn = wn_for(c_out);
  const int64_t bx = div_up(num_targets, bm_for(1));
  if (wn > 1 && bx * div_up(pad_out(c_out), 32 * wn) < cus) wn = wn == 3 ? 1 : wn / 2;
  return wn;
}

// A third ring stage (two steps of gathers in flight instead of one) for
// 64-channel steps of 96- and 128-column tiles and for 128-channel steps of
// 32- and 64-column tiles, where the grid, at the larger block's LDS, still
// runs in one round of resident blocks.  (Also measured, kernel only: the
// stride-16 256 -> 256 layer at 64-column tiles and 128-channel steps 34.4
// -> 31.5 us, the stride-8 128 -> 128 layer 43.2 -> 38.7 us.)  (Measured on the
// config-4 layers, untuned: the stride-8 256 -> 256 transposed layer 49.2 ->
// 33.1 us, the stride-8 384 -> 256 1x1 layer 28.3 -> 22.1 us; the 529-block
// stride-4 128 -> 128 layers, two blocks per CU at 62 KiB, went 82.9 ->
// 96.2 us with the tail round, so they keep two stages.)
static bool os_deep_ring(int wn, int nks, int64_t blocks, int cus) {
  const bool wide = nks == 4 && wn >= 3, narrow = nks == 8 && wn <= 2;
  if (!wide && !narrow) return false;
  constexpr int kLdsPerCu = 160 * 1024;
  const int lds = wide ? (wn == 3 ? ring::TileOf<3, 4, 1>::C::LDS : ring::TileOf<4, 4, 1>::C::LDS)
                       : (wn == 1 ? ring::TileOf<1, 8, 1>::C::LDS : ring::TileOf<2, 8, 1>::C::LDS);
  const int waves = wide ? (wn == 3 ? ring::TileOf<3, 4, 1>::WAVES : ring::TileOf<4, 4, 1>::WAVES)
                         : ring::TileOf<2, 8, 1>::WAVES;
  const int per_cu = std::min(kLdsPerCu / lds, waves);
  return blocks <= static_cast<int64_t>(per_cu) * cus;
}

static spira_hip_os_tuning_t tuning_of(const spira_hip_os_tuning_t *t) {
  spira_hip_os_tuning_t r{};
  if (t) r = *t;
  return r;
}

static int check_tuning(const spira_hip_os_tuning_t &t) {
  SPIRA_HIP_REQUIRE(t.col_tile == 0 || t.col_tile == 32 || t.col_tile == 64 || t.col_tile == 96 || t.col_tile == 128,
                    "conv_os tuning: col_tile must be 0, 32, 64, 96 or 128");
  SPIRA_HIP_REQUIRE(t.step_channels == 0 || t.step_channels == 32 || t.step_channels == 64 ||
                        t.step_channels == 128,
                    "conv_os tuning: step_channels must be 0, 32, 64 or 128");
  SPIRA_HIP_REQUIRE(t.offset_splits >= 0 && t.offset_splits <= 128, "conv_os tuning: offset_splits must be 0..128");
  SPIRA_HIP_REQUIRE(t.offset_pack == 0 || t.offset_pack == 1 || t.offset_pack == 2 || t.offset_pack == 4,
                    "conv_os tuning: offset_pack must be 0, 1, 2 or 4");
  SPIRA_HIP_REQUIRE(t.block_order >= 0 && t.block_order <= 4, "conv_os tuning: block_order must be 0..4");
  SPIRA_HIP_REQUIRE(t.row_walk == 0 || t.row_walk == 1, "conv_os tuning: row_walk must be 0 or 1");
  SPIRA_HIP_REQUIRE(t.balance_offsets >= -1 && t.balance_offsets <= 128,
                    "conv_os tuning: balance_offsets must be -1 .. 128");
  SPIRA_HIP_REQUIRE(t.blocks_per_cu >= -1 && t.blocks_per_cu <= 8, "conv_os tuning: blocks_per_cu must be -1 .. 8");
  return kOk;
}

// The launch of one output-stationary call: column tile (wn), rows per
// block, offsets per split (jper), 16-channel slices per step (nks), kernel
// offsets per step (pack: 1, 2 or 4) and the grid.
struct OsPlan {
  int wn, bm, jper, splits, nks, pack, xcd, deep, da;
  int bal, zmax;  // work balance: offsets per part (0: off) and parts per tile at most
  int bpc;        // resident blocks per CU at most (0: no cap)
  bool aligned;
  int64_t gx, gy;
  // workspace of the work balance: the work list and its length, then the
  // partial tiles
  size_t bal_items_bytes() const { return static_cast<size_t>(gx * zmax * 4 + 4 + 255) / 256 * 256; }
  size_t bal_bytes() const {
    return bal ? bal_items_bytes() + static_cast<size_t>(gx * gy) * zmax * bm * (32 * wn) * sizeof(float) : 0;
  }
};

static OsPlan plan_os(int64_t T, int Kc, int Cin, int CinP, bool cat, int Cout, bool has_map, bool native_store,
                      const spira_hip_os_tuning_t &tn) {
  OsPlan pl{};
  const int cus = device_cu_count();
  pl.wn = os_wn(T, Cout, cus, tn.col_tile);
  pl.bm = bm_for(pl.wn);
  pl.gx = div_up(T, pl.bm);
  pl.gy = div_up(pad_out(Cout), 32 * pl.wn);
  // small layers (fewer blocks than CUs) split their offsets over grid z
  pl.jper = choose_jper(pl.gx * pl.gy, Kc, cus, tn.offset_splits);
  pl.splits = static_cast<int>(div_up(Kc, pl.jper));
  pl.aligned = Cin % 8 == 0;
  pl.xcd = tn.block_order;
  pl.nks = pl.aligned ? os_nks(CinP, pl.wn, pl.gx * pl.gy * pl.splits, cus, tn.step_channels) : 2;
  pl.pack = 1;
  // offset packing: 16- and 32-channel inputs of kernels with more than 27
  // offsets (map entries fetched per step) run four offsets per step (64-
  // or 128-channel steps) instead of a step per offset.  (Measured, kernel
  // only, 300k voxels, 125 offsets: 16 -> 16 262 -> 182 us, 32 -> 32 273 ->
  // 213 us, 32 -> 64 299 -> 256 us; with 27 offsets (map tile in LDS) it was
  // slower: 17.5 -> 18.3-20.9 us at 200k voxels.)  64-channel inputs: two
  // offsets per 128-channel step when the column tile is at most 64 wide
  // (64 -> 64 at 125 offsets 420 -> 390 us; 64 -> 128 594 -> 601 us, so
  // wider tiles keep one offset per step).  A tuning's offset_pack 1
  // switches it off, 2 packs pairs of 16- or 32-channel offsets.
  const int want = tn.offset_pack == 0 ? 4 : tn.offset_pack;
  const bool packable = native_store && has_map && !cat && pl.aligned && pl.splits == 1 && Kc > ring::kMapTileK;
  if (packable && want > 1 && (CinP == 16 || CinP == 32)) {
    pl.pack = want;
    pl.nks = want == 2 ? CinP / 8 : CinP / 4;  // KC = pack * CinP
  } else if (packable && want > 1 && CinP == 64 && pl.wn <= 2) {
    pl.pack = 2;
    pl.nks = 8;
  }
  pl.deep = pl.pack == 1 && os_deep_ring(pl.wn, pl.nks, pl.gx * pl.gy * pl.splits, cus) ? 1 : 0;
  // Gathered rows two steps ahead in registers (run_da): 64- and
  // 128-channel steps of 96- and 128-column tiles with two LDS stages, maps
  // held in LDS.  (64-channel steps: s1 96 -> 96 52.0 -> 45.2 us, s4 192 ->
  // 128 99.3 -> 87.3 us.)
  // (Measured, kernel only, config-4 maps: s4 128 -> 128 56.5 -> 50.9 us,
  // s8 256 -> 256 row-ordered 90.6 -> 78.3 us, s8 384 -> 256 138.7 ->
  // 123.6 us, s2 96 -> 96 57.4 -> 53.2 us; 64-column tiles, at 158 VGPRs,
  // went 58.8 -> 65.2 us, so they keep the plain ring.)
  pl.da = (pl.pack == 1 && !pl.deep && pl.aligned && (pl.nks == 8 || pl.nks == 4) && pl.wn >= 3 && has_map &&
           Kc <= ring::kMapTileK)
              ? 1
              : 0;
  // the one-wave-per-SIMD build where the grid is about one block per CU
  if (pl.da && pl.wn == 4 && pl.nks == 8 && pl.gx * pl.gy * pl.splits * 4 <= static_cast<int64_t>(cus) * 5) pl.da = 2;
  pl.bpc = tn.blocks_per_cu > 0 ? tn.blocks_per_cu : 0;
  // work balance: parts of at most bal offsets, up to 8 per tile
  pl.bal = 0;
  pl.zmax = 1;
  if (native_store && has_map && pl.splits == 1 && pl.pack == 1 && pl.aligned && tn.balance_offsets > 0 &&
      Kc <= 128 && pl.bm == 128) {
    const int z = static_cast<int>(std::min<int64_t>(8, div_up(Kc, tn.balance_offsets)));
    if (z > 1) {
      pl.bal = tn.balance_offsets;
      pl.zmax = z;
      pl.xcd = 0;  // (the work list sets the block order)
    }
  }
  return pl;
}

template <int MODE>
static void launch_os_any(const OsPlan &pl, dim3 grid, hipStream_t s, const int32_t *map, const int32_t *order,
                          const uint64_t *rowmask, int64_t T, int Kc, const Operands &op, void *Y,
                          const Epilogue &epi) {
  const int wn = pl.wn, jper = pl.jper, nks = pl.nks;
  const bool cat = op.X2 != nullptr;
  if constexpr (MODE == kStoreNative) {
    if (pl.pack == 4) {
      if (nks == 4) launch_os<MODE, true, 4, false, 4>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else launch_os<MODE, true, 8, false, 4>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      return;
    }
    if (pl.pack == 2) {
      if (nks == 2) launch_os<MODE, true, 2, false, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 4) launch_os<MODE, true, 4, false, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else launch_os<MODE, true, 8, false, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      return;
    }
  }
  if (!pl.aligned) launch_os<MODE, false, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (cat) {
    // channel concatenations: storage-dtype outputs (split or not)
    if constexpr (MODE == kStoreNative || MODE == kAtomicF32) {
      if (nks == 8 && pl.deep)
        launch_os<MODE, true, 8, true, 1, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 8 && pl.da == 2)
        launch_os<MODE, true, 8, true, 1, 0, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 8 && pl.da)
        launch_os<MODE, true, 8, true, 1, 0, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 8) launch_os<MODE, true, 8, true>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 4 && pl.deep)
        launch_os<MODE, true, 4, true, 1, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 4 && pl.da)
        launch_os<MODE, true, 4, true, 1, 0, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else if (nks == 4) launch_os<MODE, true, 4, true>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
      else launch_os<MODE, true, 2, true>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
    }
  } else if (nks == 8 && pl.deep)
    launch_os<MODE, true, 8, false, 1, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 8 && pl.da == 2)
    launch_os<MODE, true, 8, false, 1, 0, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 8 && pl.da)
    launch_os<MODE, true, 8, false, 1, 0, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 8) launch_os<MODE, true, 8>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 4 && pl.deep)
    launch_os<MODE, true, 4, false, 1, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 4 && pl.da)
    launch_os<MODE, true, 4, false, 1, 0, 1>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else if (nks == 4) launch_os<MODE, true, 4>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
  else launch_os<MODE, true, 2>(wn, grid, s, map, order, rowmask, T, Kc, jper, op, Y, epi, pl.xcd | (pl.bpc << 8));
}

template <bool AL>
static void launch_ws(int wn, dim3 grid, hipStream_t s, const int32_t *in_idx, const int32_t *out_idx,
                      const int32_t *naddrs, int R, int64_t nfwd, int Kw, int woffset, const Operands &op,
                      float *Yacc) {
#define SPIRA_WS_CALL(W)                                                                                       \
  hipLaunchKernelGGL((ws_kernel<W, AL>), grid, dim3(256), 0, s, in_idx, out_idx, naddrs, R, nfwd, \
                     Kw, woffset, op, Yacc)
  SPIRA_WN_SWITCH(wn, SPIRA_WS_CALL)
#undef SPIRA_WS_CALL
}

template <bool AL>
static void launch_gg(int wn, dim3 grid, hipStream_t s, const GroupTable &gt, const Operands &op, float *Yb) {
#define SPIRA_GG_CALL(W) \
  hipLaunchKernelGGL((gg_kernel<W, AL>), grid, dim3(256), 0, s, gt, op, Yb)
  SPIRA_WN_SWITCH(wn, SPIRA_GG_CALL)
#undef SPIRA_GG_CALL
}

template <int MODE>
static void launch_os_f32(hipStream_t s, const int32_t *map, int64_t T, int Kc, const void *X, int Cin,
                          const void *W, int Cout, void *Y, const Epilogue &epi) {
  if (T == 0 || Cout == 0) return;
  const bool wide = Cout > 32;
  const dim3 grid(static_cast<unsigned>(div_up(T, 64)), static_cast<unsigned>(div_up(Cout, wide ? 64 : 32)));
  if (wide)
    hipLaunchKernelGGL((os_f32_kernel<4, MODE>), grid, dim3(256), 0, s, map, T, Kc, static_cast<const float *>(X),
                       Cin, static_cast<const float *>(W), Cout, Y, epi);
  else
    hipLaunchKernelGGL((os_f32_kernel<2, MODE>), grid, dim3(256), 0, s, map, T, Kc, static_cast<const float *>(X),
                       Cin, static_cast<const float *>(W), Cout, Y, epi);
}

static int fill_groups(GroupTable &gt, int K, const int32_t *rows, const int64_t *row_off, int bm) {
  SPIRA_HIP_REQUIRE(K <= kMaxGroups, "at most 128 kernel offsets are supported");
  gt.n = K;
  gt.tile_start[0] = 0;
  for (int k = 0; k < K; ++k) {
    gt.rows[k] = rows[k];
    gt.row_off[k] = row_off[k];
    gt.tile_start[k + 1] = gt.tile_start[k] + div_up(rows[k], bm);
  }
  return kOk;
}

static int fill_f32(float *p, int64_t n, float v, hipStream_t s) {
  if (n <= 0) return kOk;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, p, n, v);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

static Epilogue make_epi(const float *scale, const float *shift, const void *residual, int relu) {
  Epilogue e{};
  e.scale = scale;
  e.shift = shift;
  e.residual = residual;
  e.relu = relu;
  return e;
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {


int spira_hip_prepared_weights_bytes(int num_offsets, int c_in, int c_out, int dtype, size_t *bytes) {
  *bytes = mfma_path(dtype) ? static_cast<size_t>(num_offsets) * pad_in(c_in) * pad_out(c_out) * sizeof(_Float16) : 0;
  return kOk;
}

int spira_hip_prepare_weights(const void *weights, int num_offsets, int c_in, int c_out, int dtype, void *prepared,
                              hipStream_t stream) {
  if (!mfma_path(dtype)) return kOk;
  const int CinP = pad_in(c_in), CoutP = pad_out(c_out);
  const int64_t n = static_cast<int64_t>(num_offsets) * CinP * CoutP;
  if (n == 0) return kOk;
  hipLaunchKernelGGL(prepare_w_kernel, dim3(div_up(n, 256)), dim3(256), 0, stream,
                     static_cast<const _Float16 *>(weights), num_offsets, c_in, c_out, CinP, CoutP,
                     static_cast<_Float16 *>(prepared));
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_conv_os_workspace(int64_t num_targets, int num_offsets, int c_in, int c_out, int dtype, int out_mode,
                                const spira_hip_os_tuning_t *tuning, size_t *bytes) {
  (void)c_in;
  *bytes = 0;
  const spira_hip_os_tuning_t tn = tuning_of(tuning);
  if (int rc = check_tuning(tn)) return rc;
  if (!mfma_path(dtype) || out_mode != SPIRA_OUT_STORE || num_targets <= 0) return kOk;
  const OsPlan pl = plan_os(num_targets, num_offsets, c_in, pad_in(c_in), false, c_out, true, true, tn);
  if (pl.splits > 1)
    *bytes = static_cast<size_t>(num_targets) * c_out * sizeof(float);
  *bytes = std::max(*bytes, pl.bal_bytes());
  return kOk;
}

int spira_hip_conv_os_plan(int64_t num_targets, int num_offsets, int c_in, int c_in2, int c_out, int has_map,
                           int out_mode, const spira_hip_os_tuning_t *tuning, int32_t *plan) {
  const spira_hip_os_tuning_t tn = tuning_of(tuning);
  if (int rc = check_tuning(tn)) return rc;
  SPIRA_HIP_REQUIRE(plan != nullptr && num_targets > 0 && num_offsets > 0 && c_in > 0 && c_out > 0,
                    "conv_os_plan: empty layer or no output array");
  const int cin_all = c_in + c_in2;
  const OsPlan pl = plan_os(num_targets, num_offsets, cin_all, pad_in(cin_all), c_in2 > 0, c_out, has_map != 0,
                            out_mode == SPIRA_OUT_STORE, tn);
  plan[0] = pl.wn * 32;
  plan[1] = pl.nks * 16;
  plan[2] = pl.splits;
  plan[3] = pl.pack;
  plan[4] = static_cast<int32_t>(pl.gx);
  plan[5] = static_cast<int32_t>(pl.gy);
  plan[6] = pl.xcd;
  return kOk;
}

}  // extern "C"

// conv_os over sources (c_in channels) or over the channel concatenation
// [sources | sources2] (c_in + c_in2 channels; fp16, c_in % 32 == 0,
// c_in2 % 8 == 0)
static int conv_os_impl(int64_t num_targets, int num_offsets, const int32_t *out_in_map, const int32_t *row_order,
                        const uint64_t *group_masks, const void *sources, const void *sources2, int64_t num_sources,
                        int c_in, int c_in2, const void *weights, const void *prepared, int c_out, int dtype,
                        void *targets, int out_mode, const float *scale, const float *shift, const void *residual,
                        int relu, const spira_hip_os_tuning_t *tuning, void *workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  SPIRA_HIP_REQUIRE(dtype == SPIRA_F16 || dtype == SPIRA_F32, "conv_os: dtype must be fp16 or fp32");
  const spira_hip_os_tuning_t tn = tuning_of(tuning);
  if (int rc = check_tuning(tn)) return rc;
  SPIRA_HIP_REQUIRE(c_in2 == 0 || (sources2 && dtype == SPIRA_F16 && c_in % 32 == 0 && c_in2 % 8 == 0),
                    "conv_os_concat: fp16 only, the first part's channels a multiple of 32, the second's of 8");
  SPIRA_HIP_REQUIRE(out_mode >= SPIRA_OUT_STORE && out_mode <= SPIRA_OUT_ADD_F32, "conv_os: bad out_mode");
  SPIRA_HIP_REQUIRE(c_in2 == 0 || out_mode == SPIRA_OUT_STORE, "conv_os_concat: storage-dtype outputs only");
  SPIRA_HIP_REQUIRE(c_in > 0 && c_out > 0 && num_offsets > 0, "conv_os: empty channel / offset dimension");
  SPIRA_HIP_REQUIRE(out_mode == SPIRA_OUT_STORE || (!scale && !shift && !residual && !relu),
                    "conv_os: the epilogue applies to the storage-dtype output only");
  SPIRA_HIP_REQUIRE(group_masks == nullptr || num_offsets <= 128, "conv_os: group masks need <= 128 offsets");
  SPIRA_HIP_REQUIRE(out_in_map != nullptr || (num_offsets == 1 && num_sources == num_targets && !row_order),
                    "conv_os: without a map (identity) there must be one offset and as many sources as targets");
  if (num_targets <= 0) return kOk;
  const Epilogue epi = make_epi(scale, shift, residual, relu);
  if (tn.row_walk == 1 && dtype == SPIRA_F16 && c_in2 == 0 && c_in <= 16 && out_mode == SPIRA_OUT_STORE &&
      out_in_map != nullptr && row_order == nullptr && num_offsets <= kWalkOffsetsMax) {
    SPIRA_HIP_REQUIRE(weights != nullptr, "conv_os: the row walk reads the weights [K, c_in, c_out]");
    SPIRA_HIP_REQUIRE(num_targets * num_offsets < (int64_t(1) << 31), "conv_os: kernel map above 2 GiB");
    const int64_t nchunks = div_up(num_targets, 16);
    const dim3 grid(static_cast<unsigned>(nchunks < 1024 ? nchunks : 1024), static_cast<unsigned>(div_up(c_out, 16)));
    const auto *X = static_cast<const _Float16 *>(sources);
    const auto *W = static_cast<const _Float16 *>(weights);
    auto *Y = static_cast<_Float16 *>(targets);
    if (c_in <= 4)
      hipLaunchKernelGGL(os_walk_kernel<4>, grid, dim3(256), 0, stream, out_in_map, num_targets, num_offsets, X, c_in,
                         W, c_out, Y, epi);
    else if (c_in <= 8)
      hipLaunchKernelGGL(os_walk_kernel<8>, grid, dim3(256), 0, stream, out_in_map, num_targets, num_offsets, X, c_in,
                         W, c_out, Y, epi);
    else
      hipLaunchKernelGGL(os_walk_kernel<16>, grid, dim3(256), 0, stream, out_in_map, num_targets, num_offsets, X,
                         c_in, W, c_out, Y, epi);
    SPIRA_HIP_LAUNCH_CHECK();
    return kOk;
  }
  if (mfma_path(dtype)) {
    SPIRA_HIP_REQUIRE(prepared != nullptr, "conv_os: fp16 needs prepared weights (spira_hip_prepare_weights)");
    const int cin_all = c_in + c_in2;
    OsPlan pl = plan_os(num_targets, num_offsets, cin_all, pad_in(cin_all), c_in2 > 0, c_out,
                        out_in_map != nullptr, out_mode == SPIRA_OUT_STORE, tn);
    // (the one-wave-per-SIMD build only for row-ordered maps: their longest
    // tiles come first, so blocks past the first round are short ones)
    if (pl.da == 2 && !group_masks) pl.da = 1;
    // blocks per CU: for row-ordered maps (longest blocks first), as many as
    // fill every CU in the first round, so that no CU runs two long blocks
    // while another idles.  (Measured, kernel only, row-ordered config-4
    // layers: s8 128 -> 128 40.1 -> 32.4 us and s8 256 -> 256 at 96-column
    // tiles 101.8 -> 82.2 us at one block per CU; the 529-block s4 128 -> 128
    // 58.2 -> 53.2 us and s4 192 -> 128 89.4 -> 77.4 us at two.  Index-order
    // grids, whose blocks are all alike, keep no cap: s8 256 -> 256 went
    // 84.8 -> 93.9 us at one.)
    if (tn.blocks_per_cu == 0 && group_masks) {
      const int64_t blocks = pl.gx * pl.gy * pl.splits;
      const int cus = device_cu_count();
      pl.bpc = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(8, blocks / cus)));
    }
    const int jper = pl.jper;
    const int splits = pl.splits;
    dim3 grid(static_cast<unsigned>(pl.gx), static_cast<unsigned>(pl.gy), static_cast<unsigned>(splits));
    SPIRA_HIP_REQUIRE(num_targets * num_offsets * 4 < (int64_t(1) << 31), "conv_os: kernel map above 2 GiB");
    // (out_in_map may be null: the identity map, handled in the kernel)
    Operands op;
    int rc0 = make_operands(op, sources, num_sources, c_in, prepared, num_offsets, c_out, sources2, c_in2);
    if (rc0) return rc0;
    if (splits == 1) {
      if (out_mode == SPIRA_OUT_STORE && pl.bal && group_masks) {
        SPIRA_HIP_REQUIRE(workspace && workspace_bytes >= pl.bal_bytes(),
                          "conv_os: workspace too small (spira_hip_conv_os_workspace)");
        Epilogue eb = epi;
        char *w = static_cast<char *>(workspace);
        eb.split.offsets = pl.bal;
        eb.split.zmax = pl.zmax;
        eb.split.items = reinterpret_cast<int32_t *>(w);
        eb.split.total = eb.split.items + pl.gx * pl.zmax;
        eb.split.part = reinterpret_cast<float *>(w + pl.bal_items_bytes());
        hipLaunchKernelGGL(split_items_kernel, dim3(1), dim3(1024), 0, stream, group_masks, pl.gx, num_offsets,
                           eb.split);
        SPIRA_HIP_LAUNCH_CHECK();
        grid.x = static_cast<unsigned>(pl.gx * pl.zmax);
        launch_os_any<kStoreNative>(pl, grid, stream, out_in_map, row_order, group_masks, num_targets, num_offsets, op,
                                    targets, eb);
        SPIRA_HIP_LAUNCH_CHECK();
        const dim3 fg(static_cast<unsigned>(pl.gx * pl.gy * kFinSubs));
        auto *Yh = static_cast<_Float16 *>(targets);
        const int gy = static_cast<int>(pl.gy);
#define SPIRA_FIN_CALL(W)                                                                                       \
  hipLaunchKernelGGL(split_finalize_kernel<32 * W>, fg, dim3(256), 0, stream, group_masks, row_order, num_targets, \
                     num_offsets, c_out, gy, Yh, eb)
        SPIRA_WN_SWITCH(pl.wn, SPIRA_FIN_CALL)
#undef SPIRA_FIN_CALL

      } else if (out_mode == SPIRA_OUT_STORE)
        launch_os_any<kStoreNative>(pl, grid, stream, out_in_map, row_order, group_masks, num_targets, num_offsets, op, targets, epi);
      else if (out_mode == SPIRA_OUT_STORE_F32)
        launch_os_any<kStoreF32>(pl, grid, stream, out_in_map, row_order, group_masks, num_targets, num_offsets, op, targets, epi);
      else
        launch_os_any<kAddF32>(pl, grid, stream, out_in_map, row_order, group_masks, num_targets, num_offsets, op, targets, epi);
    } else {
      float *acc = nullptr;
      if (out_mode == SPIRA_OUT_STORE) {
        SPIRA_HIP_REQUIRE(workspace && workspace_bytes >= static_cast<size_t>(num_targets) * c_out * sizeof(float),
                          "conv_os: workspace too small (spira_hip_conv_os_workspace)");
        acc = static_cast<float *>(workspace);
      } else {
        acc = static_cast<float *>(targets);
      }
      // (the workspace arrives zeroed and the finalize pass clears it again)
      if (out_mode == SPIRA_OUT_STORE_F32) {
        int rc = fill_f32(acc, num_targets * c_out, 0.f, stream);
        if (rc) return rc;
      }
      launch_os_any<kAtomicF32>(pl, grid, stream, out_in_map, row_order, group_masks, num_targets, num_offsets, op, acc, epi);
      SPIRA_HIP_LAUNCH_CHECK();
      if (out_mode == SPIRA_OUT_STORE)
        hipLaunchKernelGGL(finalize_kernel<_Float16>, dim3(div_up(num_targets * c_out, 256)), dim3(256), 0, stream,
                           acc, num_targets, c_out, static_cast<_Float16 *>(targets), epi, 1);
    }
  } else {
    SPIRA_HIP_REQUIRE(num_targets * num_offsets < (int64_t(1) << 31) &&
                          num_sources * static_cast<int64_t>(c_in) < (int64_t(1) << 31),
                      "conv_os: fp32 operands above 2^31 elements");
    if (out_mode == SPIRA_OUT_STORE)
      launch_os_f32<kStoreNative>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights, c_out,
                                  targets, epi);
    else if (out_mode == SPIRA_OUT_STORE_F32)
      launch_os_f32<kStoreF32>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights, c_out, targets,
                               epi);
    else
      launch_os_f32<kAddF32>(stream, out_in_map, num_targets, num_offsets, sources, c_in, weights, c_out, targets,
                             epi);
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

extern "C" {

int spira_hip_conv_os(int64_t num_targets, int num_offsets, const int32_t *out_in_map, const int32_t *row_order,
                      const uint64_t *group_masks, const void *sources,
                      int64_t num_sources, int c_in, const void *weights, const void *prepared, int c_out, int dtype,
                      void *targets, int out_mode, const float *scale, const float *shift, const void *residual,
                      int relu, const spira_hip_os_tuning_t *tuning, void *workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  return conv_os_impl(num_targets, num_offsets, out_in_map, row_order, group_masks, sources, nullptr, num_sources,
                      c_in, 0, weights, prepared, c_out, dtype, targets, out_mode, scale, shift, residual, relu,
                      tuning, workspace, workspace_bytes, stream);
}

int spira_hip_conv_os_concat(int64_t num_targets, int num_offsets, const int32_t *out_in_map,
                             const int32_t *row_order, const uint64_t *group_masks, const void *sources,
                             const void *sources2, int64_t num_sources, int c_in, int c_in2, const void *prepared,
                             int c_out, void *targets, int out_mode, const float *scale, const float *shift,
                             const void *residual, int relu, const spira_hip_os_tuning_t *tuning, void *workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(sources2 != nullptr && c_in2 > 0, "conv_os_concat: needs a second source part");
  return conv_os_impl(num_targets, num_offsets, out_in_map, row_order, group_masks, sources, sources2, num_sources,
                      c_in, c_in2, nullptr, prepared, c_out, SPIRA_F16, targets, out_mode, scale, shift, residual,
                      relu, tuning, workspace, workspace_bytes, stream);
}

int spira_hip_conv_ws_fused(int64_t num_sources, int64_t num_targets, const int32_t *in_idx, const int32_t *out_idx,
                            int rows, const int32_t *naddrs, const int32_t *qnaddrs, int64_t num_pairs,
                            int64_t quantized_pairs, int weight_offset, int mirror_rows, const void *sources,
                            int c_in, const void *weights, const void *prepared, int num_weights, int c_out,
                            int dtype, float *target_acc, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(dtype == SPIRA_F16 || dtype == SPIRA_F32, "conv_ws_fused: dtype must be fp16 or fp32");
  SPIRA_HIP_REQUIRE(rows >= 1 || num_pairs == 0, "conv_ws_fused: rows must be positive");
  SPIRA_HIP_REQUIRE(weight_offset + std::max(mirror_rows, rows) <= num_weights,
                    "conv_ws_fused: weight rows out of range");
  if (num_pairs <= 0) return kOk;
  const int Kw = mirror_rows;
  if (mfma_path(dtype)) {
    SPIRA_HIP_REQUIRE(prepared != nullptr, "conv_ws_fused: fp16 needs prepared weights");
    SPIRA_HIP_REQUIRE(rows <= kMaxGroups, "conv_ws_fused: at most 128 offset rows");
    const int CinP = pad_in(c_in), CoutP = pad_out(c_out);
    const int wn = wn_for(c_out);
    const int bm = bm_for(wn);
    // tiles: sum over rows of ceil(rows_r / bm) <= num_pairs / bm + rows
    const int64_t nfwd = div_up(num_pairs, bm) + rows;
    (void)quantized_pairs;
    dim3 grid(static_cast<unsigned>(Kw > 0 ? 2 * nfwd : nfwd), static_cast<unsigned>(div_up(CoutP, 32 * wn)));
    Operands op;
    // the mirrored pass gathers target rows, so the feature rows cover both
    int rc0 = make_operands(op, sources, std::max(num_sources, Kw > 0 ? num_targets : int64_t(0)), c_in, prepared,
                            num_weights, c_out);
    if (rc0) return rc0;
    if (c_in % 8 == 0)
      launch_ws<true>(wn, grid, stream, in_idx, out_idx, naddrs, rows, nfwd, Kw, weight_offset, op, target_acc);
    else
      launch_ws<false>(wn, grid, stream, in_idx, out_idx, naddrs, rows, nfwd, Kw, weight_offset, op, target_acc);
  } else {
    const int64_t n = (Kw > 0 ? 2 : 1) * num_pairs * c_out;
    hipLaunchKernelGGL(ws_fused_generic_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, in_idx, out_idx,
                       naddrs, rows, Kw, weight_offset, num_pairs, static_cast<const float *>(sources), c_in,
                       static_cast<const float *>(weights), c_out, target_acc);
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
                      int dtype, const void *buffer_in, const void *weights, const void *prepared, float *buffer_out,
                      hipStream_t stream) {
  GroupTable gt{};
  const int bm = bm_for(wn_for(c_out));
  int rc = fill_groups(gt, num_offsets, rows, padded_offsets, bm);
  if (rc) return rc;
  if (num_offsets <= 0) return kOk;
  if (mfma_path(dtype)) {
    SPIRA_HIP_REQUIRE(prepared != nullptr, "ws_gemm: fp16 needs prepared weights");
    const int64_t tiles = gt.tile_start[num_offsets];
    if (tiles == 0) return kOk;
    const int CinP = pad_in(c_in), CoutP = pad_out(c_out);
    const int wn = wn_for(c_out);
    dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(div_up(CoutP, 32 * wn)));
    int64_t total = 0;
    for (int k = 0; k < num_offsets; ++k) total = std::max<int64_t>(total, padded_offsets[k] + rows[k]);
    Operands op;
    int rc0 = make_operands(op, buffer_in, total, c_in, prepared, num_offsets, c_out);
    if (rc0) return rc0;
    if (c_in % 8 == 0) launch_gg<true>(wn, grid, stream, gt, op, buffer_out);
    else launch_gg<false>(wn, grid, stream, gt, op, buffer_out);
  } else {
    int64_t total = 0;
    for (int k = 0; k < num_offsets; ++k) total = std::max<int64_t>(total, padded_offsets[k] + rows[k]);
    const int64_t n = total * c_out;
    if (n == 0) return kOk;
    hipLaunchKernelGGL(group_gemm_generic_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, gt, total,
                       static_cast<const float *>(buffer_in), c_in, static_cast<const float *>(weights), c_out,
                       buffer_out);
  }
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_ws_scatter(int64_t num_targets, int c_out, int num_offsets, int dtype, const int32_t *target_masks,
                         const int64_t *padded_offsets, const float *buffer, const float *base, const float *scale,
                         const float *shift, const void *residual, int relu, void *targets, hipStream_t stream) {
  const Epilogue epi = make_epi(scale, shift, residual, relu);
  SPIRA_HIP_REQUIRE(num_offsets <= kMaxGroups, "ws_scatter: at most 128 offsets");
  if (num_targets <= 0) return kOk;
  OffsetTable ot{};
  ot.n = num_offsets;
  for (int k = 0; k < num_offsets; ++k) ot.off[k] = padded_offsets[k];
  const int64_t n = num_targets * c_out;
  if (dtype == SPIRA_F16)
    hipLaunchKernelGGL(scatter_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_targets, c_out,
                       target_masks, buffer, static_cast<_Float16 *>(targets), base, epi);
  else
    hipLaunchKernelGGL(scatter_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, ot, num_targets, c_out,
                       target_masks, buffer, static_cast<float *>(targets), base, epi);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_finalize(const float *acc, int64_t num_targets, int c_out, int dtype, const float *scale,
                       const float *shift, const void *residual, int relu, void *targets, hipStream_t stream) {
  const int64_t n = num_targets * c_out;
  if (n <= 0) return kOk;
  const Epilogue epi = make_epi(scale, shift, residual, relu);
  if (dtype == SPIRA_F16)
    hipLaunchKernelGGL(finalize_kernel<_Float16>, dim3(div_up(n, 256)), dim3(256), 0, stream,
                       const_cast<float *>(acc), num_targets, c_out, static_cast<_Float16 *>(targets), epi, 0);
  else
    hipLaunchKernelGGL(finalize_kernel<float>, dim3(div_up(n, 256)), dim3(256), 0, stream, const_cast<float *>(acc),
                       num_targets, c_out, static_cast<float *>(targets), epi, 0);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

}  // extern "C"
