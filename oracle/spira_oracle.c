/*
 * spira_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C (OpenMP) restatement of the reference Spira algorithms on the
 * kernel-map / sparse-convolution path.  It is the parity checker for the HIP
 * library (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg) and
 * must never be linked into, imported by or called from the product path.
 *
 * All keys are carried in uint64_t containers; `bits` (32 or 64) selects the
 * reference's packing layout and the modulus of the key arithmetic.
 *
 * Reference files restated (paths under source/csrc/spira/ unless noted):
 *   compress_layout.h:11-44            packing layouts (x12/y12/z8, x24/y24/z16)
 *   cuda/kernels/compress.cuh:9-46     Compress / UnCompress
 *   torch/cuda_arg_sort_coordinates.cu:86-98   downsample mask
 *   torch/cuda_sparse_convolution_mapping.cu:10-50, 114-157, 159-209
 *                                      offset tables and the L1 permutation
 *   cuda/kernels/query_sorted.cuh:8-201, cuda/device/binary_search.cuh:10-21
 *                                      lower-bound search + kz z-scan, layouts
 *   cuda/functions/query_sorted_index.cu:146-209, 424-495, 703-776, 843-908
 *                                      pair compaction / nbsizes / masks
 *   cuda/kernels/quantifier_wstat.cuh:8-66      (quantised) exclusive scans
 *   cuda/kernels/generate_masks_from_kernel_map.cuh:10-62  masks (+ mirror)
 *   cuda/kernels/convert_transposed_os.cuh:7-16 transposed OS map inverse
 *   cuda/functions/sparse_convolution.cu:488-515, 744-764  padding buckets
 *
 * Parity pins (tests/test_oracle.py): every function here is checked against
 * an independent formulation -- numpy closed forms for packing/masks/sorting,
 * brute-force dense-grid neighbour lookup for the search, set-based
 * recomputation for compaction and masks, inverse-permutation identities for
 * the transposed map and a float64 einsum for the feature sums.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

typedef struct { int xs, ys; uint64_t xones, yones, zones, modmask; } layout_t;

/* compress_layout.h:11-44 */
static layout_t layout_of(int bits) {
  layout_t L;
  if (bits == 32) {
    L.xs = 20; L.ys = 8; L.xones = 0xFFFu; L.yones = 0xFFFu; L.zones = 0xFFu;
    L.modmask = 0xFFFFFFFFull;
  } else {
    L.xs = 40; L.ys = 16; L.xones = 0xFFFFFFull; L.yones = 0xFFFFFFull;
    L.zones = 0xFFFFull; L.modmask = ~0ull;
  }
  return L;
}

int orc_threads(void) { return omp_get_max_threads(); }

/* compress.cuh:9-23: ux = (CT)int32, key = ux<<X | uy<<Y | uz (mod 2^bits). */
void orc_pack(const int32_t *coords, int64_t n, int bits, uint64_t *keys) {
  layout_t L = layout_of(bits);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t ux = (uint64_t)(int64_t)coords[3 * i + 0] & L.modmask;
    uint64_t uy = (uint64_t)(int64_t)coords[3 * i + 1] & L.modmask;
    uint64_t uz = (uint64_t)(int64_t)coords[3 * i + 2] & L.modmask;
    keys[i] = ((ux << L.xs) | (uy << L.ys) | uz) & L.modmask;
  }
}

/* compress.cuh:28-46 */
void orc_unpack(const uint64_t *keys, int64_t n, int bits, int32_t *coords) {
  layout_t L = layout_of(bits);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t k = keys[i];
    coords[3 * i + 0] = (int32_t)((k >> L.xs) & L.xones);
    coords[3 * i + 1] = (int32_t)((k >> L.ys) & L.yones);
    coords[3 * i + 2] = (int32_t)(k & L.zones);
  }
}

/* cuda_arg_sort_coordinates.cu:86-89: per-axis mask clearing the low bits of
 * (stride-1); identical to flooring each coordinate to the stride for powers
 * of two. */
uint64_t orc_downsample_mask(int bits, int sx, int sy, int sz) {
  layout_t L = layout_of(bits);
  uint64_t xm = L.xones & ~((uint64_t)(uint32_t)(sx - 1));
  uint64_t ym = L.yones & ~((uint64_t)(uint32_t)(sy - 1));
  uint64_t zm = L.zones & ~((uint64_t)(uint32_t)(sz - 1));
  if (bits == 32) { xm &= 0xFFFFFFFFull; ym &= 0xFFFFFFFFull; zm &= 0xFFFFFFFFull; }
  return ((xm << L.xs) | (ym << L.ys) | zm) & L.modmask;
}

static int64_t kmin_of(int k) { return (k % 2 == 1) ? -(k / 2) : -(k / 2) + 1; }

/* cuda_sparse_convolution_mapping.cu:10-50: O = kx*ky xy-offsets, x outer,
 * y inner, z pinned at kz_min*sz; arithmetic modulo 2^bits. */
int orc_offsets(int kx, int ky, int kz, int sx, int sy, int sz, int bits, uint64_t *out) {
  layout_t L = layout_of(bits);
  int idx = 0;
  for (int64_t ix = kmin_of(kx); ix <= kx / 2; ++ix)
    for (int64_t iy = kmin_of(ky); iy <= ky / 2; ++iy) {
      uint64_t v = (uint64_t)(ix * sx) * (1ull << L.xs) + (uint64_t)(iy * sy) * (1ull << L.ys) +
                   (uint64_t)(kmin_of(kz) * sz);
      out[idx++] = v & L.modmask;
    }
  return idx;
}

/* cuda_sparse_convolution_mapping.cu:114-157: all K offsets, z innermost. */
int orc_offsets_full(int kx, int ky, int kz, int sx, int sy, int sz, int bits, uint64_t *out) {
  layout_t L = layout_of(bits);
  int idx = 0;
  for (int64_t ix = kmin_of(kx); ix <= kx / 2; ++ix)
    for (int64_t iy = kmin_of(ky); iy <= ky / 2; ++iy)
      for (int64_t iz = kmin_of(kz); iz <= kz / 2; ++iz) {
        uint64_t v = (uint64_t)(ix * sx) * (1ull << L.xs) + (uint64_t)(iy * sy) * (1ull << L.ys) +
                     (uint64_t)(iz * sz);
        out[idx++] = v & L.modmask;
      }
  return idx;
}

/* cuda_sparse_convolution_mapping.cu:159-209: data[canonical k] = row position;
 * offsets with |dx|+|dy|+|dz| < (dataflow-1)/2 come first.  Returns the number
 * of front ("dense") offsets. */
int orc_indexes_l1(int kx, int ky, int kz, int dataflow, int32_t *data) {
  int thr = (dataflow - 1) / 2, front = 0;
  for (int64_t x = kmin_of(kx); x < kmin_of(kx) + kx; ++x)
    for (int64_t y = kmin_of(ky); y < kmin_of(ky) + ky; ++y)
      for (int64_t z = kmin_of(kz); z < kmin_of(kz) + kz; ++z)
        if (llabs(x) + llabs(y) + llabs(z) < thr) ++front;
  int fp = 0, bp = front, k = 0;
  for (int64_t x = kmin_of(kx); x < kmin_of(kx) + kx; ++x)
    for (int64_t y = kmin_of(ky); y < kmin_of(ky) + ky; ++y)
      for (int64_t z = kmin_of(kz); z < kmin_of(kz) + kz; ++z)
        data[k++] = (llabs(x) + llabs(y) + llabs(z) < thr) ? fp++ : bp++;
  return front;
}

/* binary_search.cuh:10-21 (unsigned compare on CT). */
static int64_t lower_bound_u64(const uint64_t *a, int64_t n, uint64_t v) {
  int64_t l = 0, r = n;
  while (l < r) {
    int64_t m = (l + r) >> 1;
    if (a[m] >= v) r = m; else l = m + 1;
  }
  return l;
}

enum { ORC_OS = 0, ORC_WS = 1, ORC_HYBRID = 2, ORC_NOZ = 3 };

/* query_sorted.cuh:8-163.  For each target t and xy offset o:
 *   c = tgt[t] + off[o]; idx = lower_bound(src, c); entry(iz=0) = idx if src[idx]==c
 *   for iz >= 1: idx += (src[idx] <= c); c += sz; entry = idx if idx<S && src[idx]==c
 * An index equal to S (the reference reads one past the end there) is -1.
 * layout ORC_OS: [Tp, K], column iz*O + o (z-major, query_sorted.cuh:246-256)
 * layout ORC_WS: [K, Tp], row o*kz + iz        (query_sorted.cuh:126-149)
 * layout ORC_HYBRID: [K, Tp], row perm[o*kz+iz] (query_sorted.cuh:175-206)
 * layout ORC_NOZ: [Tp, K] canonical, one full search per offset (:261-297).
 * Padded targets t in [T, Tp) are all -1. */
void orc_search(const uint64_t *src, int64_t S, const uint64_t *tgt, int64_t T, int64_t Tp,
                int bits, int kx, int ky, int kz, int sx, int sy, int sz, int layout,
                const int32_t *perm, int32_t *map) {
  layout_t L = layout_of(bits);
  uint64_t offs[4096];
  int O, K;
  if (layout == ORC_NOZ) {
    O = orc_offsets_full(kx, ky, kz, sx, sy, sz, bits, offs);
    K = O;
  } else {
    O = orc_offsets(kx, ky, kz, sx, sy, sz, bits, offs);
    K = O * kz;
  }
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < Tp; ++t) {
    for (int o = 0; o < O; ++o) {
      int32_t res[64];
      int nz = (layout == ORC_NOZ) ? 1 : kz;
      if (t >= T) {
        for (int iz = 0; iz < nz; ++iz) res[iz] = -1;
      } else {
        uint64_t c = (tgt[t] + offs[o]) & L.modmask;
        int64_t idx = lower_bound_u64(src, S, c);
        res[0] = (idx < S && src[idx] == c) ? (int32_t)idx : -1;
        for (int iz = 1; iz < nz; ++iz) {
          if (idx < S && src[idx] <= c) ++idx;
          c = (c + (uint64_t)(uint32_t)sz) & L.modmask;
          res[iz] = (idx < S && src[idx] == c) ? (int32_t)idx : -1;
        }
      }
      for (int iz = 0; iz < nz; ++iz) {
        int k = o * nz + iz;
        if (layout == ORC_OS) map[t * K + iz * O + o] = res[iz];
        else if (layout == ORC_WS) map[(int64_t)k * Tp + t] = res[iz];
        else if (layout == ORC_HYBRID) map[(int64_t)perm[k] * Tp + t] = res[iz];
        else map[t * K + o] = res[0];
      }
    }
  }
}

/* query_sorted_index.cu:146-209 (+ quantifier_wstat.cuh:8-41): rows
 * [row0, row0+R) of a [*, Tp] WS map are compacted in (row, t) order into
 * in_idx (the map value, source) / out_idx (t, target); nbsizes[r] counts row
 * r; naddrs / qnaddrs are the exclusive scans of nbsizes and of nbsizes
 * rounded up to multiples of q.  Returns the pair count P. */
int64_t orc_ws_pairs(const int32_t *map, int64_t Tp, int row0, int R, int q,
                     int32_t *nbsizes, int32_t *naddrs, int32_t *qnaddrs,
                     int32_t *in_idx, int32_t *out_idx) {
  int64_t p = 0;
  naddrs[0] = 0; qnaddrs[0] = 0;
  for (int r = 0; r < R; ++r) {
    const int32_t *row = map + (int64_t)(row0 + r) * Tp;
    int32_t cnt = 0;
    for (int64_t t = 0; t < Tp; ++t)
      if (row[t] != -1) {
        if (in_idx) { in_idx[p] = row[t]; out_idx[p] = (int32_t)t; }
        ++p; ++cnt;
      }
    nbsizes[r] = cnt;
    naddrs[r + 1] = naddrs[r] + cnt;
    qnaddrs[r + 1] = qnaddrs[r] + (cnt + q - 1) / q * q;
  }
  return p;
}

/* query_sorted_index.cu:424-495 + generate_masks_from_kernel_map.cuh:10-62:
 * masks [Km, S] / [Km, T] start at -1; for each compacted row r and its i-th
 * valid entry (t, s): source_masks[r, s] = target_masks[r, t] = i.  With
 * `half`, row Km-1-r also gets source_masks[., t] = target_masks[., s] = i
 * unless 2r+1 == Km.  nbsizes[r] counts row r (R rows). */
void orc_gs_masks(const int32_t *map, int64_t S, int64_t T, int64_t Tp, int row0, int R,
                  int Km, int half, int32_t *smask, int32_t *tmask, int32_t *nbsizes) {
  for (int64_t i = 0; i < (int64_t)Km * S; ++i) smask[i] = -1;
  for (int64_t i = 0; i < (int64_t)Km * T; ++i) tmask[i] = -1;
  for (int r = 0; r < R; ++r) {
    const int32_t *row = map + (int64_t)(row0 + r) * Tp;
    int32_t rank = 0;
    for (int64_t t = 0; t < Tp; ++t) {
      int32_t s = row[t];
      if (s == -1) continue;
      smask[(int64_t)r * S + s] = rank;
      tmask[(int64_t)r * T + t] = rank;
      if (half && 2 * r + 1 != Km) {
        smask[(int64_t)(Km - 1 - r) * S + t] = rank;
        tmask[(int64_t)(Km - 1 - r) * T + s] = rank;
      }
      ++rank;
    }
    nbsizes[r] = rank;
  }
}

/* convert_transposed_os.cuh:7-16: out[s, k] = t where map[t, k] = s; the
 * output has Sp rows and starts at -1 (cuda_sparse_convolution_mapping.cu:1817). */
void orc_convert_transposed_os(const int32_t *map, int64_t Tp, int K, int64_t Sp, int32_t *out) {
  for (int64_t i = 0; i < Sp * K; ++i) out[i] = -1;
  for (int64_t i = 0; i < Tp * K; ++i) {
    int32_t s = map[i];
    if (s < 0) continue;
    out[(int64_t)s * K + i % K] = (int32_t)(i / K);
  }
}

/* sparse_convolution.cu:488-515: greedy merge of adjacent offsets while the
 * padding redundancy stays within threshold.  has_thr=0 is "None" (merge all);
 * a negative threshold never merges.  Returns the bucket count; bounds holds
 * nb+1 entries. */
int orc_padding_buckets(int K, const int32_t *sizes, int has_thr, double thr, int32_t *bounds) {
  int nb = 0;
  bounds[0] = 0;
  for (int i = 0; i < K; ++i) {
    int j = i;
    uint64_t actual = (uint64_t)sizes[i], summit = (uint64_t)sizes[i];
    while (i + 1 < K) {
      actual += (uint64_t)sizes[i + 1];
      if ((uint64_t)sizes[i + 1] > summit) summit = (uint64_t)sizes[i + 1];
      uint64_t padded = summit * (uint64_t)((i + 1) - j + 1);
      double red = (double)(padded - actual) / (double)actual;
      if (has_thr && (thr < 0 || red > thr)) break;
      ++i;
    }
    bounds[++nb] = i + 1;
  }
  return nb;
}

/* Output-stationary feature sum in float64 (the semantics of
 * output_stat.cuh:20-1031): Y[t, :] = sum_j X[map[t, j], :] @ W[j]. */
void orc_conv_os(const int32_t *map, int64_t T, int Kc, const double *X, int Cin,
                 const double *W, int Cout, double *Y) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < T; ++t) {
    double *y = Y + t * Cout;
    for (int c = 0; c < Cout; ++c) y[c] = 0.0;
    for (int j = 0; j < Kc; ++j) {
      int32_t s = map[t * Kc + j];
      if (s < 0) continue;
      const double *x = X + (int64_t)s * Cin;
      const double *w = W + (int64_t)j * Cin * Cout;
      for (int ci = 0; ci < Cin; ++ci) {
        double xv = x[ci];
        const double *wr = w + (int64_t)ci * Cout;
        for (int c = 0; c < Cout; ++c) y[c] += xv * wr[c];
      }
    }
  }
}

/* Pair-list feature sum in float64 (the semantics of weight_stat.cuh and of
 * the gather -> GEMM -> scatter path): Y[out[p]] += X[in[p]] @ W[w[p]].
 * Y is accumulated into (not cleared).  Serial over pairs, so exact order. */
void orc_conv_pairs(int64_t P, const int32_t *in_idx, const int32_t *out_idx, const int32_t *widx,
                    const double *X, int Cin, const double *W, int Cout, double *Y) {
  /* Y[out[p]] += X[in[p]] @ W[widx[p]].  The pairs are bucketed by output
   * row (a stable counting sort, so each row still sums its pairs in list
   * order) and the rows are summed in parallel. */
  if (P <= 0) return;
  int64_t nout = 0;
  for (int64_t p = 0; p < P; ++p)
    if (out_idx[p] + 1 > nout) nout = out_idx[p] + 1;
  int64_t *start = (int64_t *)calloc((size_t)nout + 1, sizeof(int64_t));
  int64_t *order = (int64_t *)malloc((size_t)P * sizeof(int64_t));
  for (int64_t p = 0; p < P; ++p) start[out_idx[p] + 1]++;
  for (int64_t t = 0; t < nout; ++t) start[t + 1] += start[t];
  {
    int64_t *fill = (int64_t *)malloc((size_t)nout * sizeof(int64_t));
    for (int64_t t = 0; t < nout; ++t) fill[t] = start[t];
    for (int64_t p = 0; p < P; ++p) order[fill[out_idx[p]]++] = p;
    free(fill);
  }
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < nout; ++t) {
    double *y = Y + t * Cout;
    for (int64_t q = start[t]; q < start[t + 1]; ++q) {
      const int64_t p = order[q];
      const double *x = X + (int64_t)in_idx[p] * Cin;
      const double *w = W + (int64_t)widx[p] * Cin * Cout;
      for (int ci = 0; ci < Cin; ++ci) {
        double xv = x[ci];
        const double *wr = w + (int64_t)ci * Cout;
        for (int c = 0; c < Cout; ++c) y[c] += xv * wr[c];
      }
    }
  }
  free(start);
  free(order);
}

/* float32-accumulating output-stationary sum: the CPU baseline's compute leg
 * (same arithmetic class as the GPU path: fp32 multiply-accumulate). */
void orc_conv_os_f32(const int32_t *map, int64_t T, int Kc, const float *X, int Cin,
                     const float *W, int Cout, float *Y) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < T; ++t) {
    float *y = Y + t * Cout;
    for (int c = 0; c < Cout; ++c) y[c] = 0.f;
    for (int j = 0; j < Kc; ++j) {
      int32_t s = map[t * Kc + j];
      if (s < 0) continue;
      const float *x = X + (int64_t)s * Cin;
      const float *w = W + (int64_t)j * Cin * Cout;
      for (int ci = 0; ci < Cin; ++ci) {
        float xv = x[ci];
        const float *wr = w + (int64_t)ci * Cout;
        for (int c = 0; c < Cout; ++c) y[c] += xv * wr[c];
      }
    }
  }
}
