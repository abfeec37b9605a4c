// Voxelization front-end: points -> sorted unique int32 voxel coordinates.
//
// Reference semantics: sparse_quantize (datasets/helpers.py:14-30):
//   coords = floor(points / voxel) (float64 division, then int32);
//   keep the first point of every value of ravel_hash(coords)
//     = x*73856093 ^ y*19349663 ^ z*83492791 over the coordinates cast to
//       uint64 (helpers.py:8-12; distinct voxels whose hashes collide
//       collapse to the first of them, as there);
//   sort the kept coordinates lexicographically by (x, y, z).
//
// GPU design: one pass quantizes and hashes every point; a stable radix sort
// of (hash, point index) puts each hash's first point at the head of its run;
// the run heads are keyed by (y, z) and then, stably, by x (two radix sorts,
// the non-heads keyed past every real voxel so that they sort last); the
// first `count` rows of the output are the result.  No host synchronisation:
// the count stays on the device.
#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <rocprim/rocprim.hpp>

#include <algorithm>

namespace spira_hip {

template <typename PT>
__global__ void quantize_hash_kernel(int64_t n, const PT *__restrict__ pts, double vx, double vy, double vz,
                                     int32_t *__restrict__ coords, uint64_t *__restrict__ hash,
                                     int32_t *__restrict__ iota) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t x = static_cast<int32_t>(floor(static_cast<double>(pts[3 * i]) / vx));
  const int32_t y = static_cast<int32_t>(floor(static_cast<double>(pts[3 * i + 1]) / vy));
  const int32_t z = static_cast<int32_t>(floor(static_cast<double>(pts[3 * i + 2]) / vz));
  coords[3 * i] = x;
  coords[3 * i + 1] = y;
  coords[3 * i + 2] = z;
  // int32 -> uint64 sign-extends, as numpy's astype(np.uint64) does
  const uint64_t ux = static_cast<uint64_t>(static_cast<int64_t>(x));
  const uint64_t uy = static_cast<uint64_t>(static_cast<int64_t>(y));
  const uint64_t uz = static_cast<uint64_t>(static_cast<int64_t>(z));
  hash[i] = (ux * 73856093ull) ^ (uy * 19349663ull) ^ (uz * 83492791ull);
  iota[i] = static_cast<int32_t>(i);
}

constexpr uint64_t kPastEveryVoxel = ~uint64_t(0);

// Run heads of the hash-sorted points: key (y, z) with the signs flipped so
// that unsigned order is signed order; other entries get the largest key.
__global__ void head_keys_kernel(int64_t n, const uint64_t *__restrict__ hash_s, const int32_t *__restrict__ idx_s,
                                 const int32_t *__restrict__ coords, uint64_t *__restrict__ yz,
                                 int32_t *__restrict__ val, uint32_t *__restrict__ count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const bool head = i == 0 || hash_s[i] != hash_s[i - 1];
  if (head) {
    const int32_t p = idx_s[i];
    const uint32_t y = static_cast<uint32_t>(coords[3 * p + 1]) ^ 0x80000000u;
    const uint32_t z = static_cast<uint32_t>(coords[3 * p + 2]) ^ 0x80000000u;
    yz[i] = (static_cast<uint64_t>(y) << 32) | z;
    val[i] = p;
    atomicAdd(count, 1u);
  } else {
    yz[i] = kPastEveryVoxel;
    val[i] = -1;
  }
}

__global__ void x_keys_kernel(int64_t n, const int32_t *__restrict__ val, const int32_t *__restrict__ coords,
                              uint32_t *__restrict__ xk) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t p = val[i];
  xk[i] = p < 0 ? 0xFFFFFFFFu : (static_cast<uint32_t>(coords[3 * p]) ^ 0x80000000u);
}

__global__ void gather_coords_kernel(int64_t n, const int32_t *__restrict__ val, const int32_t *__restrict__ coords,
                                     int32_t *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t p = val[i];
#pragma unroll
  for (int a = 0; a < 3; ++a) out[3 * i + a] = p < 0 ? 0 : coords[3 * p + a];
}

__global__ void zero_u32_kernel(uint32_t *p) { *p = 0; }

struct VoxelizeParts {
  int32_t *coords, *iota, *idx_s, *val, *val_s, *val_f;
  uint64_t *hash, *hash_s, *yz, *yz_s;
  uint32_t *xk, *xk_s;
  void *tmp;
  size_t tmp_bytes, total;
};

static VoxelizeParts voxelize_parts(int64_t n, void *base) {
  size_t b1 = 0, b2 = 0;
  (void)rocprim::radix_sort_pairs(nullptr, b1, static_cast<const uint64_t *>(nullptr),
                                  static_cast<uint64_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(n), 0, 64);
  (void)rocprim::radix_sort_pairs(nullptr, b2, static_cast<const uint32_t *>(nullptr),
                                  static_cast<uint32_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                  static_cast<int32_t *>(nullptr), static_cast<size_t>(n), 0, 32);
  VoxelizeParts v{};
  v.tmp_bytes = std::max(b1, b2);
  char *p = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *q = p ? p + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return q;
  };
  v.coords = reinterpret_cast<int32_t *>(take(n * 3 * sizeof(int32_t)));
  v.iota = reinterpret_cast<int32_t *>(take(n * sizeof(int32_t)));
  v.idx_s = reinterpret_cast<int32_t *>(take(n * sizeof(int32_t)));
  v.val = reinterpret_cast<int32_t *>(take(n * sizeof(int32_t)));
  v.val_s = reinterpret_cast<int32_t *>(take(n * sizeof(int32_t)));
  v.val_f = reinterpret_cast<int32_t *>(take(n * sizeof(int32_t)));
  v.hash = reinterpret_cast<uint64_t *>(take(n * sizeof(uint64_t)));
  v.hash_s = reinterpret_cast<uint64_t *>(take(n * sizeof(uint64_t)));
  v.yz = reinterpret_cast<uint64_t *>(take(n * sizeof(uint64_t)));
  v.yz_s = reinterpret_cast<uint64_t *>(take(n * sizeof(uint64_t)));
  v.xk = reinterpret_cast<uint32_t *>(take(n * sizeof(uint32_t)));
  v.xk_s = reinterpret_cast<uint32_t *>(take(n * sizeof(uint32_t)));
  v.tmp = take(v.tmp_bytes);
  v.total = off;
  return v;
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

int spira_hip_voxelize_workspace(int64_t num_points, size_t *bytes) {
  *bytes = num_points <= 0 ? 0 : voxelize_parts(num_points, nullptr).total;
  return kOk;
}

int spira_hip_voxelize(const void *points, int64_t num_points, int points_f64, double vx, double vy, double vz,
                       int32_t *coords, uint32_t *count, void *workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  SPIRA_HIP_REQUIRE(num_points >= 0 && num_points < (int64_t(1) << 31), "voxelize: num_points out of range");
  SPIRA_HIP_REQUIRE(vx > 0 && vy > 0 && vz > 0, "voxelize: voxel sizes must be positive");
  SPIRA_HIP_REQUIRE(count != nullptr, "voxelize: count must not be null");
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(1), 0, stream, count);
  SPIRA_HIP_LAUNCH_CHECK();
  const int64_t n = num_points;
  if (n == 0) return kOk;
  SPIRA_HIP_REQUIRE(workspace != nullptr && workspace_bytes >= voxelize_parts(n, nullptr).total,
                    "voxelize: workspace too small");
  VoxelizeParts v = voxelize_parts(n, workspace);
  const dim3 grid(static_cast<unsigned>(div_up(n, 256)));
  if (points_f64)
    hipLaunchKernelGGL(quantize_hash_kernel<double>, grid, dim3(256), 0, stream, n,
                       static_cast<const double *>(points), vx, vy, vz, v.coords, v.hash, v.iota);
  else
    hipLaunchKernelGGL(quantize_hash_kernel<float>, grid, dim3(256), 0, stream, n,
                       static_cast<const float *>(points), vx, vy, vz, v.coords, v.hash, v.iota);
  SPIRA_HIP_LAUNCH_CHECK();
  size_t tb = v.tmp_bytes;
  SPIRA_HIP_TRY(rocprim::radix_sort_pairs(v.tmp, tb, v.hash, v.hash_s, v.iota, v.idx_s, static_cast<size_t>(n), 0,
                                          64, stream));
  hipLaunchKernelGGL(head_keys_kernel, grid, dim3(256), 0, stream, n, v.hash_s, v.idx_s, v.coords, v.yz, v.val,
                     count);
  SPIRA_HIP_LAUNCH_CHECK();
  tb = v.tmp_bytes;
  SPIRA_HIP_TRY(rocprim::radix_sort_pairs(v.tmp, tb, v.yz, v.yz_s, v.val, v.val_s, static_cast<size_t>(n), 0, 64,
                                          stream));
  hipLaunchKernelGGL(x_keys_kernel, grid, dim3(256), 0, stream, n, v.val_s, v.coords, v.xk);
  SPIRA_HIP_LAUNCH_CHECK();
  tb = v.tmp_bytes;
  SPIRA_HIP_TRY(rocprim::radix_sort_pairs(v.tmp, tb, v.xk, v.xk_s, v.val_s, v.val_f, static_cast<size_t>(n), 0, 32,
                                          stream));
  hipLaunchKernelGGL(gather_coords_kernel, grid, dim3(256), 0, stream, n, v.val_f, v.coords, coords);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

}  // extern "C"
