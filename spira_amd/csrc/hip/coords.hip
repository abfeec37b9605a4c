// Packed voxel keys: pack / unpack, flatten + argsort, stride downsampling.
//
// Reference semantics: compress.cuh:9-46 (pack/unpack),
// arg_sort_coodrinates.cu:36-192 (sort, sort+unique),
// (stride downsampling: downsample.hip).
#include "common.hpp"
#include "../../../include/spira_hip.h"

#include <rocprim/rocprim.hpp>

#include <mutex>
#include <unordered_map>

namespace spira_hip {

static thread_local std::string g_last_error;
void set_error(const std::string &msg) { g_last_error = msg; }
const char *get_error() { return g_last_error.c_str(); }

int device_cu_count() {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  cache[dev] = cus;
  return cus;
}

// key = (CT)x << XS | (CT)y << YS | (CT)z, each int32 converted to CT first
template <typename CT>
__global__ void pack_kernel(int64_t n, const int32_t *__restrict__ coords, CT *__restrict__ keys) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t *c = coords + 3 * i;
  CT ux = static_cast<CT>(c[0]), uy = static_cast<CT>(c[1]), uz = static_cast<CT>(c[2]);
  keys[i] = (ux << Layout<CT>::XS) | (uy << Layout<CT>::YS) | uz;
}

template <typename CT>
__global__ void pack_iota_kernel(int64_t n, const int32_t *__restrict__ coords, CT *__restrict__ keys,
                                 int32_t *__restrict__ iota) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t *c = coords + 3 * i;
  CT ux = static_cast<CT>(c[0]), uy = static_cast<CT>(c[1]), uz = static_cast<CT>(c[2]);
  keys[i] = (ux << Layout<CT>::XS) | (uy << Layout<CT>::YS) | uz;
  iota[i] = static_cast<int32_t>(i);
}

template <typename CT>
__global__ void unpack_kernel(int64_t n, const CT *__restrict__ keys, int32_t *__restrict__ coords) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  CT k = keys[i];
  int32_t *c = coords + 3 * i;
  c[0] = static_cast<int32_t>((k >> Layout<CT>::XS) & Layout<CT>::XONES);
  c[1] = static_cast<int32_t>((k >> Layout<CT>::YS) & Layout<CT>::YONES);
  c[2] = static_cast<int32_t>(k & Layout<CT>::ZONES);
}

static inline bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// ---------------------------------------------------------------------------
// workspace layouts
// ---------------------------------------------------------------------------
template <typename CT> static size_t sort_temp_bytes(int64_t n) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, bytes, static_cast<const CT *>(nullptr), static_cast<CT *>(nullptr),
                            static_cast<const int32_t *>(nullptr), static_cast<int32_t *>(nullptr),
                            static_cast<size_t>(n), 0, 8 * sizeof(CT));
  return bytes;
}

static inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

template <typename CT> static size_t flatten_ws(int64_t n) {
  return align256(n * sizeof(CT)) + align256(n * sizeof(int32_t)) + align256(sort_temp_bytes<CT>(n));
}

template <typename CT>
static int flatten_sort_impl(const int32_t *coords, int64_t n, CT *keys_out, int32_t *perm_out, void *ws,
                             size_t ws_bytes, hipStream_t s) {
  SPIRA_HIP_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "flatten_sort: n out of range");
  if (n == 0) return kOk;
  SPIRA_HIP_REQUIRE(ws != nullptr && ws_bytes >= flatten_ws<CT>(n), "flatten_sort: workspace too small");
  char *p = static_cast<char *>(ws);
  CT *keys_in = reinterpret_cast<CT *>(p);
  p += align256(n * sizeof(CT));
  int32_t *iota = reinterpret_cast<int32_t *>(p);
  p += align256(n * sizeof(int32_t));
  size_t tb = sort_temp_bytes<CT>(n);
  hipLaunchKernelGGL(pack_iota_kernel<CT>, dim3(div_up(n, 256)), dim3(256), 0, s, n, coords, keys_in, iota);
  SPIRA_HIP_LAUNCH_CHECK();
  SPIRA_HIP_TRY(rocprim::radix_sort_pairs(p, tb, keys_in, keys_out, iota, perm_out, static_cast<size_t>(n), 0,
                                          8 * sizeof(CT), s));
  return kOk;
}

// ---------------------------------------------------------------------------
// Allocation-free flatten_sort: its workspace lives in a fixed device array.
// Every GPU holds its own copy of `scratch` (for the life of the process);
// host code must use the address hipGetSymbolAddress returns for the current
// device, never the array's name (a host-side stand-in).
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocMaxPoints = int64_t(1) << 20;
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once
// per device; nullptr (with the error set) on failure.
static void *noalloc_scratch() {
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("flatten_sort_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error(std::string("flatten_sort_noalloc: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace spira_hip

using namespace spira_hip;

extern "C" {

const char *spira_hip_last_error(void) { return get_error(); }

int spira_hip_pack(const int32_t *coords, int64_t n, int key_bits, void *keys, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "pack: key_bits must be 32 or 64");
  if (n <= 0) return kOk;
  if (key_bits == 64)
    hipLaunchKernelGGL(pack_kernel<uint64_t>, dim3(div_up(n, 256)), dim3(256), 0, stream, n, coords,
                       static_cast<uint64_t *>(keys));
  else
    hipLaunchKernelGGL(pack_kernel<uint32_t>, dim3(div_up(n, 256)), dim3(256), 0, stream, n, coords,
                       static_cast<uint32_t *>(keys));
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_unpack(const void *keys, int64_t n, int key_bits, int32_t *coords, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "unpack: key_bits must be 32 or 64");
  if (n <= 0) return kOk;
  if (key_bits == 64)
    hipLaunchKernelGGL(unpack_kernel<uint64_t>, dim3(div_up(n, 256)), dim3(256), 0, stream, n,
                       static_cast<const uint64_t *>(keys), coords);
  else
    hipLaunchKernelGGL(unpack_kernel<uint32_t>, dim3(div_up(n, 256)), dim3(256), 0, stream, n,
                       static_cast<const uint32_t *>(keys), coords);
  SPIRA_HIP_LAUNCH_CHECK();
  return kOk;
}

int spira_hip_flatten_sort_workspace(int64_t n, int key_bits, size_t *bytes) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "flatten_sort: key_bits must be 32 or 64");
  *bytes = n <= 0 ? 0 : (key_bits == 64 ? flatten_ws<uint64_t>(n) : flatten_ws<uint32_t>(n));
  return kOk;
}

int spira_hip_flatten_sort(const int32_t *coords, int64_t n, int key_bits, void *keys_out, int32_t *perm_out,
                           void *workspace, size_t workspace_bytes, hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "flatten_sort: key_bits must be 32 or 64");
  if (key_bits == 64)
    return flatten_sort_impl<uint64_t>(coords, n, static_cast<uint64_t *>(keys_out), perm_out, workspace,
                                       workspace_bytes, stream);
  return flatten_sort_impl<uint32_t>(coords, n, static_cast<uint32_t *>(keys_out), perm_out, workspace,
                                     workspace_bytes, stream);
}

int spira_hip_flatten_sort_noalloc(const int32_t *coords, int64_t n, int key_bits, void *keys_out, int32_t *perm_out,
                                   hipStream_t stream) {
  SPIRA_HIP_REQUIRE(key_bits == 32 || key_bits == 64, "flatten_sort_noalloc: key_bits must be 32 or 64");
  SPIRA_HIP_REQUIRE(n >= 0 && n <= kNoAllocMaxPoints,
                    "flatten_sort_noalloc: at most 1048576 points (n = " + std::to_string(n) + ")");
  if (n == 0) return kOk;
  const size_t need = key_bits == 64 ? flatten_ws<uint64_t>(n) : flatten_ws<uint32_t>(n);
  SPIRA_HIP_REQUIRE(need <= kNoAllocScratchBytes, "flatten_sort_noalloc: workspace of " + std::to_string(need) +
                                                      " bytes exceeds the fixed scratch");
  void *ws = noalloc_scratch();
  if (ws == nullptr) return kHipError;
  // every buffer in the scratch is fully written before it is read (pack +
  // iota, then the sort), so nothing needs clearing between calls
  return spira_hip_flatten_sort(coords, n, key_bits, keys_out, perm_out, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
