// Shared helpers of the gfx950 kernel library (libspira_hip.so).
#pragma once

#include <cstring>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace spira_hip {

// ---------------------------------------------------------------------------
// error reporting: every extern "C" entry point returns 0 on success or a
// non-zero code, with the message kept per thread for spira_hip_last_error().
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
const char *get_error();

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kHipError = 2,
  kUnsupported = 3,
};

#define SPIRA_HIP_TRY(expr)                                                        \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess) {                                                        \
      ::spira_hip::set_error(std::string(#expr) + " failed: " + hipGetErrorString(_e) + \
                             " (" + __FILE__ + ":" + std::to_string(__LINE__) + ")"); \
      return ::spira_hip::kHipError;                                               \
    }                                                                              \
  } while (0)

#define SPIRA_HIP_REQUIRE(cond, msg)                                               \
  do {                                                                             \
    if (!(cond)) {                                                                 \
      ::spira_hip::set_error(std::string(msg));                                    \
      return ::spira_hip::kInvalidArgument;                                        \
    }                                                                              \
  } while (0)

#define SPIRA_HIP_LAUNCH_CHECK() SPIRA_HIP_TRY(hipGetLastError())

// ---------------------------------------------------------------------------
// packed coordinate layouts: 32-bit keys x12|y12|z8, 64-bit keys x24|y24|z16
// (the reference's compress_layout.h:11-44; the bit layout is a data format
// shared with existing callers, so it is kept identical).
// ---------------------------------------------------------------------------
template <typename CT> struct Layout;
template <> struct Layout<uint32_t> {
  static constexpr int XS = 20, YS = 8;
  static constexpr uint32_t XONES = 0xFFFu, YONES = 0xFFFu, ZONES = 0xFFu;
};
template <> struct Layout<uint64_t> {
  static constexpr int XS = 40, YS = 16;
  static constexpr uint64_t XONES = 0xFFFFFFull, YONES = 0xFFFFFFull, ZONES = 0xFFFFull;
};

inline int64_t div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return div_up(a, b) * b; }

// number of CUs, cached per device
int device_cu_count();

// ---------------------------------------------------------------------------
// wave64 primitives
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// number of set bits of `mask` below this lane
__device__ __forceinline__ int lane_prefix(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

template <typename T> __device__ __forceinline__ T wave_min(T v);
template <typename T> __device__ __forceinline__ T wave_max(T v);

template <> __device__ __forceinline__ uint64_t wave_min(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor(v, o, 64);
    v = w < v ? w : v;
  }
  return v;
}
template <> __device__ __forceinline__ uint64_t wave_max(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
template <> __device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t w = __shfl_xor(v, o, 64);
    v = w < v ? w : v;
  }
  return v;
}
template <> __device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

// broadcast a wave-uniform value held in a VGPR to an SGPR
template <typename T> __device__ __forceinline__ T uniform(T v) {
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ uint64_t uniform(uint64_t v) {
  uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ int64_t uniform(int64_t v) {
  return static_cast<int64_t>(uniform(static_cast<uint64_t>(v)));
}

}  // namespace spira_hip
