// Shared helpers of the torch host layer (the `_C` extension module).
// This layer owns tensor validation, allocation and stream selection; all
// device work goes through the C ABI of libspira_hip.so (include/spira_hip.h).
#pragma once

#include <torch/extension.h>
#include <ATen/hip/HIPContext.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <optional>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "../../../include/spira_hip.h"

namespace spira_host {

// Errors surface as RuntimeError("[Spira] ...") like the reference's
// SpiraException (common/exception.h:9-28), which the selector catches.
template <typename... Args> [[noreturn]] inline void fail(Args &&...args) {
  std::ostringstream os;
  os << "[Spira] ";
  (os << ... << args);
  throw std::runtime_error(os.str());
}

#define SPIRA_CHECK_ARG(cond, ...)                  \
  do {                                              \
    if (!(cond)) ::spira_host::fail(__VA_ARGS__);   \
  } while (0)

inline void check_rc(int rc, const char *what) {
  if (rc != 0) fail(what, ": ", spira_hip_last_error());
}

inline hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

inline void require_device(const torch::Tensor &t, const char *name) {
  SPIRA_CHECK_ARG(t.is_cuda(), name, " must be a GPU tensor");
  SPIRA_CHECK_ARG(t.is_contiguous(), name, " must be contiguous");
}

inline int key_bits_of(const torch::Tensor &keys) {
  if (keys.scalar_type() == torch::kInt64) return 64;
  if (keys.scalar_type() == torch::kInt32) return 32;
  fail("Cannot find implementation for coordinate dtype ", keys.scalar_type());
}

inline int64_t round128(int64_t n) { return (n + 127) / 128 * 128; }

inline torch::Tensor empty_i32(torch::IntArrayRef shape, const torch::Device &dev) {
  return torch::empty(shape, torch::TensorOptions(dev).dtype(torch::kInt32));
}

inline torch::Tensor workspace(size_t bytes, const torch::Device &dev) {
  return torch::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)}, torch::TensorOptions(dev).dtype(torch::kUInt8));
}

// Fork work from the current stream onto n pool streams and join it back:
// every side stream first waits for the work already queued on the current
// stream, and join() makes the current stream wait for every side stream, so
// tensors allocated on the current stream stay valid for the side work.
class StreamFan {
 public:
  StreamFan(const torch::Device &dev, size_t n) : main_(current_stream()) {
    if (n == 0) return;
    hipEvent_t e = event(0);
    check_hip(hipEventRecord(e, main_));
    for (size_t i = 0; i < n; ++i) {
      side_.push_back(c10::hip::getStreamFromPool(false, dev.index()));
      check_hip(hipStreamWaitEvent(side_.back().stream(), e, 0));
    }
  }
  hipStream_t operator[](size_t i) const { return side_[i].stream(); }
  size_t size() const { return side_.size(); }
  void join() {
    for (size_t i = 0; i < side_.size(); ++i) {
      hipEvent_t e = event(i + 1);
      check_hip(hipEventRecord(e, side_[i].stream()));
      check_hip(hipStreamWaitEvent(main_, e, 0));
    }
    side_.clear();
  }
  ~StreamFan() {
    if (!side_.empty()) {
      try { join(); } catch (...) {}
    }
  }

 private:
  static void check_hip(hipError_t e) {
    if (e != hipSuccess) fail("HIP error: ", hipGetErrorString(e));
  }
  // Timing-free events, created once per (device, slot) and reused: an
  // event may be recorded again once the waits on its previous record are
  // enqueued (each wait captures the record it follows), and creating and
  // destroying events costs more host time than the fan-out's launches.
  static hipEvent_t event(size_t slot) {
    int dev = 0;
    check_hip(hipGetDevice(&dev));
    static std::mutex mu;
    static std::map<std::pair<int, size_t>, hipEvent_t> pool;
    std::lock_guard<std::mutex> lock(mu);
    auto &e = pool[{dev, slot}];
    if (!e) check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return e;
  }
  hipStream_t main_;
  std::vector<c10::hip::HIPStream> side_;
};

using Int3 = std::tuple<int, int, int>;

// The 9-tuple returned by the map builders (reference:
// torch/cuda_sparse_convolution_mapping.cu:211-892).
using KmapTuple = std::tuple<int64_t, int64_t, torch::Tensor, std::optional<torch::Tensor>,
                             std::optional<torch::Tensor>, std::optional<torch::Tensor>,
                             std::optional<torch::Tensor>, std::optional<int32_t>, std::optional<int32_t>>;

// kernel offset row order for the hybrid dataflows
// (reference: generate_indexes_L1, torch/cuda_sparse_convolution_mapping.cu:159-209)
std::vector<int32_t> indexes_l1(int kx, int ky, int kz, int dataflow, int *front);

// ---- registration entry points, one per source file ----
void register_coords(pybind11::module_ &m);
void register_mapping(pybind11::module_ &m);
void register_conv(pybind11::module_ &m);

}  // namespace spira_host
