// Coordinate entry points of `_C`: flatten + sort, unflatten, downsample and
// the multi-stream downsample of every target stride.
// Reference: torch/cuda_arg_sort_coordinates.cu:11-208.
#include "host_common.h"

#include <cstring>

namespace spira_host {

// (coords [N,3] int32, is_double) -> (sorted keys [N] int64|int32, perm [N] int32)
// (reference: CUDAFlattenSort, torch/cuda_arg_sort_coordinates.cu:11-39)
std::pair<torch::Tensor, torch::Tensor> flatten_sort(const torch::Tensor &coordinates, bool is_double) {
  SPIRA_CHECK_ARG(coordinates.dim() == 2 && coordinates.size(1) == 3, "coordinates must be [N, 3]");
  SPIRA_CHECK_ARG(coordinates.scalar_type() == torch::kInt32, "coordinates must be int32");
  require_device(coordinates, "coordinates");
  const auto dev = coordinates.device();
  const int64_t n = coordinates.size(0);
  const int bits = is_double ? 64 : 32;
  auto keys = torch::empty({n}, torch::TensorOptions(dev).dtype(is_double ? torch::kInt64 : torch::kInt32));
  auto perm = empty_i32({n}, dev);
  size_t ws_bytes = 0;
  check_rc(spira_hip_flatten_sort_workspace(n, bits, &ws_bytes), "flatten_sort");
  auto ws = workspace(ws_bytes, dev);
  check_rc(spira_hip_flatten_sort(coordinates.data_ptr<int32_t>(), n, bits, keys.data_ptr(),
                                  perm.data_ptr<int32_t>(), ws.data_ptr(), ws_bytes, current_stream()),
           "flatten_sort");
  return {keys, perm};
}

// keys [N] -> coords [N,3] int32 (reference: CUDAUnFlatten, :41-65)
torch::Tensor unflatten(const torch::Tensor &keys) {
  SPIRA_CHECK_ARG(keys.dim() == 1, "keys must be 1-D");
  require_device(keys, "keys");
  const int bits = key_bits_of(keys);
  auto out = empty_i32({keys.size(0), 3}, keys.device());
  check_rc(spira_hip_unpack(keys.data_ptr(), keys.size(0), bits, out.data_ptr<int32_t>(), current_stream()),
           "unflatten");
  return out;
}

static void downsample_into(const torch::Tensor &keys, int sx, int sy, int sz, torch::Tensor &out,
                            uint32_t *d_count, hipStream_t stream) {
  const int bits = key_bits_of(keys);
  const int64_t n = keys.size(0);
  size_t ws_bytes = 0;
  check_rc(spira_hip_downsample_workspace(n, bits, &ws_bytes), "downsample");
  auto ws = workspace(ws_bytes, keys.device());
  check_rc(spira_hip_downsample(keys.data_ptr(), n, bits, sx, sy, sz, out.data_ptr(), d_count, ws.data_ptr(),
                                ws_bytes, stream),
           "downsample");
}

// (keys [N], sx, sy, sz) -> sorted unique downsampled keys [N']
// (reference: CUDADownsample, :68-105; blocking read of N' like the reference's)
torch::Tensor downsample(const torch::Tensor &keys, int sx, int sy, int sz) {
  SPIRA_CHECK_ARG(keys.dim() == 1, "coordinates should be already flattened");
  require_device(keys, "keys");
  key_bits_of(keys);
  auto out = torch::empty_like(keys);
  auto count = torch::zeros({1}, torch::TensorOptions(keys.device()).dtype(torch::kInt32));
  downsample_into(keys, sx, sy, sz, out, reinterpret_cast<uint32_t *>(count.data_ptr<int32_t>()),
                  current_stream());
  const int64_t nu = count.cpu().item<int32_t>();
  return out.slice(0, 0, nu);
}

// Whether the target strides form a chain spira_hip_downsample_chain takes:
// powers of two, each a multiple of the previous one per axis (the first of
// 1), with x ratio times y ratio at most 16 per level.
static bool chainable(const std::vector<Int3> &strides) {
  int prev[3] = {1, 1, 1};
  auto pow2 = [](int v) { return v > 0 && (v & (v - 1)) == 0; };
  for (auto &t : strides) {
    const int cur[3] = {std::get<0>(t), std::get<1>(t), std::get<2>(t)};
    for (int a = 0; a < 3; ++a)
      if (!pow2(cur[a]) || cur[a] % prev[a] != 0) return false;
    if ((cur[0] / prev[0]) * (cur[1] / prev[1]) > 16) return false;
    for (int a = 0; a < 3; ++a) prev[a] = cur[a];
  }
  return true;
}

// The chained downsample queued on the current stream with no host read:
// the outputs at full capacity (n keys each), then a device int32 tensor of
// B + 1 entries, the level counts and the unsorted-input flag.  Empty if the
// strides do not chain or there are no keys (the caller then takes
// streamed_output_generate).
std::vector<torch::Tensor> downsample_chain_launch(const torch::Tensor &keys, const std::vector<Int3> &strides) {
  SPIRA_CHECK_ARG(keys.dim() == 1, "coordinates should be already flattened");
  require_device(keys, "keys");
  const int bits = key_bits_of(keys);
  const auto dev = keys.device();
  const int64_t n = keys.size(0);
  const size_t B = strides.size();
  std::vector<torch::Tensor> outs;
  if (n == 0 || B == 0 || !chainable(strides)) return outs;
  std::vector<int32_t> st;
  for (auto &t : strides) {
    auto [sx, sy, sz] = t;
    st.insert(st.end(), {sx, sy, sz});
  }
  std::vector<void *> ptrs;
  for (size_t i = 0; i < B; ++i) {
    outs.push_back(torch::empty_like(keys));
    ptrs.push_back(outs.back().data_ptr());
  }
  auto cnt = torch::zeros({static_cast<int64_t>(B + 1)}, torch::TensorOptions(dev).dtype(torch::kInt32));
  size_t cwb = 0;
  check_rc(spira_hip_downsample_chain_workspace(n, bits, &cwb), "downsample_chain_launch");
  auto cws = workspace(cwb, dev);
  uint32_t *c = reinterpret_cast<uint32_t *>(cnt.data_ptr<int32_t>());
  check_rc(spira_hip_downsample_chain(keys.data_ptr(), n, bits, static_cast<int>(B), st.data(), ptrs.data(), c, c + B,
                                      cws.data_ptr(), cwb, current_stream()),
           "downsample_chain_launch");
  outs.push_back(cnt);
  return outs;
}

// One downsample per target stride: every plan on the current stream, one
// host read of all plans, then each execution on its own pool stream, and
// one host read of all counts at the end (reference:
// CUDAStreamedOutputGenerate, :107-200).
std::vector<torch::Tensor> streamed_output_generate(const torch::Tensor &keys, const std::vector<Int3> &strides) {
  SPIRA_CHECK_ARG(keys.dim() == 1, "coordinates should be already flattened");
  require_device(keys, "keys");
  const int bits = key_bits_of(keys);
  const auto dev = keys.device();
  const int64_t n = keys.size(0);
  const size_t B = strides.size();
  // Nested power-of-two strides (2, 4, 8, 16 ...): every level from the
  // previous one, no host read until the counts (spira_hip_downsample_chain);
  // keys that turn out unsorted fall through to the per-stride path below.
  if (auto launched = downsample_chain_launch(keys, strides); !launched.empty()) {
    auto cnt = launched.back();
    auto h = cnt.cpu();
    const int32_t *hc = h.data_ptr<int32_t>();
    if (hc[B] == 0) {
      std::vector<torch::Tensor> res;
      for (size_t i = 0; i < B; ++i) res.push_back(launched[i].slice(0, 0, hc[i]));
      return res;
    }
  }
  auto counts = torch::zeros({static_cast<int64_t>(std::max<size_t>(B, 1))},
                             torch::TensorOptions(dev).dtype(torch::kInt32));
  constexpr int64_t PB = sizeof(spira_hip_downsample_plan_t);
  auto plans = torch::empty({static_cast<int64_t>(std::max<size_t>(B, 1)) * PB},
                            torch::TensorOptions(dev).dtype(torch::kUInt8));
  // outputs and workspaces are allocated on the current stream before the
  // fan-out; the current stream waits for every side stream afterwards
  std::vector<torch::Tensor> outs, wss;
  size_t wsb = 0;
  check_rc(spira_hip_downsample_workspace(n, bits, &wsb), "downsample");
  for (size_t i = 0; i < B; ++i) {
    outs.push_back(torch::empty_like(keys));
    wss.push_back(workspace(wsb, dev));
  }
  std::vector<spira_hip_downsample_plan_t> hplans(B);
  if (n > 0 && B > 0) {
    for (size_t i = 0; i < B; ++i) {
      auto [sx, sy, sz] = strides[i];
      check_rc(spira_hip_downsample_plan(
                   keys.data_ptr(), n, bits, sx, sy, sz,
                   reinterpret_cast<spira_hip_downsample_plan_t *>(plans.data_ptr<uint8_t>() + i * PB),
                   wss[i].data_ptr(), wsb, current_stream()),
               "streamed_output_generate");
    }
    auto h = plans.cpu();
    std::memcpy(hplans.data(), h.data_ptr<uint8_t>(), B * PB);
  }
  {
    StreamFan fan(dev, B);
    for (size_t i = 0; i < B; ++i) {
      auto [sx, sy, sz] = strides[i];
      check_rc(spira_hip_downsample_execute(keys.data_ptr(), n, bits, sx, sy, sz, n > 0 ? &hplans[i] : nullptr,
                                            outs[i].data_ptr(),
                                            reinterpret_cast<uint32_t *>(counts.data_ptr<int32_t>() + i),
                                            wsb ? wss[i].data_ptr() : nullptr, wsb, fan[i]),
               "streamed_output_generate");
    }
    fan.join();
  }
  auto h = counts.cpu();
  std::vector<torch::Tensor> res;
  for (size_t i = 0; i < B; ++i) res.push_back(outs[i].slice(0, 0, h.data_ptr<int32_t>()[i]));
  return res;
}

// GPU voxelization (reference: sparse_quantize, datasets/helpers.py:14-30):
// points [N, 3] float32 / float64 on the device -> sorted unique voxel
// coordinates [M, 3] int32 (one host read of M).
torch::Tensor voxelize(const torch::Tensor &points, double vx, double vy, double vz) {
  require_device(points, "points");
  SPIRA_CHECK_ARG(points.dim() == 2 && points.size(1) == 3, "points must be [N, 3]");
  SPIRA_CHECK_ARG(points.scalar_type() == torch::kFloat || points.scalar_type() == torch::kDouble,
                  "points must be float32 or float64");
  auto p = points.contiguous();
  const int64_t n = p.size(0);
  auto coords = empty_i32({std::max<int64_t>(n, 1), 3}, p.device());
  auto count = torch::zeros({1}, torch::TensorOptions(p.device()).dtype(torch::kInt32));
  size_t wsb = 0;
  check_rc(spira_hip_voxelize_workspace(n, &wsb), "voxelize");
  auto ws = workspace(wsb, p.device());
  check_rc(spira_hip_voxelize(p.data_ptr(), n, p.scalar_type() == torch::kDouble ? 1 : 0, vx, vy, vz,
                              coords.data_ptr<int32_t>(), reinterpret_cast<uint32_t *>(count.data_ptr<int32_t>()),
                              wsb ? ws.data_ptr() : nullptr, wsb, current_stream()),
           "voxelize");
  const int64_t m = count.cpu().item<int32_t>();
  return coords.slice(0, 0, m);
}

void register_coords(pybind11::module_ &m) {
  m.def("voxelize", &voxelize);
  m.def("cuda_flatten_sort", &flatten_sort);
  m.def("cuda_unflatten", &unflatten);
  m.def("cuda_downsample", &downsample);
  m.def("cuda_streamed_output_generate", &streamed_output_generate);
  m.def("cuda_downsample_chain_launch", &downsample_chain_launch);
}

}  // namespace spira_host
