// Kernel-map entry points of `_C`: single map, network-wide streamed build,
// the no-z-scan ablation and the transposed OS map.
// Reference: torch/cuda_sparse_convolution_mapping.cu:211-1838.
#include "host_common.h"

#include <algorithm>
#include <cstdlib>

namespace spira_host {

std::vector<int32_t> indexes_l1(int kx, int ky, int kz, int dataflow, int *front) {
  // data[canonical k] = row; offsets with |dx|+|dy|+|dz| < (dataflow-1)/2
  // come first, both halves in canonical order.
  const int thr = (dataflow - 1) / 2;
  auto kmin = [](int k) { return (k % 2 == 1) ? -(k / 2) : -(k / 2) + 1; };
  int nf = 0;
  for (int x = kmin(kx); x < kmin(kx) + kx; ++x)
    for (int y = kmin(ky); y < kmin(ky) + ky; ++y)
      for (int z = kmin(kz); z < kmin(kz) + kz; ++z)
        if (std::abs(x) + std::abs(y) + std::abs(z) < thr) ++nf;
  std::vector<int32_t> data;
  int fp = 0, bp = nf;
  for (int x = kmin(kx); x < kmin(kx) + kx; ++x)
    for (int y = kmin(ky); y < kmin(ky) + ky; ++y)
      for (int z = kmin(kz); z < kmin(kz) + kz; ++z)
        data.push_back(std::abs(x) + std::abs(y) + std::abs(z) < thr ? fp++ : bp++);
  *front = nf;
  return data;
}

// A map whose device work is queued; pair lists (odd dataflows) still need
// the host-side pair count before their output can be allocated.
struct PendingMap {
  int64_t S = 0, T = 0, Tp = 0, ntiles = 0;
  int K = 0, dataflow = 0, dense = 0, R = 0, row0 = 0;
  bool half = false;
  torch::Tensor map, counts, tile_offsets, nbsizes, naddrs, qnaddrs, sizes, smask, tmask;
  // scratch of the pair/mask scan.  Held here (not freed when stage_map
  // returns) because the scan may run on a side stream: the caching
  // allocator would hand a freed block straight to the next map's scan on
  // another stream, and two decoupled look-back scans sharing one flag array
  // can wait on each other forever.
  torch::Tensor scan_ws;
};

static void check_keys(const torch::Tensor &src, const torch::Tensor &tgt) {
  SPIRA_CHECK_ARG(src.dim() == 1 && tgt.dim() == 1, "sources and targets must be flattened keys");
  require_device(src, "sources");
  require_device(tgt, "targets");
  SPIRA_CHECK_ARG(src.scalar_type() == tgt.scalar_type(), "sources and targets must have the same key dtype");
  key_bits_of(src);
}

// half: -1 = automatic (S == T and K odd), 0 = never, 1 = when K odd
// `job` (dataflow 0 only, may be null): the search is not launched but
// described there, for a caller that batches the searches of several maps.
static PendingMap stage_map(const torch::Tensor &src, const torch::Tensor &tgt, const Int3 &ksize,
                            const Int3 &sstride, int dataflow, int half, hipStream_t stream,
                            spira_hip_kmap_job_t *job = nullptr) {
  check_keys(src, tgt);
  SPIRA_CHECK_ARG(dataflow >= 0 && dataflow <= 8, "dataflow must be in [0, 8]");
  const auto dev = src.device();
  const int bits = key_bits_of(src);
  auto [kx, ky, kz] = ksize;
  auto [sx, sy, sz] = sstride;
  PendingMap pm;
  pm.S = src.size(0);
  pm.T = tgt.size(0);
  pm.Tp = round128(pm.T);
  pm.ntiles = pm.Tp / 64;
  pm.K = kx * ky * kz;
  pm.dataflow = dataflow;
  const int K = pm.K;

  if (dataflow == 0) {
    pm.map = empty_i32({pm.Tp, K}, dev);
    if (job) {
      *job = spira_hip_kmap_job_t{src.data_ptr(), pm.S, tgt.data_ptr(), pm.T, kx, ky, kz, sx, sy, sz,
                                  pm.map.data_ptr<int32_t>()};
      return pm;
    }
    check_rc(spira_hip_kmap_search(src.data_ptr(), pm.S, tgt.data_ptr(), pm.T, bits, kx, ky, kz, sx, sy, sz,
                                   SPIRA_KMAP_OS, nullptr, pm.map.data_ptr<int32_t>(), nullptr, stream),
             "binary_search");
    return pm;
  }

  std::vector<int32_t> perm;
  int layout = SPIRA_KMAP_WS;
  if (dataflow <= 2) {
    pm.half = (half < 0) ? (pm.S == pm.T && K % 2 == 1) : (half == 1 && K % 2 == 1);
    pm.row0 = 0;
    pm.R = pm.half ? (K + 1) / 2 : K;
  } else {
    SPIRA_CHECK_ARG(kz == 3 || kz == 5, "Currently hybrid dataflows support kernel size 3 or 5 along z");
    int front = 0;
    perm = indexes_l1(kx, ky, kz, dataflow, &front);
    pm.dense = perm[0];  // first offset (a corner) is always in the back part
    pm.half = true;
    pm.row0 = pm.dense;
    pm.R = (K - pm.dense) / 2;
    layout = SPIRA_KMAP_HYBRID;
  }
  pm.map = empty_i32({K, pm.Tp}, dev);
  pm.counts = empty_i32({K, pm.ntiles}, dev);
  check_rc(spira_hip_kmap_search(src.data_ptr(), pm.S, tgt.data_ptr(), pm.T, bits, kx, ky, kz, sx, sy, sz, layout,
                                 perm.empty() ? nullptr : perm.data(), pm.map.data_ptr<int32_t>(),
                                 pm.counts.data_ptr<int32_t>(), stream),
           "binary_search");

  const int64_t ncounts = static_cast<int64_t>(pm.R) * pm.ntiles;
  pm.tile_offsets = empty_i32({std::max<int64_t>(ncounts, 1)}, dev);
  pm.nbsizes = empty_i32({pm.R}, dev);
  const bool pairs = dataflow % 2 == 1;
  if (pairs) {
    pm.naddrs = empty_i32({pm.R + 1}, dev);
    pm.qnaddrs = empty_i32({pm.R + 1}, dev);
    pm.sizes = empty_i32({2}, dev);
  }
  size_t ws_bytes = 0;
  check_rc(spira_hip_kmap_scan_workspace(ncounts, &ws_bytes), "binary_search");
  pm.scan_ws = workspace(ws_bytes, dev);
  auto &ws = pm.scan_ws;
  check_rc(spira_hip_kmap_scan(pm.counts.data_ptr<int32_t>() + static_cast<int64_t>(pm.row0) * pm.ntiles, pm.R,
                               pm.ntiles, 128, pm.tile_offsets.data_ptr<int32_t>(), pm.nbsizes.data_ptr<int32_t>(),
                               pairs ? pm.naddrs.data_ptr<int32_t>() : nullptr,
                               pairs ? pm.qnaddrs.data_ptr<int32_t>() : nullptr,
                               pairs ? pm.sizes.data_ptr<int32_t>() : nullptr, ws.data_ptr(), ws_bytes, stream),
           "binary_search");
  if (!pairs) {
    const int Km = (dataflow <= 2) ? K : K - pm.dense;
    pm.smask = empty_i32({Km, pm.S}, dev);
    pm.tmask = empty_i32({Km, pm.T}, dev);
    check_rc(spira_hip_kmap_emit_masks(pm.map.data_ptr<int32_t>(), pm.S, pm.T, pm.Tp, pm.row0, pm.R, Km,
                                       pm.half ? 1 : 0, pm.tile_offsets.data_ptr<int32_t>(),
                                       pm.smask.data_ptr<int32_t>(), pm.tmask.data_ptr<int32_t>(), stream),
             "binary_search");
  }
  return pm;
}

static KmapTuple finish_map(PendingMap &pm, int32_t P, int32_t QP, hipStream_t stream) {
  const auto dev = pm.map.device();
  torch::Tensor first = pm.map;
  if (pm.dataflow > 4) first = pm.map.narrow(0, 0, pm.dense).t().contiguous();
  if (pm.dataflow == 0) return KmapTuple(pm.S, pm.T, pm.map, {}, {}, {}, {}, {}, {});
  if (pm.dataflow % 2 == 0)
    return KmapTuple(pm.S, pm.T, first, pm.smask, pm.tmask, pm.nbsizes, {}, {}, {});
  auto nbmaps = empty_i32({2, P}, dev);
  if (P > 0)
    check_rc(spira_hip_kmap_emit_pairs(pm.map.data_ptr<int32_t>(), pm.Tp, pm.row0, pm.R,
                                       pm.tile_offsets.data_ptr<int32_t>(), nbmaps.data_ptr<int32_t>(),
                                       nbmaps.data_ptr<int32_t>() + P, stream),
             "binary_search");
  return KmapTuple(pm.S, pm.T, first, nbmaps, pm.nbsizes, pm.naddrs, pm.qnaddrs, P, QP);
}

// (reference: CUDABinarySearch / BinarySearch<CT>, mapping.cu:211-892, 1728-1752)
KmapTuple binary_search(const torch::Tensor &sources, const torch::Tensor &targets, const Int3 &kernel_size,
                        const Int3 &source_stride, int dataflow) {
  auto stream = current_stream();
  auto pm = stage_map(sources, targets, kernel_size, source_stride, dataflow, -1, stream);
  int32_t P = 0, QP = 0;
  if (dataflow % 2 == 1) {
    auto h = pm.sizes.cpu();
    P = h.data_ptr<int32_t>()[0];
    QP = h.data_ptr<int32_t>()[1];
  }
  return finish_map(pm, P, QP, stream);
}

// Output-stationary maps on one pool stream each instead of back to back on
// the current stream.  Off by default: measured on MI355X, the fan-out's
// host work (an event record and wait per stream) costs more than the
// overlap returns -- config-4 step 2.92 ms concurrent vs 2.85 ms serial,
// config 5 (seven 125-offset maps) 4.75 vs 4.71 ms.
static bool &concurrent_maps() {
  static bool on = false;
  return on;
}
void set_concurrent_maps(bool on) { concurrent_maps() = on; }

// Network-wide build: map i reads sources voxels[i/2] and targets
// voxels[(i+1)/2] (the layer list alternates submanifold / downsampling
// maps); every map runs on its own pool stream and the pair counts of all
// maps are read back with a single synchronisation.
// (reference: CUDABinarySearchStreamed / BinarySearchStreamed<CT>, mapping.cu:894-1645, 1757-1779)
std::vector<KmapTuple> binary_search_streamed(const std::vector<torch::Tensor> &voxels,
                                              const std::vector<Int3> &kernel_sizes,
                                              const std::vector<Int3> &source_strides,
                                              const std::vector<int> &dataflow, int64_t begin) {
  const size_t n = kernel_sizes.size();
  SPIRA_CHECK_ARG(begin >= 0 && static_cast<size_t>(begin) <= n, "begin out of range");
  const size_t b0 = static_cast<size_t>(begin);
  SPIRA_CHECK_ARG(source_strides.size() == n && dataflow.size() == n,
                  "All argument lists must have the same length in build_kmap_streamed");
  SPIRA_CHECK_ARG(!voxels.empty(), "voxels must not be empty");
  for (size_t i = b0; i < n; ++i)
    SPIRA_CHECK_ARG((i + 1) / 2 < voxels.size(), "not enough voxel sets for ", n, " maps");
  const auto dev = voxels[0].device();
  std::vector<PendingMap> pending(n);
  auto sizes_host = torch::empty({static_cast<int64_t>(std::max<size_t>(2 * n, 2))},
                                 torch::TensorOptions().dtype(torch::kInt32).pinned_memory(true));
  std::vector<KmapTuple> out;
  // Every map on a pool stream of its own (concurrent_maps()), so that the
  // searches of all layers run concurrently; by default output-stationary maps
  // (one search kernel each) go back to back on the current stream and the
  // other dataflows (several kernels and a size read-back per map) on pool
  // streams.  The current stream waits for all of them.
  std::vector<size_t> side_of(n, 0);
  size_t nside = 0;
  for (size_t i = b0; i < n; ++i)
    if (concurrent_maps() || dataflow[i] != 0) side_of[i] = nside++;
  StreamFan fan(dev, nside);
  const hipStream_t cur = current_stream();
  auto stream_of = [&](size_t i) {
    return (concurrent_maps() || dataflow[i] != 0) ? fan[side_of[i]] : cur;
  };
  // output-stationary maps on the current stream: their searches are
  // batched into one launch per kernel shape, after every map is allocated
  std::vector<spira_hip_kmap_job_t> jobs;
  for (size_t i = b0; i < n; ++i) {
    // half maps: dataflow 2 uses the position in the list (mapping.cu:1129),
    // the other dataflows compare the set sizes (mapping.cu:955)
    const int half = (dataflow[i] == 2) ? (i % 2 == 0 ? 1 : 0) : -1;
    const bool batched = dataflow[i] == 0 && !concurrent_maps();
    spira_hip_kmap_job_t job{};
    pending[i] = stage_map(voxels[i / 2], voxels[(i + 1) / 2], kernel_sizes[i], source_strides[i], dataflow[i],
                           half, stream_of(i), batched ? &job : nullptr);
    if (batched) jobs.push_back(job);
    if (dataflow[i] % 2 == 1) {
      SPIRA_CHECK_ARG(hipMemcpyAsync(sizes_host.data_ptr<int32_t>() + 2 * i, pending[i].sizes.data_ptr<int32_t>(),
                                     2 * sizeof(int32_t), hipMemcpyDeviceToHost, stream_of(i)) == hipSuccess,
                      "size read-back failed");
    }
  }
  if (!jobs.empty())
    check_rc(spira_hip_kmap_search_batch(static_cast<int>(jobs.size()), jobs.data(), key_bits_of(voxels[0]), cur),
             "binary_search_streamed");
  // Odd dataflows need their pair counts on the host; hybrid dataflows above
  // 4 transpose their dense part on the current stream in finish_map, so the
  // side stream that wrote the map must be complete first.
  for (size_t i = b0; i < n; ++i)
    if (dataflow[i] % 2 == 1 || dataflow[i] > 4)
      SPIRA_CHECK_ARG(hipStreamSynchronize(stream_of(i)) == hipSuccess, "stream synchronisation failed");
  for (size_t i = b0; i < n; ++i) {
    const int32_t *h = sizes_host.data_ptr<int32_t>() + 2 * i;
    out.push_back(finish_map(pending[i], dataflow[i] % 2 == 1 ? h[0] : 0, dataflow[i] % 2 == 1 ? h[1] : 0,
                             stream_of(i)));
  }
  fan.join();
  return out;
}

// (reference: CUDABinarySearchNoSmallZ, mapping.cu:1647-1690, 1784-1806)
KmapTuple binary_search_no_small_z(const torch::Tensor &sources, const torch::Tensor &targets,
                                   const Int3 &kernel_size, const Int3 &source_stride) {
  check_keys(sources, targets);
  auto [kx, ky, kz] = kernel_size;
  auto [sx, sy, sz] = source_stride;
  const int64_t S = sources.size(0), T = targets.size(0), Tp = round128(T);
  auto map = empty_i32({Tp, kx * ky * kz}, sources.device());
  check_rc(spira_hip_kmap_search(sources.data_ptr(), S, targets.data_ptr(), T, key_bits_of(sources), kx, ky, kz,
                                 sx, sy, sz, SPIRA_KMAP_NOZ, nullptr, map.data_ptr<int32_t>(), nullptr,
                                 current_stream()),
           "binary_search_no_small_z");
  return KmapTuple(S, T, map, {}, {}, {}, {}, {}, {});
}

// (reference: CUDAConvertTransposedOs, mapping.cu:1809-1830)
// partition: the map's entries partition the sources (a down-sampling map
// whose kernel is its stride), which one pass inverts
torch::Tensor convert_transposed_os(const torch::Tensor &out_in_map, int64_t num_sources, bool partition) {
  SPIRA_CHECK_ARG(out_in_map.dim() == 2 && out_in_map.scalar_type() == torch::kInt32,
                  "out_in_map must be a 2-D int32 tensor");
  require_device(out_in_map, "out_in_map");
  const int64_t Sp = round128(num_sources);
  auto out = empty_i32({Sp, out_in_map.size(1)}, out_in_map.device());
  if (partition)
    check_rc(spira_hip_convert_transposed_os_partition(out_in_map.data_ptr<int32_t>(), out_in_map.size(0),
                                                       static_cast<int>(out_in_map.size(1)), num_sources, Sp,
                                                       out.data_ptr<int32_t>(), current_stream()),
             "convert_transposed_os");
  else
    check_rc(spira_hip_convert_transposed_os(out_in_map.data_ptr<int32_t>(), out_in_map.size(0),
                                             static_cast<int>(out_in_map.size(1)), Sp, out.data_ptr<int32_t>(),
                                             current_stream()),
             "convert_transposed_os");
  return out;
}

// Kernel-only timing of the map search (output-stationary layout): `reps`
// back-to-back launches into one preallocated map between two HIP events;
// returns ms per launch.  No reference counterpart: a measurement probe for
// the roofline report (the reference times build_kmap from Python,
// scripts/mapping_experiment.py:81-101).
float time_kmap_search(const torch::Tensor &sources, const torch::Tensor &targets, const Int3 &kernel_size,
                       const Int3 &source_stride, int64_t reps) {
  check_keys(sources, targets);
  SPIRA_CHECK_ARG(reps >= 1, "reps must be positive");
  auto [kx, ky, kz] = kernel_size;
  auto [sx, sy, sz] = source_stride;
  const int64_t S = sources.size(0), T = targets.size(0), Tp = round128(T);
  auto map = empty_i32({std::max<int64_t>(Tp, 1), kx * ky * kz}, sources.device());
  auto s = current_stream();
  auto launch = [&] {
    check_rc(spira_hip_kmap_search(sources.data_ptr(), S, targets.data_ptr(), T, key_bits_of(sources), kx, ky, kz,
                                   sx, sy, sz, SPIRA_KMAP_OS, nullptr, map.data_ptr<int32_t>(), nullptr, s),
             "time_kmap_search");
  };
  launch();
  hipEvent_t a, b;
  SPIRA_CHECK_ARG(hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess, "event creation failed");
  SPIRA_CHECK_ARG(hipEventRecord(a, s) == hipSuccess, "event record failed");
  for (int64_t i = 0; i < reps; ++i) launch();
  SPIRA_CHECK_ARG(hipEventRecord(b, s) == hipSuccess, "event record failed");
  SPIRA_CHECK_ARG(hipEventSynchronize(b) == hipSuccess, "event synchronisation failed");
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return ms / static_cast<float>(reps);
}

void register_mapping(pybind11::module_ &m) {
  m.def("time_kmap_search", &time_kmap_search);
  m.def("set_concurrent_maps", &set_concurrent_maps);
  m.def("cuda_binary_search", &binary_search);
  m.def("cuda_binary_search_streamed", &binary_search_streamed, pybind11::arg("voxels"), pybind11::arg("kernel_sizes"),
        pybind11::arg("source_strides"), pybind11::arg("dataflow"), pybind11::arg("begin") = 0);
  m.def("cuda_binary_search_no_small_z", &binary_search_no_small_z);
  m.def("cuda_convert_transposed_os", &convert_transposed_os, pybind11::arg("out_in_map"), pybind11::arg("num_sources"),
        pybind11::arg("partition") = false);
}

}  // namespace spira_host
